"""GPU parity: HCA write path (compress + append + window ring + state ring)
and the HCA decode index rows, bit-exact against the oracle."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, bf16_values, randn_bf16, to_dev
from oracle import hca as oh
from oracle import indexer as oi
from oracle import paged

pytestmark = pytest.mark.gpu


class HcaCase:
    def __init__(self, rng, dim, num_seqs, max_pos, ring, rope="plain", bf16=False):
        self.dim, self.B, self.ring = dim, num_seqs, ring
        lp = (max_pos + 63) // 64
        spans = max_pos // 128 + 1
        cp = (spans + 63) // 64
        rp = ring // 64
        perm = rng.permutation(num_seqs * (lp + cp + rp)).astype(np.int32)
        self.bt = perm[: num_seqs * lp].reshape(num_seqs, lp)
        self.comp_bt = perm[num_seqs * lp : num_seqs * (lp + cp)].reshape(num_seqs, cp)
        self.ring_pages = perm[num_seqs * (lp + cp) :].reshape(num_seqs, rp)
        self.pages = len(perm)
        self.ape = (rng.standard_normal((128, dim)) * 0.5).astype(np.float32)
        self.norm_w = (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
        # the compressor's RoPE table at position 128 j (compress_rope_theta);
        # "yarn": YaRN frequencies and attention factor, as the HCA config uses
        table = oi.yarn_cos_sin if rope == "yarn" else oi.rope_cos_sin
        self.cos_sin = table(np.arange(spans) * 128, 64, 1.6e5)
        self.state_slot = rng.permutation(num_seqs + 2)[:num_seqs].astype(np.int32)
        self.st = oh.HcaState(self.pages, dim, num_seqs + 2, bf16=bf16)


def _run_call(dev, case, rng, starts, counts, gpu, fused=False):
    D = case.dim
    positions, token_seq, qsl = [], [], [0]
    for b, (p0, n) in enumerate(zip(starts, counts)):
        positions += list(range(p0, p0 + n))
        token_seq += [b] * n
        qsl.append(qsl[-1] + n)
    positions = np.array(positions, np.int64)
    token_seq = np.array(token_seq, np.int32)
    qsl = np.array(qsl, np.int32)
    T = len(positions)
    latent = randn_bf16(rng, (T, D))
    kv_score = randn_bf16(rng, (T, 2 * D))
    slots = paged.slots_from_block_table(case.bt, token_seq, positions)
    oh.hca_write(case.st, latent, kv_score, positions, token_seq, qsl, slots, case.ring_pages, case.ring,
                 case.comp_bt, case.state_slot, case.ape, case.norm_w, 1e-6, case.cos_sin)
    from ernie_kv import ops

    d = lambda a: to_dev(a, dev)  # noqa: E731
    kvs_t = bf16_tensor(kv_score, dev)
    if fused:
        if fused == "ws" and "ws" not in gpu:  # decode-sized calls split each span over dim / 64 workgroups
            gpu["ws"] = ops.hca_write_workspace(case.B, D, dev)
        if fused == "ws-spans" and "ws" not in gpu:  # and prefill calls over D / 64 one-wave workgroups
            gpu["ws"] = ops.hca_write_workspace(case.B, D, dev, max_query_len=1000)
        ops.hca_write(bf16_tensor(latent, dev), kvs_t, d(slots), d(positions), d(token_seq), d(qsl), int(max(counts)),
                      gpu["state"], d(case.state_slot), d(case.ape), d(case.norm_w), 1e-6, d(case.cos_sin),
                      d(case.comp_bt), d(case.ring_pages), case.ring, gpu["pool"], workspace=gpu.get("ws"))
        return
    ops.hca_compress(kvs_t, d(positions), d(qsl), int(max(counts)), gpu["state"], d(case.state_slot),
                     d(case.ape), d(case.norm_w), 1e-6, d(case.cos_sin), d(case.comp_bt), gpu["pool"])
    ops.hca_append(bf16_tensor(latent, dev), kvs_t, d(slots), d(positions), d(token_seq), d(qsl), gpu["pool"],
                   d(case.ring_pages), case.ring, gpu["state"], d(case.state_slot))


def _counters_zero(ws) -> bool:
    """The workspace's arrival counters (one u32 per span slot it holds, at
    its start) are all zero."""
    record = 4 + (576 + 144) * 4
    return int(ws[: 4 * (ws.numel() // record)].sum()) == 0


@pytest.mark.parametrize("rope", ["plain", "yarn"])
@pytest.mark.parametrize("fused", [False, True, "ws", "ws-spans"],
                         ids=["compress+append", "hca_write", "hca_write+ws", "hca_write+ws-spans"])
@pytest.mark.parametrize("dim", [576, 512])
def test_hca_write_path_exact(dev, dim, fused, rope):
    rng = np.random.default_rng(dim)
    case = HcaCase(rng, dim, num_seqs=3, max_pos=1400, ring=192, rope=rope)
    gpu = {
        "pool": torch.zeros((case.pages, paged.fp8_page_bytes(dim)), dtype=torch.uint8, device=dev),
        "state": torch.zeros((case.B + 2, 256, 2 * dim), dtype=torch.bfloat16, device=dev),
    }
    # chunked prefill, partial spans carried in the state ring, then MTP-style
    # 3-token steps, a rollback re-append, a long chunk, and a prefill call in
    # which one sequence has no rows.
    calls = [
        ([0, 0, 0], [300, 100, 128]),
        ([300, 100, 128], [3, 200, 2]),
        ([303, 300, 130], [3, 3, 3]),
        ([304, 301, 131], [3, 3, 3]),  # rollback: re-append from one position back
        ([307, 304, 134], [900, 1, 700]),
        ([1207, 305, 834], [0, 260, 130]),  # spans 2 and 3 of sequence 1, span 6 of sequence 2 (from the ring)
    ]
    for starts, counts in calls:
        _run_call(dev, case, rng, starts, counts, gpu, fused)
        torch.cuda.synchronize()
        assert np.array_equal(gpu["pool"].cpu().numpy(), case.st.pool), f"pool mismatch after call {starts}"
        got_state = bf16_values(gpu["state"]).reshape(case.st.state.shape)
        assert np.array_equal(got_state, case.st.state), f"state mismatch after call {starts}"
        if "ws" in gpu:  # the arrival counters are left zero
            assert _counters_zero(gpu["ws"])


@pytest.mark.parametrize("fused", [True, "ws", "ws-spans"], ids=["hca_write", "hca_write+ws", "hca_write+ws-spans"])
@pytest.mark.parametrize("dim", [576, 512])
def test_hca_write_path_exact_bf16(dev, dim, fused):
    """The bf16 pool (ekv_hca_write_bf16: rows stored as given, compressed
    rows rounded to bf16) over the same call sequence as the fp8 test:
    chunked prefill, 3-token steps, a rollback re-append, long chunks."""
    rng = np.random.default_rng(dim + 7)
    case = HcaCase(rng, dim, num_seqs=3, max_pos=1400, ring=192, rope="yarn", bf16=True)
    gpu = {
        "pool": torch.zeros((case.pages * 64, dim), dtype=torch.bfloat16, device=dev),
        "state": torch.zeros((case.B + 2, 256, 2 * dim), dtype=torch.bfloat16, device=dev),
    }
    calls = [
        ([0, 0, 0], [300, 100, 128]),
        ([300, 100, 128], [3, 200, 2]),
        ([303, 300, 130], [3, 3, 3]),
        ([304, 301, 131], [3, 3, 3]),
        ([307, 304, 134], [900, 1, 700]),
        ([1207, 305, 834], [0, 260, 130]),
    ]
    for starts, counts in calls:
        _run_call(dev, case, rng, starts, counts, gpu, fused)
        torch.cuda.synchronize()
        got = gpu["pool"].view(torch.uint8).reshape(case.pages, -1).cpu().numpy()
        assert np.array_equal(got, case.st.pool), f"pool mismatch after call {starts}"
        got_state = bf16_values(gpu["state"]).reshape(case.st.state.shape)
        assert np.array_equal(got_state, case.st.state), f"state mismatch after call {starts}"
        if "ws" in gpu:
            assert _counters_zero(gpu["ws"])


@pytest.mark.parametrize("rope", ["plain", "yarn"])
@pytest.mark.parametrize("fused", [False, True, "ws"], ids=["compress+append", "hca_write", "hca_write+ws"])
@pytest.mark.parametrize("dim", [576, 512])
def test_hca_write_decode_completes_spans(dev, dim, fused, rope):
    """Calls of fewer than 128 rows per sequence (decode, drafts) that complete
    spans whose first rows sit in the state ring (the compressor's straddle
    path).  Spans start 125, 126, 127 and 1 rows before the call."""
    rng = np.random.default_rng(40 + dim)
    case = HcaCase(rng, dim, num_seqs=3, max_pos=600, ring=192, rope=rope)
    gpu = {
        "pool": torch.zeros((case.pages, paged.fp8_page_bytes(dim)), dtype=torch.uint8, device=dev),
        "state": torch.zeros((case.B + 2, 256, 2 * dim), dtype=torch.bfloat16, device=dev),
    }
    calls = [
        ([0, 0, 0], [125, 255, 126]),     # prefill, partial spans left in the state ring
        ([125, 255, 126], [3, 1, 3]),     # completes span 0, span 1 (one row), span 0 (two rows)
        ([128, 256, 129], [127, 127, 127]),  # span 1 of sequence 2: one ring row, 127 new
        ([255, 383, 256], [1, 1, 3]),     # span 1 and span 2 by their last row
    ]
    for starts, counts in calls:
        _run_call(dev, case, rng, starts, counts, gpu, fused)
        torch.cuda.synchronize()
        assert np.array_equal(gpu["pool"].cpu().numpy(), case.st.pool), f"pool mismatch after call {starts}"
        got_state = bf16_values(gpu["state"]).reshape(case.st.state.shape)
        assert np.array_equal(got_state, case.st.state), f"state mismatch after call {starts}"
        if "ws" in gpu:  # the arrival counters are left zero
            assert _counters_zero(gpu["ws"])


def test_hca_decode_indices(dev):
    from ernie_kv import ops

    rng = np.random.default_rng(4)
    case = HcaCase(rng, 576, num_seqs=4, max_pos=9000, ring=192)
    positions = np.array([0, 126, 127, 128, 5000, 8999], np.int64)
    req = np.array([0, 1, 2, 3, 1, 2], np.int32)
    width = 9000 // 128 + 128
    out = torch.full((6, width), -9, dtype=torch.int32, device=dev)
    lens = torch.zeros(6, dtype=torch.int32, device=dev)
    ops.hca_decode_indices(to_dev(positions, dev), to_dev(req, dev), to_dev(case.comp_bt, dev),
                           to_dev(case.ring_pages, dev), case.ring, out, lens)
    ref, rl = oh.hca_decode_indices(positions, req, case.comp_bt, case.ring_pages, case.ring, width)
    assert np.array_equal(out.cpu().numpy(), ref)
    assert np.array_equal(lens.cpu().numpy(), rl)


@pytest.mark.parametrize("dim", [576, 512])
def test_hca_decode_end_to_end(dev, dim):
    """Config-2 shape, scaled down: sequences of random context length are
    prefilled through ekv_hca_write (latent rows, compressed spans, window
    ring), then one decode token per sequence attends over its compressed
    entries and window ring: the index rows (ekv_hca_decode_indices) match
    the oracle exactly and the decode output is within the bf16 tolerance
    (|out - ref| <= 2e-3 + 2e-2 |ref|) of the fp64 oracle."""
    from ernie_kv import ops
    from oracle import decode as od

    rng = np.random.default_rng(50 + dim)
    B, H, ring = 5, 64, 192
    ctx = rng.integers(300, 2600, B)
    ctx[0] = 128  # exactly one compressed entry and a full window
    case = HcaCase(rng, dim, num_seqs=B, max_pos=int(ctx.max()) + 8, ring=ring)
    gpu = {
        "pool": torch.zeros((case.pages, paged.fp8_page_bytes(dim)), dtype=torch.uint8, device=dev),
        "state": torch.zeros((case.B + 2, 256, 2 * dim), dtype=torch.bfloat16, device=dev),
    }
    _run_call(dev, case, rng, [0] * B, ctx.tolist(), gpu, True)
    torch.cuda.synchronize()
    assert np.array_equal(gpu["pool"].cpu().numpy(), case.st.pool)

    positions = (ctx - 1).astype(np.int64)
    req = np.arange(B, dtype=np.int32)
    width = int(ctx.max()) // 128 + 128
    idx = torch.full((B, width), -9, dtype=torch.int32, device=dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    ops.hca_decode_indices(to_dev(positions, dev), to_dev(req, dev), to_dev(case.comp_bt, dev),
                           to_dev(case.ring_pages, dev), ring, idx, lens)
    ref_idx, ref_len = oh.hca_decode_indices(positions, req, case.comp_bt, case.ring_pages, ring, width)
    assert np.array_equal(idx.cpu().numpy(), ref_idx) and np.array_equal(lens.cpu().numpy(), ref_len)

    q = randn_bf16(rng, (B, H, dim))
    sinks = rng.standard_normal(H).astype(np.float32)
    scale = 256 ** -0.5
    out = torch.empty((B, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, H), dtype=torch.float32, device=dev)
    ops.sparse_mla_decode(bf16_tensor(q, dev), gpu["pool"], idx, scale, out, lse, sinks=to_dev(sinks, dev),
                          lengths=lens)
    ref_o, ref_l = od.sparse_mla_decode(q, lambda sl: od.gather_rows_fp8(case.st.pool, sl, dim), ref_idx, scale,
                                        512, sinks)
    got = bf16_values(out).astype(np.float64)
    err = np.abs(got - ref_o)
    assert np.all(err <= 2e-3 + 2e-2 * np.abs(ref_o)), f"max err {err.max()}"
    gl = lse.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(gl - ref_l) <= 2e-3 * np.maximum(1.0, np.abs(ref_l)))


def test_hca_decode_step_graph_replay(dev):
    """The HCA decode step -- ekv_hca_write of one new token per sequence
    (two of them complete a span), ekv_hca_decode_indices and
    ekv_sparse_mla_decode -- captured in a HIP graph: nothing inside
    synchronizes with the host or allocates, and each of three replays, with
    eager work and synchronizations between them, equals the eager step bit
    for bit (the step is idempotent: it rewrites the same slots)."""
    from ernie_kv import ops

    g = torch.Generator(device=dev).manual_seed(91)
    B, D, ring, H = 8, 576, 128, 64
    ctx = torch.tensor([300, 1024, 777, 2048, 1500, 129, 640, 2999], dtype=torch.int64)  # 1024, 2048: span ends
    spans = int(ctx.max()) // 128 + 1
    comp_pp, ring_pp = (spans + 63) // 64, ring // 64
    pages = B * (comp_pp + ring_pp + 1)
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(5)).to(torch.int32)
    comp_bt = perm[: B * comp_pp].view(B, comp_pp).to(dev)
    ring_pages = perm[B * comp_pp: B * (comp_pp + ring_pp)].view(B, ring_pp).to(dev)
    lat_page = perm[B * (comp_pp + ring_pp):].to(torch.int64)
    pos = ctx - 1
    codes = torch.randint(0, 256, (pages, 64 * D), device=dev, dtype=torch.uint8, generator=g)
    codes -= ((codes & 0x7F) == 0x7F).to(torch.uint8)
    scales = torch.full((pages, 64), 2.0 ** -8, device=dev, dtype=torch.float32)
    pool = torch.cat([codes, scales.view(torch.uint8)], dim=1).contiguous()
    ang = (torch.arange(spans, dtype=torch.float64)[:, None] * 128.0) * (
        1.6e5 ** (-torch.arange(32, dtype=torch.float64) * 2.0 / 64))[None, :]
    rnd = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)  # noqa: E731
    st = dict(latent=rnd(B, D), kv_score=rnd(B, 2 * D), state=rnd(B, 256, 2 * D), q=rnd(B, H, D),
              slots=(lat_page * 64 + pos % 64).to(dev), positions=pos.to(dev),
              token_seq=torch.arange(B, dtype=torch.int32, device=dev),
              qsl=torch.arange(B + 1, dtype=torch.int32, device=dev),
              state_slot=torch.arange(B, dtype=torch.int32, device=dev),
              ape=(0.5 * torch.randn(128, D, device=dev, generator=g)).contiguous(),
              norm_w=(1.0 + 0.1 * torch.randn(D, device=dev, generator=g)).contiguous(),
              cos_sin=torch.cat([torch.cos(ang), torch.sin(ang)], 1).to(torch.float32).to(dev),
              sinks=torch.randn(H, device=dev, generator=g))
    width = spans + ring
    idx = torch.empty((B, width), dtype=torch.int32, device=dev)
    lens = torch.empty(B, dtype=torch.int32, device=dev)
    out = torch.empty((B, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, H), dtype=torch.float32, device=dev)
    ws = ops.decode_workspace(B, H, width, dev)
    write_ws = ops.hca_write_workspace(B, D, dev)

    def step():
        ops.hca_write(st["latent"], st["kv_score"], st["slots"], st["positions"], st["token_seq"], st["qsl"], 1,
                      st["state"], st["state_slot"], st["ape"], st["norm_w"], 1e-6, st["cos_sin"], comp_bt,
                      ring_pages, ring, pool, workspace=write_ws)
        ops.hca_decode_indices(st["positions"], st["token_seq"], comp_bt, ring_pages, ring, idx, lens)
        ops.sparse_mla_decode(st["q"], pool, idx, 256 ** -0.5, out, lse, sinks=st["sinks"], lengths=lens,
                              workspace=ws)

    step()
    torch.cuda.synchronize()
    want = [x.clone() for x in (pool, st["state"], idx, lens, out, lse)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(0)
        lse.fill_(0)
        idx.fill_(-5)
        lens.fill_(0)
        _ = (st["q"][:, :, :64].float() @ st["q"][:, :, :64].float().transpose(1, 2).contiguous()).sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (pool, st["state"], idx, lens, out, lse)
        for name, a_, b_ in zip(["pool", "state", "idx", "lens", "out", "lse"], got, want):
            assert torch.equal(a_.view(torch.uint8) if a_.dtype == torch.bfloat16 else a_,
                               b_.view(torch.uint8) if b_.dtype == torch.bfloat16 else b_), f"replay {rep}: {name}"


def test_hca_write_graph_keeps_compression_the_capture_batch_skipped(dev):
    """A captured graph keeps the 128-span compression even when the batch it
    was captured with completes no span (the reference's
    test_compressor_skip_not_baked_into_cuda_graph,
    test_dsa_backend.py:92-127): ekv_hca_write_step is captured with
    positions that complete nothing, then replayed with positions of which two
    complete a span; the pool, state ring, index rows and lengths equal an
    eager call on the replay's inputs from the same starting state."""
    from ernie_kv import ops

    g = torch.Generator(device=dev).manual_seed(23)
    B, D, ring, window = 6, 576, 192, 128
    ctx_capture = torch.tensor([300, 1000, 777, 2000, 1500, 130], dtype=torch.int64)  # no span ends
    ctx_replay = torch.tensor([301, 1024, 778, 2048, 1501, 131], dtype=torch.int64)   # 1024, 2048 end spans
    spans = int(ctx_replay.max()) // 128 + 1
    comp_pp, ring_pp = (spans + 63) // 64, ring // 64
    lat_pp = (int(ctx_replay.max()) + 63) // 64
    pages = B * (comp_pp + ring_pp + lat_pp)
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(6)).to(torch.int32)
    comp_bt = perm[: B * comp_pp].view(B, comp_pp).to(dev)
    ring_pages = perm[B * comp_pp: B * (comp_pp + ring_pp)].view(B, ring_pp).to(dev)
    lat_bt = perm[B * (comp_pp + ring_pp):].view(B, lat_pp).to(torch.int64)
    rnd = lambda *s_: torch.randn(*s_, device=dev, generator=g).to(torch.bfloat16)  # noqa: E731
    ang = (torch.arange(spans, dtype=torch.float64)[:, None] * 128.0) * (
        1.6e5 ** (-torch.arange(32, dtype=torch.float64) * 2.0 / 64))[None, :]
    seq = torch.arange(B)

    def inputs(ctx):
        pos = ctx - 1
        return pos.to(dev), (lat_bt[seq, pos // 64] * 64 + pos % 64).to(dev)

    pos_c, slots_c = inputs(ctx_capture)
    pos_r, slots_r = inputs(ctx_replay)
    args = dict(latent=rnd(B, D), kv_score=rnd(B, 2 * D), slot_mapping=slots_c.clone(), positions=pos_c.clone(),
                token_seq=seq.to(torch.int32).to(dev), qsl=torch.arange(B + 1, dtype=torch.int32, device=dev),
                max_query_len=1, state_slot=torch.arange(B, dtype=torch.int32, device=dev),
                ape=(0.5 * torch.randn(128, D, device=dev, generator=g)).contiguous(),
                norm_w=(1.0 + 0.1 * torch.randn(D, device=dev, generator=g)).contiguous(), eps=1e-6,
                cos_sin=torch.cat([torch.cos(ang), torch.sin(ang)], 1).to(torch.float32).to(dev),
                comp_block_table=comp_bt, ring_pages=ring_pages, ring=ring)
    state0 = rnd(B, 256, 2 * D)
    pool0 = torch.randint(0, 126, (pages, paged.fp8_page_bytes(D)), device=dev, dtype=torch.uint8, generator=g)
    width = int(ctx_replay.max()) // 128 + window
    pool, state = pool0.clone(), state0.clone()
    idx = torch.full((B, width), -7, dtype=torch.int32, device=dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    ws = ops.hca_write_workspace(B, D, dev)

    def step():
        ops.hca_write_step(pool=pool, state=state, window=window, out=idx, lengths=lens, workspace=ws, **args)

    step()  # warm-up with the capture batch
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    def reset(pos, slots):
        pool.copy_(pool0)
        state.copy_(state0)
        idx.fill_(-7)
        lens.zero_()
        args["positions"].copy_(pos)
        args["slot_mapping"].copy_(slots)
        torch.cuda.synchronize()

    reset(pos_r, slots_r)
    step()  # eager on the replay's inputs
    torch.cuda.synchronize()
    want = [x.clone() for x in (pool, state, idx, lens)]
    assert not torch.equal(want[0], pool0), "the replay batch must write"
    for rep in range(2):
        reset(pos_r, slots_r)
        graph.replay()
        torch.cuda.synchronize()
        for name, a_, b_ in zip(["pool", "state", "idx", "lens"], (pool, state, idx, lens), want):
            assert torch.equal(a_.view(torch.uint8) if a_.dtype == torch.bfloat16 else a_,
                               b_.view(torch.uint8) if b_.dtype == torch.bfloat16 else b_), f"replay {rep}: {name}"
    # the two completed spans were written: their compressed slots differ from the starting pool
    for b_, j in ((1, 1023 // 128), (3, 2047 // 128)):
        page = int(comp_bt[b_, j // 64])
        off = (j % 64) * D
        assert not torch.equal(pool[page, off:off + D], pool0[page, off:off + D]), f"span {j} of sequence {b_}"


@pytest.mark.parametrize("rows", [1, 3, 130], ids=["decode", "drafts", "prefill-sized"])
@pytest.mark.parametrize("use_ws", [False, True], ids=["no-ws", "ws"])
def test_hca_write_step_matches_separate_calls(dev, rows, use_ws):
    """ekv_hca_write_step (the write and the step's index rows, one launch for
    decode-sized calls) leaves the same pool, state ring, index rows and
    lengths as ekv_hca_write followed by ekv_hca_decode_indices with the
    call's slots."""
    from ernie_kv import ops

    g = torch.Generator(device=dev).manual_seed(17 + rows)
    B, D, ring, window = 4, 576, 192, 128
    ctx = torch.tensor([300, 1024, 777, 2048], dtype=torch.int64)  # the call's last positions are ctx - 1
    spans = int(ctx.max()) // 128 + 2
    comp_pp, ring_pp = (spans + 63) // 64, ring // 64
    lat_pp = (int(ctx.max()) + 63) // 64
    pages = B * (comp_pp + ring_pp + lat_pp)
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    comp_bt = perm[: B * comp_pp].view(B, comp_pp).to(dev)
    ring_pages = perm[B * comp_pp: B * (comp_pp + ring_pp)].view(B, ring_pp).to(dev)
    lat_bt = perm[B * (comp_pp + ring_pp):].view(B, lat_pp).to(torch.int64)
    pos = torch.cat([torch.arange(int(c) - rows, int(c)) for c in ctx])
    seq = torch.arange(B).repeat_interleave(rows)
    slots = lat_bt[seq, pos // 64] * 64 + pos % 64
    T = B * rows
    rnd = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)  # noqa: E731
    ang = (torch.arange(spans, dtype=torch.float64)[:, None] * 128.0) * (
        1.6e5 ** (-torch.arange(32, dtype=torch.float64) * 2.0 / 64))[None, :]
    args = dict(latent=rnd(T, D), kv_score=rnd(T, 2 * D), slot_mapping=slots.to(dev), positions=pos.to(dev),
                token_seq=seq.to(torch.int32).to(dev),
                qsl=(torch.arange(B + 1, dtype=torch.int32) * rows).to(dev), max_query_len=rows,
                state_slot=torch.arange(B, dtype=torch.int32, device=dev),
                ape=(0.5 * torch.randn(128, D, device=dev, generator=g)).contiguous(),
                norm_w=(1.0 + 0.1 * torch.randn(D, device=dev, generator=g)).contiguous(), eps=1e-6,
                cos_sin=torch.cat([torch.cos(ang), torch.sin(ang)], 1).to(torch.float32).to(dev),
                comp_block_table=comp_bt, ring_pages=ring_pages, ring=ring)
    state0 = rnd(B, 256, 2 * D)
    pool0 = torch.randint(0, 256, (pages, paged.fp8_page_bytes(D)), device=dev, dtype=torch.uint8, generator=g)
    width = int(ctx.max()) // 128 + window
    outs = []
    for fused in (False, True):
        pool, state = pool0.clone(), state0.clone()
        idx = torch.full((T, width), -7, dtype=torch.int32, device=dev)
        lens = torch.zeros(T, dtype=torch.int32, device=dev)
        ws = ops.hca_write_workspace(B, D, dev, max_query_len=rows) if use_ws else None
        if fused:
            ops.hca_write_step(pool=pool, state=state, window=window, out=idx, lengths=lens, workspace=ws, **args)
        else:
            ops.hca_write(pool=pool, state=state, workspace=ws, **args)
            ops.hca_decode_indices(args["positions"], args["token_seq"], comp_bt, ring_pages, ring, idx, lens, window,
                                   query_start_loc=args["qsl"], slot_mapping=args["slot_mapping"])
        torch.cuda.synchronize()
        outs.append((pool, state.view(torch.int16), idx, lens))
        if ws is not None:
            assert _counters_zero(ws)
    for name, a_, b_ in zip(["pool", "state", "idx", "lens"], *outs):
        assert torch.equal(a_, b_), name
