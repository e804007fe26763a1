"""GPU parity for the DSA read path's indexer: merge, Hadamard, q quant,
exact scoring and exact top-k (all bit-exact against the oracle)."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, bf16_values, permuted_block_table, randn_bf16, to_dev
from oracle import indexer as oi
from oracle import paged
from oracle.fp8 import quantize_rows
from oracle.merge import merge_swa_topk as merge_ref

pytestmark = pytest.mark.gpu
WINDOW, TOPK = 128, 2048


def test_merge_swa_topk_known_answer(dev):
    """Transcription of test_dsa_backend.py:18-37 (exact)."""
    from ernie_kv import ops

    positions = torch.tensor([0, 5, 127, 128, 200, 2175, 2176, 5000], device=dev)
    num_tokens, width = positions.shape[0], TOPK + WINDOW
    g = torch.Generator().manual_seed(0)
    topk = torch.randint(0, 1 << 20, (num_tokens, TOPK), dtype=torch.int32, generator=g).to(dev)
    out = torch.full((num_tokens, width), -7, dtype=torch.int32, device=dev)
    ops.merge_swa_topk(topk, out, positions, WINDOW)
    for row, pos in enumerate(positions.tolist()):
        seq = pos + 1
        n, w = min(max(seq - WINDOW, 0), TOPK), min(seq, WINDOW)
        expected = torch.full((width,), -1, dtype=torch.int32)
        expected[:n] = topk[row, :n].cpu()
        expected[n : n + w] = torch.arange(seq - w, seq, dtype=torch.int32)
        torch.testing.assert_close(out[row].cpu(), expected, rtol=0, atol=0)
    ref = merge_ref(topk.cpu().numpy(), positions.cpu().numpy(), width, WINDOW)
    assert np.array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("T", [1, 3, 33])
def test_indexer_prep_exact(dev, T):
    """k_norm + NeoX rope + Hadamard of q and k (attention.py:955-969),
    bit-exact against the oracle; varied positions (one outside the table
    stays unrotated), row scales and a constant k row."""
    from ernie_kv import ops

    rng = np.random.default_rng(100 + T)
    q = randn_bf16(rng, (T, 64, 128), scale=2.0)
    k = (rng.standard_normal((T, 128)) * rng.uniform(0.05, 20, (T, 1)) + rng.uniform(-3, 3, (T, 1))).astype(np.float32)
    k[0] = 0.75  # constant row: normalizes to the bias
    k = bf16_values(bf16_tensor(k, "cpu"))
    w = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    b = (0.1 * rng.standard_normal(128)).astype(np.float32)
    table_rows = 70000
    pos = rng.integers(0, table_rows, T).astype(np.int64)
    pos[-1] = table_rows + 5 if T > 1 else pos[-1]
    cs_table = oi.rope_cos_sin(np.arange(table_rows), 64, 8e6)
    qo, ko = ops.indexer_prep(bf16_tensor(q, dev), bf16_tensor(k, dev), to_dev(w, dev), to_dev(b, dev), 1e-6,
                              to_dev(cs_table, dev), to_dev(pos, dev))
    cs = np.where((pos < table_rows)[:, None], cs_table[np.minimum(pos, table_rows - 1)],
                  np.concatenate([np.ones(32), np.zeros(32)]).astype(np.float32))
    rq, rk = oi.indexer_prep(q, k, w, b, 1e-6, cs.astype(np.float32))
    assert np.array_equal(bf16_values(ko), rk)
    assert np.array_equal(bf16_values(qo), rq)


@pytest.mark.parametrize("num_rows", [1, 2, 5, 6, 7, 64, 129, 1026])
def test_hadamard_rows_exact(dev, num_rows):
    from ernie_kv import ops

    rng = np.random.default_rng(num_rows)
    x = randn_bf16(rng, (num_rows, 128))
    y = bf16_values(ops.hadamard_rows(bf16_tensor(x, dev)))
    assert np.array_equal(y, oi.hadamard_rows(x))
    h = oi.hadamard_matrix() / np.sqrt(128)
    ref = x.astype(np.float64) @ h
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-2  # test_dsa_backend.py:73-89 bound


@pytest.mark.parametrize("w_dtype", ["bf16", "fp32"])
def test_indexer_q_quant_exact(dev, w_dtype):
    from ernie_kv import ops

    rng = np.random.default_rng(3)
    T, H = 5, 64
    q = randn_bf16(rng, (T, H, 128), scale=2.0)
    q[0, 0] = 0.0
    w = randn_bf16(rng, (T, H)) if w_dtype == "bf16" else rng.standard_normal((T, H)).astype(np.float32)
    wt = bf16_tensor(w, dev) if w_dtype == "bf16" else to_dev(w, dev)
    q8, wf, dig = ops.indexer_q_quant(bf16_tensor(q, dev), wt)
    codes, wref = oi.quantize_q(q, w)
    assert np.array_equal(q8.cpu().numpy(), codes)
    assert np.array_equal(wf.cpu().numpy().view(np.uint32), wref.view(np.uint32))
    iq = oi.int_repr(codes)
    d = dig.cpu().numpy().astype(np.int64)  # [T, 3, H, 128]
    recon = d[:, 0] + 64 * d[:, 1] + 4096 * d[:, 2]
    assert np.array_equal(recon, iq)
    assert np.abs(d).max() <= 63


def _keys(rng, n, kind, spikes):
    """Key rows of one sequence: N(0,1), plus structure that stresses the selection."""
    k = randn_bf16(rng, (n, 128))
    if kind == "prototypes":  # 40 distinct rows -> many exact ties at many levels
        k = randn_bf16(rng, (40, 128))[rng.integers(0, 40, n)]
    elif kind == "near_ties":  # one base row with tiny perturbations -> near-equal scores
        base = randn_bf16(rng, (128,))
        k = np.repeat(base[None], n, 0)
        j = rng.integers(0, 128, n)
        k[np.arange(n), j] = randn_bf16(rng, (n,)) * 0.05
    elif kind == "constant":  # every score equal -> every token is a candidate
        k = np.repeat(randn_bf16(rng, (1, 128)), n, 0)
    if spikes > 0:
        k[rng.random(n) < spikes] = randn_bf16(rng, (128,), 3.0)
    return k


def _indexer_setup(dev, rng, lengths, num_seqs=None, pages_per_seq=None, spikes=0.0, kind="normal"):
    T = len(lengths)
    num_seqs = num_seqs or T
    max_len = max(max(lengths), 1)
    pages_per_seq = pages_per_seq or (max_len + 63) // 64 + 1
    bt = permuted_block_table(rng, num_seqs, pages_per_seq)
    kv_pages = num_seqs * pages_per_seq
    kcache = np.zeros((kv_pages, paged.fp8_page_bytes(128)), np.uint8)
    req = np.arange(T, dtype=np.int32) % num_seqs
    for b in range(num_seqs):
        n = pages_per_seq * 64
        k = _keys(rng, n, kind, spikes)
        s = np.arange(n)
        slots = bt[b, s // 64] * 64 + s % 64
        c, sc = quantize_rows(k)
        paged.write_fp8_rows(kcache, slots, c, sc, 128)
    q = randn_bf16(rng, (T, 64, 128))
    w = randn_bf16(rng, (T, 64))
    return dict(bt=bt, kcache=kcache, req=req, q=q, w=w, max_len=max_len)


def test_indexer_scores_exact(dev):
    from ernie_kv import ops

    rng = np.random.default_rng(7)
    lengths = np.array([0, 1, 100, 777, 3000], np.int32)
    st = _indexer_setup(dev, rng, lengths)
    q8, wf, dig = ops.indexer_q_quant(bf16_tensor(st["q"], dev), bf16_tensor(st["w"], dev))
    T = len(lengths)
    scores = torch.full((T, st["max_len"]), -123.0, device=dev)
    ops.indexer_score(dig, wf, to_dev(st["kcache"], dev), to_dev(st["bt"], dev), to_dev(st["req"], dev),
                      to_dev(lengths, dev), st["max_len"], scores)
    codes, wref = oi.quantize_q(st["q"], st["w"])
    got = scores.cpu().numpy()
    for t in range(T):
        n = int(lengths[t])
        s = np.arange(n)
        slots = st["bt"][st["req"][t], s // 64] * 64 + s % 64
        kc, ks = paged.read_fp8_rows(st["kcache"], slots, 128)
        ref = oi.exact_scores(codes[t], wref[t], kc, ks)
        assert np.array_equal(got[t, :n].view(np.uint32), ref.view(np.uint32)), f"row {t}"
        assert np.all(got[t, n:] == -123.0)


@pytest.mark.parametrize("n", [0, 1, 2047, 2048, 2049, 131072])
def test_topk_select_spikes_and_ties(dev, n):
    """Scores N(0,1) with 5% exactly +4.0 (more spikes than k), lowest index wins ties."""
    from ernie_kv import ops

    rng = np.random.default_rng(n)
    rows = 3
    L = max(n, 1)
    sc = rng.standard_normal((rows, L)).astype(np.float32)
    sc[rng.random((rows, L)) < 0.05] = 4.0
    sc[1] = 1.5  # all equal
    sc[2, : L // 2] = -0.0  # signed zeros tie with +0
    sc[2, L // 2 :] = 0.0
    lengths = np.array([n, n, n], np.int32)
    out = torch.full((rows, TOPK), -9, dtype=torch.int32, device=dev)
    ops.topk_select(to_dev(sc, dev), to_dev(lengths, dev), TOPK, out)
    got = out.cpu().numpy()
    for r in range(rows):
        ref = oi.topk_ascending((sc[r, :n] + np.float32(0.0)).astype(np.float32), TOPK)
        assert np.array_equal(got[r], ref), f"row {r}"


@pytest.mark.parametrize("kind,spikes", [("normal", 0.05), ("normal", 0.0), ("prototypes", 0.0),
                                         ("near_ties", 0.0), ("constant", 0.0)])
def test_indexer_topk_end_to_end(dev, kind, spikes):
    """Filter + exact rescoring + exact select == oracle top-k, bit for bit."""
    from ernie_kv import ops

    rng = np.random.default_rng(17)
    lengths = np.array([0, 50, 2047, 2048, 2049, 2100, 9000, 20000], np.int32)
    st = _indexer_setup(dev, rng, lengths, spikes=spikes, kind=kind)
    q8, wf, dig = ops.indexer_q_quant(bf16_tensor(st["q"], dev), bf16_tensor(st["w"], dev))
    T = len(lengths)
    out = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    ops.indexer_topk(q8, dig, wf, to_dev(st["kcache"], dev), to_dev(st["bt"], dev), to_dev(st["req"], dev),
                     to_dev(lengths, dev), st["max_len"], out)
    codes, wref = oi.quantize_q(st["q"], st["w"])
    ref, _ = oi.indexer_topk(codes, wref, st["kcache"], st["bt"], st["req"], lengths, TOPK)
    assert np.array_equal(out.cpu().numpy(), ref)


def test_indexer_topk_stages_match_one_call(dev):
    """ekv_indexer_filter + ekv_indexer_select == ekv_indexer_topk, and the
    top-k rows hold only tokens of their own (windowed) range."""
    from ernie_kv import ops

    rng = np.random.default_rng(23)
    lengths = np.array([3000, 12000, 64], np.int32)
    st = _indexer_setup(dev, rng, lengths, num_seqs=2, spikes=0.05)
    q8, wf, dig = ops.indexer_q_quant(bf16_tensor(st["q"], dev), bf16_tensor(st["w"], dev))
    args = (to_dev(st["kcache"], dev), to_dev(st["bt"], dev), to_dev(st["req"], dev), to_dev(lengths, dev))
    T = len(lengths)
    a = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    b = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    ops.indexer_topk(q8, dig, wf, *args, st["max_len"], a)
    ws = ops.indexer_topk_workspace(T, st["max_len"], dev)
    ops.indexer_filter(q8, dig, wf, *args, st["max_len"], ws)
    ops.indexer_select(dig, wf, *args, st["max_len"], b, ws)
    assert torch.equal(a, b)
    # the select's merged output == ekv_merge_swa_topk of its top-k
    positions = torch.tensor(lengths.astype(np.int64) + WINDOW - 1, device=dev)
    positions[2] = 40  # shorter than the window: no top-k entries, a partial window
    c = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    merged = torch.full((T, TOPK + WINDOW + 5), -9, dtype=torch.int32, device=dev)
    ops.indexer_select(dig, wf, *args, st["max_len"], c, ws, merged=merged, positions=positions, window=WINDOW)
    assert torch.equal(a, c)
    ref_merged = torch.full_like(merged, -9)
    ops.merge_swa_topk(c, ref_merged, positions, WINDOW)
    assert torch.equal(merged, ref_merged)
    # merged_slots: the same entries as cache slots through the block table
    slots = torch.full_like(merged, -9)
    ops.indexer_select(dig, wf, *args, st["max_len"], c, ws, merged=slots, positions=positions, window=WINDOW,
                       merged_slots=True)
    bt = st["bt"][st["req"]]  # [T, pages] rows of each query's request
    m = ref_merged.cpu().numpy().astype(np.int64)
    in_table = (m >= 0) & (m // 64 < bt.shape[1])  # entries past the table are unmapped
    page = np.take_along_axis(bt, np.clip(m // 64, 0, bt.shape[1] - 1), axis=1)
    ref_slots = np.where(in_table, page * 64 + m % 64, -1)
    assert np.array_equal(slots.cpu().numpy(), ref_slots)
    got = a.cpu().numpy()
    for t in range(T):
        row = got[t][got[t] >= 0]
        assert len(row) == min(lengths[t], TOPK) and np.all(row < lengths[t]) and np.all(np.diff(row) > 0)
    # the one-call path (select inside the filter launch) writes the same
    # top-k, merged rows and slots
    for slots_mode, ref in ((False, ref_merged), (True, torch.from_numpy(ref_slots.astype(np.int32)).to(dev))):
        d = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
        m = torch.full((T, TOPK + WINDOW + 5), -9, dtype=torch.int32, device=dev)
        ops.indexer_topk_merged(q8, dig, wf, *args, st["max_len"], d, ws, merged=m, positions=positions,
                                window=WINDOW, merged_slots=slots_mode)
        assert torch.equal(a, d)
        assert torch.equal(m, ref)
    assert int(ws[:16].view(torch.int32).sum()) == 0
    assert int(ws[256: ops.indexer_topk_counter_bytes()].view(torch.int32).abs().sum()) == 0


def _device_cache(dev, seed, num_seqs, pages_per_seq, kind):
    """Indexer cache written on the device by ekv_indexer_k_insert (whose bytes
    are checked against the oracle in test_gpu_write), pages permuted."""
    from ernie_kv import ops

    g = torch.Generator(device=dev).manual_seed(seed)
    n = pages_per_seq * 64
    bt = torch.randperm(num_seqs * pages_per_seq, generator=g, device=dev).to(torch.int32)
    bt = bt.view(num_seqs, pages_per_seq).contiguous()
    kcache = torch.zeros((num_seqs * pages_per_seq, 64 * 132), dtype=torch.uint8, device=dev)
    s = torch.arange(n, device=dev)
    for b in range(num_seqs):
        if kind == "constant":  # every score of the row equal: every token is a candidate
            k = torch.randn(1, 128, generator=g, device=dev).to(torch.bfloat16).expand(n, 128).contiguous()
        else:
            k = torch.randn(n, 128, generator=g, device=dev).to(torch.bfloat16)
        slots = (bt[b, s // 64].to(torch.int64) * 64 + s % 64).contiguous()
        ops.indexer_k_insert(k, slots, kcache)
    return bt, kcache


def _topk_vs_exact_path(dev, lengths, num_seqs, max_len, kind, seed, ws=None, rows_per_seq=1):
    """ekv_indexer_topk against ekv_topk_select over ekv_indexer_score's exact
    scores (both bit-exact against the oracle in the tests above); returns the
    workspace of the top-k call (a new zero-filled one unless `ws` is given).
    With rows_per_seq > 1, rows R*i .. R*i+R-1 belong to sequence i (a
    sequence's token and draft rows), else row t to sequence t % num_seqs."""
    from ernie_kv import ops

    T = len(lengths)
    bt, kcache = _device_cache(dev, seed, num_seqs, max_len // 64 + 1, kind)
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    if rows_per_seq > 1:
        req = (torch.arange(T, dtype=torch.int32, device=dev) // rows_per_seq).contiguous()
    else:
        req = (torch.arange(T, dtype=torch.int32, device=dev) % num_seqs).contiguous()
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    q = torch.randn(T, 64, 128, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(T, 64, generator=g, device=dev).to(torch.bfloat16)
    q8, wf, dig = ops.indexer_q_quant(q, w)
    out = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    if ws is None:
        ws = ops.indexer_topk_workspace(T, max_len, dev)
    ops.indexer_topk(q8, dig, wf, kcache, bt, req, lens, max_len, out, ws)
    scores = torch.empty((T, max_len), dtype=torch.float32, device=dev)
    ops.indexer_score(dig, wf, kcache, bt, req, lens, max_len, scores)
    ref = torch.full_like(out, -9)
    ops.topk_select(scores, lens, TOPK, ref)
    bad = (out != ref).any(dim=1).nonzero().flatten().tolist()
    assert not bad, f"rows {bad} differ"
    return ws


@pytest.mark.parametrize("kind", ["normal", "constant"])
def test_indexer_topk_long_rows_match_exact_path(dev, kind):
    """Rows long enough that one filter workgroup owns more than 2048 tokens
    (constant keys: all of them candidates, scored over several passes)."""
    from ernie_kv import ops

    lengths = [262144, 200000, 131072, 70000, 2049, 5000, 0, 180000]
    T, max_len = len(lengths), 262144
    ws = _topk_vs_exact_path(dev, lengths, T, max_len, kind, seed=5)
    # the workspace starts with four counters of waits for the bound that
    # gave up, then (from byte 256) the fused kernel's per-row counters,
    # which every call leaves zero
    assert int(ws[:16].view(torch.int32).sum()) == 0
    assert int(ws[256: ops.indexer_topk_counter_bytes()].view(torch.int32).abs().sum()) == 0


def test_indexer_topk_million_token_row(dev):
    """A 1,048,576-token row (config 5's longest context) beside shorter
    ones, through the fused filter: same top-2048 as the exact path."""
    ws = _topk_vs_exact_path(dev, [1048576, 262144, 4096, 2049], 4, 1048576, "normal", seed=61)
    assert int(ws[:16].view(torch.int32).sum()) == 0


@pytest.mark.parametrize("rows", [2, 3])
def test_indexer_topk_draft_rows(dev, rows):
    """Draft-token rows (the decode layout's next_n = rows): 24 rows, R per
    sequence at consecutive positions, one sequence at 1M tokens -- too long
    for the one-launch plan, so the filter / bound / verify launches run, with
    a sequence's rows reading the same pages back to back.  Same top-2048 as
    the exact path."""
    S = 24 // rows
    lengths = []
    for s_ in range(S):
        ctx = 1048576 if s_ == 0 else 65536 + 777 * s_
        lengths += [ctx - rows + 1 + r for r in range(rows)]
    ws = _topk_vs_exact_path(dev, lengths, S, 1048576, "normal", seed=70 + rows, rows_per_seq=rows)
    assert int(ws[:16].view(torch.int32).sum()) == 0


def test_indexer_topk_workspace_reused_across_shapes(dev):
    """One zero-filled workspace for calls of different row counts and
    lengths (the fused kernel's counters sit at fixed offsets and are left
    zero), including a call that takes the unfused kernels in between."""
    from ernie_kv import ops

    ws = ops.indexer_topk_workspace(1100, 70000, dev)
    _topk_vs_exact_path(dev, [70000, 3000, 65000, 12345], 4, 70000, "normal", seed=31, ws=ws)
    _topk_vs_exact_path(dev, [5000, 2100, 0, 4096, 3333, 2048, 4097], 3, 5000, "normal", seed=32, ws=ws)
    rng = np.random.default_rng(33)
    _topk_vs_exact_path(dev, rng.integers(0, 3000, 1100).astype(np.int32).tolist(), 8, 3000, "normal", seed=34,
                        ws=ws)
    _topk_vs_exact_path(dev, [60000, 4000], 2, 60000, "constant", seed=35, ws=ws)
    assert int(ws[:16].view(torch.int32).sum()) == 0
    assert int(ws[256: ops.indexer_topk_counter_bytes()].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("kind", ["normal", "constant"])
def test_indexer_topk_rows_select_alone_when_waits_give_up(dev, kind):
    """With the waits' poll limit at 0 every workgroup that waits for the
    rest of its row gives up at once: its bound is bin 0 (every token a
    candidate) and the row's last workgroup to leave selects over the lists
    alone.  The top-k still equals the exact path's, the row count of those
    selects is counted, and the counters are left zero."""
    from ernie_kv import ops

    lengths = [70000, 2049, 0, 30000, 5000, 131072, 12345, 2048]
    T, max_len = len(lengths), 131072
    prev = ops.indexer_set_spin_limit(0)
    try:
        ws = _topk_vs_exact_path(dev, lengths, 4, max_len, kind, seed=81)
    finally:
        ops.indexer_set_spin_limit(prev)
    counts = ws[:16].view(torch.int32).cpu().numpy()
    long_rows = sum(1 for n in lengths if n > TOPK)
    assert counts[2] == long_rows, f"counters {counts}"  # every row with waits selected alone
    assert int(ws[256: ops.indexer_topk_counter_bytes()].view(torch.int32).abs().sum()) == 0
    # and with the default limit again, nothing gives up
    ws2 = _topk_vs_exact_path(dev, lengths, 4, max_len, kind, seed=82)
    assert int(ws2[:16].view(torch.int32).sum()) == 0


def test_indexer_topk_four_wave_plan(dev):
    """300 query rows: more than one per CU, so the one-launch plan takes
    4-wave workgroups (about three per CU, a row over one or two of them),
    with the select in the same launch; rows long enough that some lists
    exceed what the local select holds take the rounds over workgroups."""
    from ernie_kv import ops

    rng = np.random.default_rng(41)
    lengths = rng.integers(0, 9000, 300).astype(np.int32).tolist()
    lengths[:5] = [0, 2048, 2049, 9000, 6000]
    ws = _topk_vs_exact_path(dev, lengths, 12, 9000, "normal", seed=43)
    assert int(ws[:16].view(torch.int32).sum()) == 0
    ws = _topk_vs_exact_path(dev, lengths[:40], 12, 9000, "constant", seed=44)
    assert int(ws[:16].view(torch.int32).sum()) == 0
    assert int(ws[256: ops.indexer_topk_counter_bytes()].view(torch.int32).abs().sum()) == 0


def test_indexer_topk_many_rows(dev):
    """More query rows (1100) than one launch of the fused filter can hold
    at once: the filter / bound / verify kernels run instead."""
    rng = np.random.default_rng(29)
    lengths = rng.integers(0, 6000, 1100).astype(np.int32).tolist()
    lengths[:4] = [0, 2048, 2049, 6000]
    _topk_vs_exact_path(dev, lengths, 16, 6000, "normal", seed=9)


def _adversarial_fp8_operands(rng):
    """q [64, 128] and keys [S, 128] (e4m3fn codes) built to stress the fp8
    MFMA's accumulation: maximal products of alternating and block signs that
    cancel to 0, maximal products beside subnormal ones, a few large terms
    cancelled by many small ones, every code value, and random codes."""
    from oracle.fp8 import decode_table, encode_e4m3

    valid = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    big, tiny = 448.0, 2.0 ** -9
    alt = np.where(np.arange(128) % 2 == 0, big, -big)
    block = np.where(np.arange(128) < 64, big, -big)
    mixed = np.where(np.arange(128) % 2 == 0, big, tiny)
    mixed_neg = np.where(np.arange(128) % 2 == 0, big, -tiny)
    few_big = np.concatenate([np.full(4, big), np.full(124, -big * 4 / 124)])
    exps = 2.0 ** rng.integers(-9, 9, 128) * rng.choice([-1.0, 1.0], 128)
    pats = [alt, block, mixed, mixed_neg, few_big, exps, np.full(128, big), np.full(128, tiny)]
    q_rows = [np.full(128, big), alt, block, np.where(np.arange(128) % 4 < 2, big, -big), mixed, exps]
    q = np.stack([encode_e4m3(np.asarray(r, np.float32)) for r in q_rows])
    q = np.concatenate([q, rng.choice(valid, (64 - len(q), 128))]).astype(np.uint8)
    keys = [encode_e4m3(np.asarray(p, np.float32)) for p in pats]
    keys += [encode_e4m3(np.asarray(np.roll(p, r), np.float32)) for p in pats for r in (1, 17, 64)]
    keys += [np.resize(valid, 128), np.resize(valid[::-1], 128)]
    keys = np.stack(keys).astype(np.uint8)
    rand = rng.choice(valid, (16384 - len(keys) % 16, 128)).astype(np.uint8)
    # signs of a random key matched to q row 0 (all +448): dot = sum |k| * 448,
    # and flipped halves (large partial sums that cancel)
    flip = rand[:2048].copy()
    flip[:, 64:] ^= 0x80
    k = np.concatenate([keys, rand, flip])
    k = k[: len(k) // 16 * 16]
    assert np.isfinite(decode_table()[k]).all() and np.isfinite(decode_table()[q]).all()
    return q, k


def test_filter_mfma_error_bound(dev):
    """The filter drops a token only when its upper bound U = a + e falls
    below the k-th lower bound, with e built on the assumption that each
    head's fp8-MFMA dot product is within 2^-8 * 448^2 of the exact one.
    Pinned on this device with the filter's own MFMA call over adversarial
    cancellation patterns (maximal alternating / block signs, maximal beside
    subnormal products, every code) and 18K random keys."""
    from ernie_kv import ops

    rng = np.random.default_rng(2718)
    q, k = _adversarial_fp8_operands(rng)
    got = ops.indexer_filter_dots(to_dev(q, dev), to_dev(k, dev)).cpu().numpy().astype(np.float64)
    exact = (oi.int_repr(k) @ oi.int_repr(q).T).astype(np.float64) * 2.0 ** -18
    err = np.abs(got - exact)
    bound = 2.0 ** -8 * 448.0 ** 2
    worst = float(err.max())
    print(f"fp8 MFMA dot error: max {worst:.3f} = 2^{np.log2(max(worst, 1e-30)):.2f} * 1 "
          f"(bound 2^{np.log2(bound):.2f}); {int((err > 0).sum())} of {err.size} inexact")
    assert worst <= bound, f"fp8 MFMA error {worst} exceeds the filter's assumed bound {bound}"
