"""GPU parity of the benchmark workloads that are not the headline, at the
sizes ``bench.py`` times them, against the numpy oracle:

* the chunked-prefill cache write (16 sequences x 8192 tokens at offsets in
  [0, 64K), scattered into a 1M-slot pool, every completed 128-token span
  compressed, window and state rings updated): the whole pool and the state
  ring bit-exact;
* the multi-token decode steps (3 query rows per sequence) under an
  accept/reject schedule that re-appends rejected draft slots, DSA and HCA
  layers, checked after every step.
"""

import numpy as np
import pytest
import torch

from helpers import bf16_values
from oracle import hca as oh

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def test_chunked_prefill_write_fullsize(dev):
    """bench.build_hca_write + hca_write_step (the timed call) against
    oracle.hca.hca_write: every byte of the 1,048,576-slot pool (appended
    rows, compressed entries, window ring) and the compressor state ring."""
    import bench
    from ernie_kv import ops

    st = bench.build_hca_write(torch, ops, 0)
    B, D = st["B"], st["D"]
    state0 = bf16_values(st["state"])
    _say("[hca_write] GPU call")
    bench.hca_write_step(ops, st)
    torch.cuda.synchronize()
    record = 4 + (576 + 144) * 4
    ws = st["ws"]
    assert int(ws[: 4 * (ws.numel() // record)].sum()) == 0, "arrival counters left nonzero"
    pool = st["pool"].cpu().numpy()
    state = bf16_values(st["state"])
    _say(f"[hca_write] oracle ({st['spans_done']} spans)")
    ost = oh.HcaState(pool.shape[0], D, state0.shape[0])
    ost.state[:] = state0
    cpu = lambda k: st[k].cpu().numpy()  # noqa: E731
    oh.hca_write(ost, bf16_values(st["latent"]), bf16_values(st["kv_score"]), cpu("positions"), cpu("token_seq"),
                 cpu("qsl"), cpu("slots"), cpu("ring_pages"), 128, cpu("comp_bt"), cpu("state_slot"), cpu("ape"),
                 cpu("norm_w"), 1e-6, cpu("cos_sin"))
    bad = np.flatnonzero((pool != ost.pool).any(axis=1))
    assert bad.size == 0, f"{bad.size} pages differ, first {bad[:8]}"
    assert np.array_equal(state, ost.state), "state ring differs"
    # the call did compress every completed span: each compressed slot holds a row
    comp = cpu("comp_bt")
    offs = cpu("positions")[:: st["chunk"]]
    filled = 0
    for b in range(B):
        for j in range(offs[b] // 128, (offs[b] + st["chunk"]) // 128):
            slot = oh.comp_slot(comp, b, j)
            filled += int(pool[slot // 64, 64 * D + 4 * (slot % 64): 64 * D + 4 * (slot % 64) + 4].any())
    assert filled == st["spans_done"]


def _close(got, ref, what):
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 + 2e-2 * np.abs(ref)), f"{what}: max err {err.max()}"


def test_mtp_accept_reject_steps(dev):
    """Three decode steps of the multi-token schedule (3 query rows per
    sequence: the token and two drafts, drafts accepted with p = 0.7, the
    next step starting after the last accepted row, so rejected drafts'
    slots are written again) at reduced contexts, through the DSA step and
    the HCA step exactly as bench.py runs them.  After every step, against
    an oracle that applies the same writes to its own copy of the caches:
    the indexer K and latent cache bytes, top-k and merged rows, the HCA
    pool and state ring, the HCA index rows and both decode outputs."""
    import bench
    from ernie_kv import ops
    from oracle import decode as od
    from oracle import indexer as oi
    from oracle.fp8 import quantize_rows
    from oracle.merge import logical_to_global, merge_swa_topk
    from oracle.paged import write_fp8_rows

    ctxs = [3000, 3000, 5000, 9000]
    S, R, steps = len(ctxs), bench.MTP_ROWS, 3
    firsts, accepted = bench.mtp_schedule(ctxs, steps, 1)
    assert any(a < S * R for a in accepted), "the schedule rejects some drafts"
    grow = int(firsts[-1].max() - (max(ctxs) - R)) + 64
    offs = np.tile(np.arange(R), S)
    pos_steps = [np.repeat(f, R) + offs for f in firsts]

    # ---- DSA layer
    st = bench.build_dsa_decode(torch, ops, ctxs, 3, rows_per_seq=R, spike_frac=0.0, extra_tokens=grow)
    kc = st["kcache"].cpu().numpy()
    lat = st["latent"].cpu().numpy()
    bt = st["block_table"].cpu().numpy()
    req = st["req_ids"].cpu().numpy()
    q_idx, k_new, w_idx = bf16_values(st["q_idx"]), bf16_values(st["k_new"]), bf16_values(st["w_idx"])
    lat_new, q_dec = bf16_values(st["latent_new"]), bf16_values(st["q"])
    ln_w, ln_b = st["ln_w"].cpu().numpy(), st["ln_b"].cpu().numpy()
    rope, sinks = st["rope"].cpu().numpy(), st["sinks"].cpu().numpy()
    for i, pos in enumerate(pos_steps):
        _say(f"[mtp dsa] step {i} first positions {firsts[i].tolist()}")
        slots = bt[req, pos // 64].astype(np.int64) * 64 + pos % 64
        st["positions"] = torch.from_numpy(pos.astype(np.int64)).to(dev)
        st["slots"] = torch.from_numpy(slots).to(dev)
        bench.dsa_step(ops, st)
        torch.cuda.synchronize()
        assert not st["idx_ws"][:16].view(torch.int32).cpu().numpy().any()
        rq, rk = oi.indexer_prep(q_idx, k_new, ln_w, ln_b, 1e-6, rope[pos])
        oi.k_insert(kc, rk, slots)
        c, s_ = quantize_rows(lat_new)
        write_fp8_rows(lat, slots, c, s_, 576)
        assert np.array_equal(st["kcache"].cpu().numpy(), kc), f"step {i}: indexer K cache"
        assert np.array_equal(st["latent"].cpu().numpy(), lat), f"step {i}: latent cache"
        codes_q, wf = oi.quantize_q(rq, w_idx)
        lens = oi.windowed_lengths(pos, 128)
        top, _ = oi.indexer_topk(codes_q, wf, kc, bt, req, lens, 2048)
        assert np.array_equal(st["topk"].cpu().numpy(), top), f"step {i}: top-k"
        glob = logical_to_global(merge_swa_topk(top, pos, 2176, 128), req, bt)
        assert np.array_equal(st["merged"].cpu().numpy(), glob), f"step {i}: merged rows"
        ref_o, _ = od.sparse_mla_decode(q_dec, lambda sl: od.gather_rows_fp8(lat, sl, 576), glob, 256 ** -0.5, 512,
                                        sinks)
        _close(bf16_values(st["out"]).astype(np.float64), ref_o, f"step {i}: DSA decode")
    del st
    torch.cuda.empty_cache()

    # ---- HCA layer
    ring = 64 * ((128 + R - 1 + 63) // 64)
    sh = bench.build_hca_decode(torch, ops, 3, ctxs=ctxs, rows_per_seq=R, ring=ring, extra_tokens=grow)
    D = sh["D"]
    ost = oh.HcaState(sh["pool"].shape[0], D, sh["state"].shape[0])
    ost.pool[:] = sh["pool"].cpu().numpy()
    ost.state[:] = bf16_values(sh["state"])
    base = np.repeat(sh["base"].numpy(), R)
    lat_bt = sh["lat_bt"].numpy()
    sreq = np.repeat(np.arange(S), R)
    cpu = lambda k: sh[k].cpu().numpy()  # noqa: E731
    comp_bt, ring_pages, qsl = cpu("comp_bt"), cpu("ring_pages"), cpu("qsl")
    latent, kvs, qh = bf16_values(sh["latent"]), bf16_values(sh["kv_score"]), bf16_values(sh["q"])
    for i, pos in enumerate(pos_steps):
        _say(f"[mtp hca] step {i}")
        slots = (lat_bt[sreq, (pos - base) // 64] * 64 + (pos - base) % 64).astype(np.int64)
        sh["positions"] = torch.from_numpy(pos.astype(np.int64)).to(dev)
        sh["slots"] = torch.from_numpy(slots).to(dev)
        bench.hca_decode_step(ops, sh)
        torch.cuda.synchronize()
        oh.hca_write(ost, latent, kvs, pos, cpu("token_seq"), qsl, slots, ring_pages, ring, comp_bt, cpu("state_slot"),
                     cpu("ape"), cpu("norm_w"), 1e-6, cpu("cos_sin"))
        assert np.array_equal(sh["pool"].cpu().numpy(), ost.pool), f"step {i}: HCA pool"
        assert np.array_equal(bf16_values(sh["state"]), ost.state), f"step {i}: state ring"
        ref_idx, ref_len = oh.hca_decode_indices(pos, sreq, comp_bt, ring_pages, ring, sh["width"], call_qsl=qsl,
                                                 call_slots=slots)
        assert np.array_equal(sh["idx"].cpu().numpy(), ref_idx), f"step {i}: HCA index rows"
        assert np.array_equal(sh["lens"].cpu().numpy(), ref_len)
        ref_o, _ = od.sparse_mla_decode(qh, lambda sl: od.gather_rows_fp8(ost.pool, sl, D), ref_idx, 256 ** -0.5, 512,
                                        cpu("sinks"), lengths=ref_len)
        _close(bf16_values(sh["out"]).astype(np.float64), ref_o, f"step {i}: HCA decode")


def test_hca_layer_bf16_small(dev):
    """The small bf16 HCA layer workload (bench.build_hca_small: 4 sequences
    x 4096 tokens written in one prefill call into a bf16 paged cache with
    N(0, 0.02) compressor weights, then a 16-head decode of each sequence's
    last token over its 32 compressed entries and 128 window rows) against
    the oracle: the bf16 pool and state ring bit-exact, the index rows exact,
    the decode within |err| <= 2e-3 + 2e-2 |ref|."""
    import bench
    from ernie_kv import ops
    from oracle import decode as od
    from oracle.fp8 import bf16_from_bits

    st = bench.build_hca_small(torch, ops, 0)
    B, D, ctx = st["B"], st["D"], st["ctx"]
    _say("[hca_small] GPU step")
    bench.hca_small_step(ops, st)
    torch.cuda.synchronize()
    cpu = lambda k: st[k].cpu().numpy()  # noqa: E731
    pages = st["pool"].shape[0] // 64
    ost = oh.HcaState(pages, D, B, bf16=True)
    oh.hca_write(ost, bf16_values(st["latent"]), bf16_values(st["kv_score"]), cpu("positions"), cpu("token_seq"),
                 cpu("qsl"), cpu("slots"), cpu("ring_pages"), st["ring"], cpu("comp_bt"), cpu("state_slot"),
                 cpu("ape"), cpu("norm_w"), 1e-6, cpu("cos_sin"))
    got = st["pool"].view(torch.uint8).reshape(pages, -1).cpu().numpy()
    bad = np.flatnonzero((got != ost.pool).any(axis=1))
    assert bad.size == 0, f"{bad.size} pages differ"
    assert np.array_equal(bf16_values(st["state"]), ost.state)
    ref_idx, ref_len = oh.hca_decode_indices(cpu("q_pos"), cpu("req"), cpu("comp_bt"), cpu("ring_pages"), st["ring"],
                                             st["width"])
    assert np.array_equal(cpu("idx"), ref_idx) and np.array_equal(cpu("lens"), ref_len)
    assert (ref_len == ctx // 128 + 128).all()
    vals = bf16_from_bits(ost.pool.view(np.uint16).reshape(-1, D))
    ref_o, ref_l = od.sparse_mla_decode(bf16_values(st["q"]), lambda s: od.gather_rows_bf16(vals, s), ref_idx,
                                        st["scale"], 512, cpu("sinks"), lengths=ref_len)
    _close(bf16_values(st["out"]).astype(np.float64), ref_o, "decode")
    lse = cpu("lse").astype(np.float64)
    assert np.all(np.abs(lse - ref_l) <= 2e-3 * np.maximum(1.0, np.abs(ref_l)))
