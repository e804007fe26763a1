"""GPU parity of the timed workloads at full size.

The DSA decode step exactly as ``bench.py`` times it (``build_dsa_decode`` +
``dsa_step``: the prologue with indexer prep folded into the one-launch
filter, exact scoring and select with the merged output as cache slots ->
decode) at 32 x 131,072
tokens with 5% spike keys at +4 sigma of each row's scores (every row's
top-2048 ends in a lowest-index tie among its spikes), the same step with one
random spike row in 5% of the positions, and the multi-token step at 8 x
262,144 + 1 x 1,048,576 tokens with 3 query rows per sequence, are checked
against:

* the GPU's exact path (``ekv_indexer_score`` + ``ekv_topk_select`` over the
  full score rows) for every query row, bit-exact;
* the numpy oracle for the rows whose top-k threshold is a tie among the
  spike keys and for further sampled rows: exact scores (as uint32 bits),
  top-k, merged rows (the window merge through the block table), and the
  decode output within
  |err| <= 2e-3 + 2e-2 |ref| (lse within 2e-3);
* the cache bytes the step appended, and the indexer workspace's diagnostic
  counters (waits that gave up, histograms that never summed, rows selected
  alone), which must stay 0.
"""

import numpy as np
import pytest
import torch

from helpers import bf16_values
from oracle import decode as od
from oracle import indexer as oi
from oracle.fp8 import quantize_rows
from oracle.merge import logical_to_global, merge_swa_topk

pytestmark = pytest.mark.gpu
TOPK, WINDOW = 2048, 128


def _say(msg):
    print(msg, flush=True)


def _oracle_scores(kcache_np, bt_row, n, codes_q, wf, chunk=131072):
    """Exact oracle scores of tokens 0..n-1 of one request, in chunks."""
    out = np.empty(n, np.float32)
    for s0 in range(0, n, chunk):
        s = np.arange(s0, min(n, s0 + chunk), dtype=np.int64)
        slots = bt_row[s // 64].astype(np.int64) * 64 + s % 64
        pages, rows = slots // 64, slots % 64
        codes = kcache_np[pages[:, None], rows[:, None] * 128 + np.arange(128)[None, :]]
        scol = 64 * 128 + rows[:, None] * 4 + np.arange(4)[None, :]
        scale = np.ascontiguousarray(kcache_np[pages[:, None], scol]).view(np.float32)[:, 0]
        out[s0:s0 + len(s)] = oi.exact_scores(codes_q, wf, codes, scale)
    return out


def _gather_latent(latent, slots, dim=576):
    """Dequantized fp64 rows of the fp8 latent cache at `slots` (gathered on
    the GPU, so the 2+ GB cache never crosses to the host)."""
    s = torch.from_numpy(np.asarray(slots, np.int64)).to(latent.device)
    pages, rows = s // 64, s % 64
    cols = rows[:, None] * dim + torch.arange(dim, device=latent.device)[None, :]
    codes = latent[pages[:, None], cols].cpu().numpy()
    scol = 64 * dim + rows[:, None] * 4 + torch.arange(4, device=latent.device)[None, :]
    scale = latent[pages[:, None], scol].contiguous().cpu().numpy().view(np.float32)[:, 0]
    from oracle.fp8 import decode_e4m3

    return decode_e4m3(codes).astype(np.float64) * scale.astype(np.float64)[:, None]


def _run_and_check(st, rows_to_check_extra, label, oracle_tie_rows=True):
    import bench
    from ernie_kv import ops

    B, dev = st["B"], st["kcache"].device
    _say(f"[{label}] step")
    bench.dsa_step(ops, st)
    torch.cuda.synchronize()
    counters = st["idx_ws"][:16].view(torch.int32).cpu().numpy()
    assert not counters.any(), f"indexer counters {counters}"
    topk = st["topk"].cpu().numpy()
    merged = st["merged"].cpu().numpy()
    positions = st["positions"].cpu().numpy()
    lengths = st["lengths"].cpu().numpy()
    req = st["req_ids"].cpu().numpy()
    bt = st["block_table"].cpu().numpy()
    assert np.array_equal(lengths, oi.windowed_lengths(positions, WINDOW))

    # the GPU's exact path over full score rows, every query row
    _say(f"[{label}] exact path")
    ctx = st["ctx"]
    scores = torch.empty((B, ctx), dtype=torch.float32, device=dev)
    ops.indexer_score(st["digits"], st["wf"], st["kcache"], st["block_table"], st["req_ids"], st["lengths"], ctx,
                      scores)
    top2 = torch.empty((B, TOPK), dtype=torch.int32, device=dev)
    ops.topk_select(scores, st["lengths"], TOPK, top2)
    top2 = top2.cpu().numpy()
    bad = [t for t in range(B) if not np.array_equal(topk[t], top2[t])]
    assert not bad, f"fused top-k differs from the exact path on rows {bad}"
    # the merged rows are cache slots: the window merge, then the block table
    want = logical_to_global(merge_swa_topk(topk, positions, merged.shape[1], WINDOW), req, bt)
    assert np.array_equal(merged, want)

    # the prologue's q / weights against the oracle's prep and quant
    _say(f"[{label}] prologue vs oracle")
    q_idx = bf16_values(st["q_idx"])
    k_new = bf16_values(st["k_new"])
    w_idx = bf16_values(st["w_idx"])
    rope = st["rope"].cpu().numpy()
    rq, rk = oi.indexer_prep(q_idx, k_new, st["ln_w"].cpu().numpy(), st["ln_b"].cpu().numpy(), 1e-6,
                             rope[positions])
    codes_q, wf = oi.quantize_q(rq, w_idx)
    assert np.array_equal(st["q8"].cpu().numpy(), codes_q)
    assert np.array_equal(st["wf"].cpu().numpy().view(np.uint32), wf.view(np.uint32))
    kcache_np = st["kcache"].cpu().numpy()
    slots = st["slots"].cpu().numpy()
    kc, ks = quantize_rows(rk)
    pg, r = slots // 64, slots % 64
    got_codes = kcache_np[pg[:, None], r[:, None] * 128 + np.arange(128)[None, :]]
    got_scale = np.ascontiguousarray(kcache_np[pg[:, None], 64 * 128 + r[:, None] * 4 + np.arange(4)[None, :]])
    assert np.array_equal(got_codes, kc) and np.array_equal(got_scale.view(np.float32)[:, 0], ks)

    # oracle rows: every row whose threshold is a tie, plus the extra ones
    sc_gpu = scores.cpu().numpy()
    tie_rows = []
    for t in range(B):
        n = int(lengths[t])
        sel = topk[t][topk[t] >= 0]
        if n <= TOPK or len(sel) == 0:
            continue
        thr = sc_gpu[t, sel].min()
        if (sc_gpu[t, :n] == thr).sum() > (sc_gpu[t, sel] == thr).sum():
            tie_rows.append(t)
    rows = sorted((set(tie_rows) if oracle_tie_rows else set()) | set(rows_to_check_extra))
    _say(f"[{label}] tie rows {tie_rows}; oracle rows {rows}")
    q_dec = bf16_values(st["q"])
    sinks = st["sinks"].cpu().numpy()
    out = bf16_values(st["out"]).astype(np.float64)
    lse = st["lse"].cpu().numpy().astype(np.float64)
    for t in rows:
        n = int(lengths[t])
        ref = _oracle_scores(kcache_np, bt[req[t]], n, codes_q[t], wf[t])
        assert np.array_equal(ref.view(np.uint32), sc_gpu[t, :n].view(np.uint32)), f"row {t}: scores differ"
        assert np.array_equal(oi.topk_ascending(ref, TOPK), topk[t]), f"row {t}: top-k differs"
        valid = merged[t][merged[t] >= 0]
        kv = _gather_latent(st["latent"], valid)
        ref_o, ref_l = od.sparse_mla_decode(q_dec[t:t + 1], lambda s: kv[s], np.arange(len(valid))[None],
                                            256 ** -0.5, 512, sinks)
        err = np.abs(out[t] - ref_o[0])
        assert np.all(err <= 2e-3 + 2e-2 * np.abs(ref_o[0])), f"row {t}: decode max err {err.max()}"
        assert np.all(np.abs(lse[t] - ref_l[0]) <= 2e-3 * np.maximum(1.0, np.abs(ref_l[0])))
        _say(f"[{label}] row {t} ok ({n} tokens)")
    return tie_rows


def test_headline_step_fullsize(dev):
    """The timed headline step: 32 x 131,072, N(0,1) keys, 5% spike keys per
    sequence at +4 sigma of its row's ordinary scores.  Every row's threshold
    is a tie among its spikes, broken by the lowest index: fused == the exact
    path on all 32 rows, the oracle on five of them."""
    import bench
    from ernie_kv import ops

    st = bench.build_dsa_decode(torch, ops, [131072] * 32, 0)
    sig = st["spikes"]["sigma"]
    assert min(sig) >= bench.SPIKE_SIGMA and max(sig) < bench.SPIKE_SIGMA + 0.05, sig
    ties = _run_and_check(st, [0, 5, 11, 20, 31], "b32_ctx131072", oracle_tie_rows=False)
    assert ties == list(range(32)), f"rows without a tie at the threshold: {sorted(set(range(32)) - set(ties))}"
    # the spikes are the threshold group: each row selects every ordinary
    # token above the spike score and then its lowest-index spikes
    topk = st["topk"].cpu().numpy()
    for t, cnt in enumerate(st["spikes"]["per_row"]):
        assert 2048 < cnt and (topk[t] >= 0).all()


def test_headline_random_spike_row_fullsize(dev):
    """The headline shape with uniformly random key codes and one random
    spike row copied into 5% of the positions (the random-row leg): every
    row against the exact path, the tie rows and three others against the
    oracle."""
    import bench
    from ernie_kv import ops

    st = bench.build_dsa_decode(torch, ops, [131072] * 32, 0, spikes="random_row")
    ties = _run_and_check(st, [0, 17, 31], "b32_ctx131072_random_row")
    assert len(ties) >= 1  # the random spike row ties the threshold of some rows


def test_mtp_step_fullsize(dev):
    """The multi-token DSA step at 8 x 262,144 + 1 x 1,048,576 (3 rows per
    sequence): the 1M sequence's three rows and one 262,144-token row
    against the oracle, all 27 rows against the exact path."""
    import bench
    from ernie_kv import ops

    st = bench.build_dsa_decode(torch, ops, bench.MTP_CTXS, 0, rows_per_seq=bench.MTP_ROWS, spike_frac=0.0)
    _run_and_check(st, [24, 25, 26, 4], "mtp")
