"""MXFP4 indexer (use_fp4_kv) on the GPU against the oracle: quantization
bytes, the reference's page-layout known-answer test, exact scores, the
filter's MFMA error bound and the top-k through both filter plans, bit for
bit."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, permuted_block_table, randn_bf16, to_dev
from oracle import mxfp4 as om
from oracle.fp8 import bf16_round
from oracle.indexer import topk_ascending

pytestmark = pytest.mark.gpu

TOPK = 2048
WINDOW = 128


def _tie_rows(rng, rows):
    """bf16 rows whose groups hit every e2m1 midpoint exactly: each group holds
    6 * 2**s (fixing the scale at 2**s) and the seven midpoints times 2**s."""
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    x = np.zeros((rows, 128), np.float32)
    for r in range(rows):
        for grp in range(4):
            s = float(2.0 ** rng.integers(-20, 20))
            vals = np.concatenate([[6.0], mids, -mids, rng.uniform(-6, 6, 17)]).astype(np.float32)
            rng.shuffle(vals)
            x[r, 32 * grp:32 * grp + 32] = vals * np.float32(s)
    return bf16_round(x)


def test_mxfp4_quant_bytes(dev):
    from ernie_kv import ops

    rng = np.random.default_rng(1)
    x = randn_bf16(rng, (300, 128)) * np.exp(rng.uniform(-30, 30, (300, 1))).astype(np.float32)
    x = bf16_round(x.astype(np.float32))
    x[7, :32] = 0.0            # all-zero group: scale byte 0
    x[8, 40:72] = -0.0
    x[9, :] = 1e-38            # subnormal quotient amax / 6
    x[10:40] = _tie_rows(rng, 30)
    values, scales = ops.mxfp4_quant(bf16_tensor(x, dev))
    rv, rs = om.quantize(x)
    assert np.array_equal(scales.cpu().numpy(), rs)
    assert np.array_equal(values.cpu().numpy(), rv)


def test_indexer_q_quant_fp4(dev):
    from ernie_kv import ops

    rng = np.random.default_rng(2)
    T = 37
    full = randn_bf16(rng, (T, 64, 136), 2.0)  # strided heads: q = full[..., :128]
    full[3, 5, :64] = 0.0
    q = bf16_tensor(full, dev)[..., :128]
    w = randn_bf16(rng, (T, 64))
    values, scales, wout = ops.indexer_q_quant_fp4(q, bf16_tensor(w, dev))
    rv, rs, rw = om.quantize_q(full[..., :128], w)
    assert np.array_equal(values.cpu().numpy(), rv)
    assert np.array_equal(scales.cpu().numpy().view(np.uint8).reshape(T, 64, 4), rs)
    assert np.array_equal(wout.cpu().numpy().view(np.uint32), rw.view(np.uint32))


def test_k_insert_fp4_known_answer(dev):
    """test_indexer_fp4.py:71-90: rows of slots 0 and 1 in a 9216-byte page
    filled with 173 -- values at [0, 128), scales at [4096, 4104), nothing
    else written; then a permuted multi-page insert with skipped slots."""
    from ernie_kv import ops

    rng = np.random.default_rng(3)
    k = randn_bf16(rng, (2, 128))
    storage = torch.full((1, 9216), 173, dtype=torch.uint8, device=dev)
    ops.indexer_k_insert_fp4(bf16_tensor(k, dev), torch.tensor([0, 1], device=dev), storage)
    rv, rs = om.quantize(k)
    got = storage.cpu().numpy()
    assert np.array_equal(got[0, :128].reshape(2, 64), rv)
    assert np.array_equal(got[0, 4096:4104].reshape(2, 4), rs)
    mask = np.ones(9216, bool)
    mask[:128] = False
    mask[4096:4104] = False
    assert np.all(got[0, mask] == 173)

    T, pages = 500, 12
    k = randn_bf16(rng, (T, 128), 3.0)
    k[::7] = bf16_round(k[::7] * np.float32(1e-4))
    slots = rng.permutation(pages * 64)[:T].astype(np.int64)
    slots[::11] = -1
    cache = torch.full((pages, 9216), 173, dtype=torch.uint8, device=dev)
    ops.indexer_k_insert_fp4(bf16_tensor(k, dev), to_dev(slots, dev), cache)
    ref = np.full((pages, 9216), 173, np.uint8)
    om.k_insert(ref, k, slots)
    assert np.array_equal(cache.cpu().numpy(), ref)
    # _store_indexer_fp4 of the same rows (pre-quantized) writes the same bytes
    v, s = ops.mxfp4_quant(bf16_tensor(k, dev))
    cache2 = torch.full((pages, 9216), 173, dtype=torch.uint8, device=dev)
    ops.indexer_store_fp4(v, s, to_dev(slots, dev), cache2)
    assert torch.equal(cache, cache2)


def _keys(rng, n, kind, spikes):
    k = randn_bf16(rng, (n, 128))
    if kind == "prototypes":
        k = randn_bf16(rng, (40, 128))[rng.integers(0, 40, n)]
    elif kind == "constant":
        k = np.repeat(randn_bf16(rng, (1, 128)), n, 0)
    elif kind == "scaled":  # blocks of very different magnitudes
        k = k * np.exp(rng.uniform(-6, 6, (n, 4))).repeat(32, axis=1).astype(np.float32)
        k = bf16_round(k)
    if spikes > 0:
        k[rng.random(n) < spikes] = randn_bf16(rng, (128,), 3.0)
    return k


def _setup(rng, lengths, num_seqs=None, spikes=0.0, kind="normal"):
    T = len(lengths)
    num_seqs = num_seqs or T
    max_len = max(max(lengths), 1)
    pages_per_seq = (max_len + 63) // 64 + 1
    bt = permuted_block_table(rng, num_seqs, pages_per_seq)
    kcache = np.zeros((num_seqs * pages_per_seq, om.page_bytes()), np.uint8)
    for b in range(num_seqs):
        n = pages_per_seq * 64
        s = np.arange(n)
        om.k_insert(kcache, _keys(rng, n, kind, spikes), bt[b, s // 64] * 64 + s % 64)
    q = randn_bf16(rng, (T, 64, 128))
    q[:, :, 96:] *= np.float32(30.0)
    w = randn_bf16(rng, (T, 64))
    req = np.arange(T, dtype=np.int32) % num_seqs
    return dict(bt=bt, kcache=kcache, req=req, q=bf16_round(q), w=w, max_len=max_len)


def _dev_args(dev, st, lengths):
    return (to_dev(st["kcache"], dev), to_dev(st["bt"], dev), to_dev(st["req"], dev), to_dev(lengths, dev))


@pytest.mark.parametrize("kind", ["normal", "scaled"])
def test_indexer_scores_fp4_exact(dev, kind):
    from ernie_kv import ops

    rng = np.random.default_rng(7)
    lengths = np.array([0, 1, 100, 777, 3000], np.int32)
    st = _setup(rng, lengths, kind=kind)
    qv, qs, wf = ops.indexer_q_quant_fp4(bf16_tensor(st["q"], dev), bf16_tensor(st["w"], dev))
    T = len(lengths)
    scores = torch.full((T, st["max_len"]), -123.0, device=dev)
    ops.indexer_score_fp4(qv, qs, wf, *_dev_args(dev, st, lengths), st["max_len"], scores)
    rv, rs, rw = om.quantize_q(st["q"], st["w"])
    got = scores.cpu().numpy()
    for t in range(T):
        n = int(lengths[t])
        s = np.arange(n)
        kv, ks = om.read_rows(st["kcache"], st["bt"][st["req"][t], s // 64] * 64 + s % 64)
        ref = om.exact_scores(rv[t], rs[t], rw[t], kv, ks)
        assert np.array_equal(got[t, :n].view(np.uint32), ref.view(np.uint32)), f"row {t}"
        assert np.all(got[t, n:] == -123.0)


def test_filter_mfma_fp4_error_bound(dev):
    """The fp4 filter's bound assumes each head's scaled-MFMA dot product is
    within 2^-18 * M of the exact one, with M = 1152 * sum_b 2^(sq_b + sk_b -
    254) the largest magnitude the block scales allow (the rest of its 2^-16
    covers the contract's and the head sums' fp32 roundings).  The bound is on
    M, not on the actual block sums: the MFMA aligns its accumulation to the
    scales, so a large-scale block that sums to zero still costs precision.
    Pinned with the filter's own MFMA call over blocks of widely different
    scales that cancel, maximal blocks, all codes, and random rows.  Blocks
    sharing one scale are exact (every partial sum fits fp32)."""
    from ernie_kv import ops

    rng = np.random.default_rng(2719)
    S = 8192
    q_codes = rng.integers(0, 16, (64, 128)).astype(np.uint8)
    k_codes = rng.integers(0, 16, (S, 128)).astype(np.uint8)
    q_codes[0] = 7                       # all +6
    q_codes[1, ::2], q_codes[1, 1::2] = 7, 15  # +6, -6 alternating
    k_codes[:64] = 7
    k_codes[64:128, :64], k_codes[64:128, 64:] = 7, 15
    qs = rng.integers(100, 154, (64, 4)).astype(np.uint8)
    ks = rng.integers(100, 154, (S, 4)).astype(np.uint8)
    qs[:8] = 127                          # equal scales: exact
    ks[:1024] = 127
    ks[2048:4096, 0] = 150                # one dominant block cancelled ...
    ks[2048:4096, 1:] = 104               # ... beside tiny ones
    pack = lambda c: (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)
    qv, kv = pack(q_codes), pack(k_codes)
    got = ops.indexer_filter_dots_fp4(to_dev(qv, dev), to_dev(qs.view(np.int32).reshape(64), dev),
                                      to_dev(kv, dev), to_dev(ks.view(np.int32).reshape(S), dev))
    got = got.cpu().numpy().astype(np.float64)
    iq, ik = om.int2(qv).reshape(64, 4, 32), om.int2(kv).reshape(S, 4, 32)
    d = np.einsum("sbd,hbd->shb", ik, iq).astype(np.float64)
    e = ks.astype(np.int64)[:, None, :] + qs.astype(np.int64)[None, :, :] - 256
    tb = d * np.ldexp(1.0, e)
    exact = tb.sum(-1)
    mag = np.abs(tb).sum(-1)
    pot = 1152.0 * np.ldexp(1.0, e + 2).sum(-1)  # 1152 * sum_b 2^(sq_b + sk_b - 254)
    err = np.abs(got - exact)
    rel = err / pot
    worst = float(rel.max())
    act = np.where(mag > 0, err / np.where(mag > 0, mag, 1.0), 0.0)
    print(f"fp4 MFMA dot error: max 2^{np.log2(max(worst, 1e-300)):.2f} of M "
          f"(2^{np.log2(max(float(act.max()), 1e-300)):.2f} of sum_b |T_b|); "
          f"{int((err > 0).sum())} of {err.size} inexact")
    assert np.all(err[:1024, :8] == 0.0), "equal-scale blocks must be exact"
    assert worst <= 2.0 ** -18, f"fp4 MFMA error 2^{np.log2(worst):.2f} exceeds the filter's 2^-18"


@pytest.mark.parametrize("kind,spikes", [("normal", 0.05), ("normal", 0.0), ("prototypes", 0.0),
                                         ("constant", 0.0), ("scaled", 0.0)])
def test_indexer_topk_fp4_end_to_end(dev, kind, spikes):
    """Filter + exact rescoring + exact select == oracle top-k, bit for bit."""
    from ernie_kv import ops

    rng = np.random.default_rng(17)
    lengths = np.array([0, 50, 2047, 2048, 2049, 2100, 9000, 20000], np.int32)
    st = _setup(rng, lengths, spikes=spikes, kind=kind)
    qv, qs, wf = ops.indexer_q_quant_fp4(bf16_tensor(st["q"], dev), bf16_tensor(st["w"], dev))
    T = len(lengths)
    out = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    ws = ops.indexer_topk_workspace(T, st["max_len"], dev)
    ops.indexer_topk_fp4(qv, qs, wf, *_dev_args(dev, st, lengths), st["max_len"], out, ws)
    rv, rs, rw = om.quantize_q(st["q"], st["w"])
    ref, _ = om.indexer_topk(rv, rs, rw, st["kcache"], st["bt"], st["req"], lengths, TOPK)
    assert np.array_equal(out.cpu().numpy(), ref)
    assert int(ws[:16].view(torch.int32).sum()) == 0  # no wait gave up


def test_indexer_topk_fp4_stages_and_merge(dev):
    """filter_fp4 + select_fp4 == topk_fp4; the merged output equals
    merge_swa_topk of the top-k."""
    from ernie_kv import ops

    rng = np.random.default_rng(23)
    lengths = np.array([3000, 12000, 64], np.int32)
    st = _setup(rng, lengths, num_seqs=2, spikes=0.05)
    qv, qs, wf = ops.indexer_q_quant_fp4(bf16_tensor(st["q"], dev), bf16_tensor(st["w"], dev))
    args = _dev_args(dev, st, lengths)
    T = len(lengths)
    a = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    b = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    ops.indexer_topk_fp4(qv, qs, wf, *args, st["max_len"], a)
    ws = ops.indexer_topk_workspace(T, st["max_len"], dev)
    positions = torch.tensor(lengths.astype(np.int64) + WINDOW - 1, device=dev)
    merged = torch.full((T, TOPK + WINDOW), -9, dtype=torch.int32, device=dev)
    ops.indexer_filter_fp4(qv, qs, wf, *args, st["max_len"], ws)
    ops.indexer_select_fp4(qv, qs, wf, *args, st["max_len"], b, ws, merged=merged, positions=positions,
                           window=WINDOW)
    assert torch.equal(a, b)
    ref_merged = torch.full_like(merged, -9)
    ops.merge_swa_topk(a, ref_merged, positions, WINDOW)
    assert torch.equal(merged, ref_merged)
    # the one-call path (select inside the filter launch)
    c = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    m2 = torch.full_like(merged, -9)
    ops.indexer_topk_merged_fp4(qv, qs, wf, *args, st["max_len"], c, ws, merged=m2, positions=positions,
                                window=WINDOW)
    assert torch.equal(a, c)
    assert torch.equal(m2, ref_merged)
    assert int(ws[:16].view(torch.int32).sum()) == 0


def test_indexer_topk_fp4_many_rows(dev):
    """1100 query rows: more than the fused filter takes in one launch, so the
    filter / bound / verify kernels run; checked against the exact scores
    (oracle-pinned above) through the exact select, and three rows against the
    oracle."""
    from ernie_kv import ops

    rng = np.random.default_rng(29)
    lengths = rng.integers(0, 6000, 1100).astype(np.int32)
    lengths[:4] = [0, 2048, 2049, 6000]
    st = _setup(rng, [int(x) for x in lengths], num_seqs=16, spikes=0.02)
    qv, qs, wf = ops.indexer_q_quant_fp4(bf16_tensor(st["q"], dev), bf16_tensor(st["w"], dev))
    args = _dev_args(dev, st, lengths)
    T = len(lengths)
    out = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    ops.indexer_topk_fp4(qv, qs, wf, *args, st["max_len"], out)
    scores = torch.zeros((T, st["max_len"]), device=dev)
    ops.indexer_score_fp4(qv, qs, wf, *args, st["max_len"], scores)
    ref = torch.full_like(out, -9)
    ops.topk_select(scores, args[3], TOPK, ref)
    assert torch.equal(out, ref)
    rv, rs, rw = om.quantize_q(st["q"], st["w"])
    got = out.cpu().numpy()
    for t in (1, 2, 3):
        n = int(lengths[t])
        s = np.arange(n)
        kv, ks = om.read_rows(st["kcache"], st["bt"][st["req"][t], s // 64] * 64 + s % 64)
        assert np.array_equal(got[t], topk_ascending(om.exact_scores(rv[t], rs[t], rw[t], kv, ks), TOPK))
