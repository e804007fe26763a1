"""Pins of the MXFP4 indexer oracle (CPU): the e2m1 table and the
round-to-nearest encoding of triton.tools.mxfp.MXFP4Tensor off ties, the
scale's closed form, exact round trips, the reference's page-layout
known-answer test and an fp64 brute force of the scores."""

import math

import numpy as np
import pytest
import torch

from oracle import indexer as oi
from oracle import mxfp4 as om

mxfp = pytest.importorskip("triton.tools.mxfp")

TIES = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
TIES_UP = np.array([0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)


def test_e2m1_decode_table_matches_library():
    t = mxfp.MXFP4Tensor(size=(16,))
    t.data = torch.arange(16, dtype=torch.uint8)
    ref = t.to(torch.float32).numpy()
    mine = om.e2m1_decode(np.arange(16, dtype=np.uint8))
    np.testing.assert_array_equal(mine.view(np.uint32), ref.view(np.uint32))  # -0 for code 8


def test_e2m1_encode_matches_round_to_nearest_off_ties():
    rng = np.random.default_rng(0)
    y = np.concatenate([rng.uniform(-7.5, 7.5, 200_000), rng.uniform(-0.8, 0.8, 50_000),
                        [0.0, -0.0, 6.0, -6.0, 100.0, -1e-30, 1e-30]]).astype(np.float32)
    mids = np.concatenate([[0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]])
    near_tie = np.min(np.abs(np.abs(y)[:, None] - mids[None, :]), axis=1) < 1e-4
    y = y[~near_tie]
    ref = mxfp.MXFP4Tensor(data=torch.from_numpy(y.copy())).data.numpy()
    np.testing.assert_array_equal(om.e2m1_encode(y), ref)


def test_e2m1_ties_go_to_the_larger_magnitude():
    """The upstream recipe's rule at the seven midpoints (RNE would send 0.25,
    1.25, 2.5 and 5 down)."""
    for sgn in (1.0, -1.0):
        codes = om.e2m1_encode(np.float32(sgn) * TIES)
        np.testing.assert_array_equal(om.e2m1_decode(codes), np.float32(sgn) * TIES_UP)
    # just below a midpoint goes down
    below = np.nextafter(TIES, np.float32(0.0))
    np.testing.assert_array_equal(om.e2m1_decode(om.e2m1_encode(below)),
                                  np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0], np.float32))


def _closed_form_byte(amax: float) -> int:
    """Least k with amax <= 6 * 2**k (exact in float64), floored at -126; 0
    when the fp32 quotient amax / 6 underflows to zero (amax <= 3 * 2**-149)."""
    if amax <= 3.0 * 2.0 ** -149:
        return 0
    k = math.floor(math.log2(amax / 6.0)) - 2
    while 6.0 * 2.0 ** k < amax:
        k += 1
    return max(k, -126) + 127


def test_scale_byte_closed_form():
    rng = np.random.default_rng(1)
    amax = np.concatenate([
        np.abs(rng.standard_normal(20_000)) * 10.0 ** rng.uniform(-30, 30, 20_000),
        [6.0 * 2.0 ** k for k in range(-120, 120)],               # exact 6 * 2**k
        [np.nextafter(np.float32(6.0 * 2.0 ** k), np.float32(np.inf)) for k in range(-60, 60)],
        [np.nextafter(np.float32(6.0 * 2.0 ** k), np.float32(0)) for k in range(-60, 60)],
        [0.0, 1e-45, 1e-40, 3.0e38],
    ]).astype(np.float32)
    mine = om.scale_bytes(amax)
    ref = np.array([_closed_form_byte(float(a)) for a in amax], np.uint8)
    np.testing.assert_array_equal(mine, ref)


def test_quantize_bounds_and_round_trip():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 128)) * np.exp(rng.uniform(-8, 8, (64, 1)))).astype(np.float32)
    x[3, :32] = 0.0
    x[5, 40] = -0.0
    values, scales = om.quantize(x)
    assert values.shape == (64, 64) and scales.shape == (64, 4)
    assert scales[3, 0] == 0 and np.all(values[3, :16] == 0)
    xr = om.dequantize(values, scales)
    step = np.repeat(np.ldexp(1.0, scales.astype(np.int64) - 127), 32, axis=1)
    # nearest on the e2m1 grid: at most half a step (step = 2 * 0.5 * scale at the top)
    assert np.all(np.abs(xr - x) <= step * 1.0 + 1e-300)
    g = np.abs(x).reshape(64, 4, 32).max(-1)
    nz = g > 0
    s = np.ldexp(1.0, scales.astype(np.int64) - 127)
    assert np.all(g[nz] <= 6.0 * s[nz]) and np.all(g[nz] > 3.0 * s[nz])
    # representable inputs come back exactly (a 4 or 6 fixes each group's scale)
    codes = rng.integers(0, 16, (32, 128)).astype(np.uint8)
    codes[:, ::32] = rng.choice([6, 7, 14, 15], (32, 4))
    sb = rng.integers(100, 150, (32, 4)).astype(np.uint8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    xs = om.dequantize(packed, sb).astype(np.float32)
    v2, s2 = om.quantize(xs)
    np.testing.assert_array_equal(s2, sb)
    np.testing.assert_array_equal(v2, packed)


def test_store_layout_known_answer():
    """test_indexer_fp4.py:71-90: two rows into slots 0, 1 of a 9216-byte page
    filled with 173 -- values in bytes [0, 128), scales in [4096, 4104)."""
    rng = np.random.default_rng(3)
    k = rng.standard_normal((2, 128)).astype(np.float32)
    values, scales = om.quantize(k)
    storage = np.full((1, 9216), 173, np.uint8)
    om.store(storage, values, scales, np.array([0, 1]))
    np.testing.assert_array_equal(storage[0, :128].reshape(2, 64), values)
    np.testing.assert_array_equal(storage[0, 4096:4104].reshape(2, 4), scales)
    untouched = np.ones(9216, bool)
    untouched[:128] = False
    untouched[4096:4104] = False
    assert np.all(storage[0, untouched] == 173)
    # a negative slot is skipped; slot 64 + 3 lands in page 1 at offset 3
    st2 = np.full((2, 9216), 7, np.uint8)
    om.store(st2, values, scales, np.array([-1, 67]))
    assert np.all(st2[0] == 7)
    np.testing.assert_array_equal(st2[1, 3 * 64:4 * 64], values[1])
    np.testing.assert_array_equal(st2[1, 4096 + 12:4096 + 16], scales[1])
    assert om.FP4_ROW_BYTES == 68 and om.page_bytes() == 64 * 68


def test_exact_scores_against_fp64_brute_force():
    """The contract's scores against sum_h w * relu(q_hat . k_hat) in fp64 over
    the dequantized operands: equal up to the few fp32 roundings."""
    rng = np.random.default_rng(4)
    q = rng.standard_normal((64, 128)).astype(np.float32)
    q[:, 64:96] *= 40.0  # blocks of different scales
    k = rng.standard_normal((300, 128)).astype(np.float32)
    k[:, :32] *= 1e-3
    qv, qs = om.quantize(q)
    kv, ks = om.quantize(k)
    w = (rng.standard_normal(64) * 0.1).astype(np.float32)
    got = om.exact_scores(qv, qs, w, kv, ks).astype(np.float64)
    qh, kh = om.dequantize(qv, qs), om.dequantize(kv, ks)
    ref = np.maximum(kh @ qh.T, 0.0) @ w.astype(np.float64)
    tol = 1e-5 * (np.maximum(kh @ qh.T, 0.0) @ np.abs(w).astype(np.float64)) + 1e-30
    assert np.all(np.abs(got - ref) <= tol)
    # per-block integer dots: a swapped block or a dropped term moves the score
    iq, ik = om.int2(qv).reshape(64, 4, 32), om.int2(kv).reshape(300, 4, 32)
    d = np.einsum("sbd,hbd->shb", ik, iq).astype(np.float64)
    e = ks.astype(np.int64)[:, None, :] + qs.astype(np.int64)[None, :, :] - 256
    np.testing.assert_allclose((d * np.ldexp(1.0, e)).sum(-1), kh @ qh.T, rtol=1e-12, atol=0)


def test_topk_ties_lowest_index():
    """All-equal keys: the top-k is the first k tokens (lowest index wins)."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 64, 128)).astype(np.float32)
    qv, qs, w = om.quantize_q(q, np.ones((1, 64), np.float32))
    kv, ks = om.quantize(np.tile(rng.standard_normal((1, 128)).astype(np.float32), (200, 1)))
    cache = np.zeros((4, om.page_bytes()), np.uint8)
    om.store(cache, kv, ks, np.arange(200))
    bt = np.arange(4, dtype=np.int32)[None, :]
    top, scores = om.indexer_topk(qv, qs, w, cache, bt, np.zeros(1, np.int32), np.array([200]), 64)
    assert len(set(scores[0].tolist())) == 1
    np.testing.assert_array_equal(top[0], np.arange(64))
    np.testing.assert_array_equal(w, (np.ones((1, 64), np.float32) * oi.WEIGHTS_SCALE).astype(np.float32))
