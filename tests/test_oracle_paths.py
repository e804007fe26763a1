"""Pins of the oracle's path functions (CPU): page geometry, merge, indexer,
compressor and decode, against reference known-answer tests, closed forms,
library routines and brute force."""

import math

import numpy as np
import pytest
import torch

from oracle import decode as od
from oracle import hca as oh
from oracle import indexer as oi
from oracle import paged
from oracle.fp8 import bf16_round, decode_e4m3, quantize_rows
from oracle.merge import logical_to_global, merge_swa_topk

WINDOW, TOPK = 128, 2048


# ---------------------------------------------------------------- geometry
def test_packed_block_stride_alignment_closed_form():
    """test_dsa_backend.py:40-55 and attention.py:561-571."""
    a = math.lcm(512, 512 * 2, (512 + 64) * 2)
    assert a == 9216 and a % 512 == 0 and a % 1024 == 0 and a % 1152 == 0


def test_indexer_page_layout_values_then_scales():
    """Layout analog of test_indexer_fp4.py:71-90 for 132-byte fp8 rows:
    values at slot*128, scales at 64*128 + slot*4 of a page filled with 173."""
    rng = np.random.default_rng(0)
    k = bf16_round(rng.standard_normal((2, 128)).astype(np.float32))
    cache = np.full((1, 64 * 132), 173, np.uint8)
    oi.k_insert(cache, k, np.array([0, 1]))
    codes, scale = quantize_rows(k)
    assert np.array_equal(cache[0, :256].reshape(2, 128), codes)
    assert np.array_equal(cache[0, 8192:8200].view(np.float32), scale)
    assert np.all(cache[0, 256:8192] == 173) and np.all(cache[0, 8200:] == 173)


def test_slot_math_brute_force():
    rng = np.random.default_rng(1)
    bt = rng.permutation(40).astype(np.int32).reshape(4, 10)
    seq = rng.integers(0, 4, 500)
    pos = rng.integers(0, 640, 500)
    slots = paged.slots_from_block_table(bt, seq, pos)
    for s, p, sl in zip(seq, pos, slots):
        assert sl == bt[s][p // 64] * 64 + p % 64
    # logical->global keeps -1
    idx = np.array([[0, 63, 64, -1, 639]], np.int32)
    g = logical_to_global(idx, np.array([2]), bt)
    assert g[0, 3] == -1 and g[0, 2] == bt[2, 1] * 64 and g[0, 4] == bt[2, 9] * 64 + 63


def test_negative_slots_skipped():
    cache = np.zeros((1, paged.fp8_page_bytes(128)), np.uint8)
    paged.write_fp8_rows(cache, [-1], np.ones((1, 128), np.uint8), np.ones(1, np.float32), 128)
    assert not cache.any()


# ---------------------------------------------------------------- merge
def test_merge_swa_topk_known_answer():
    """Transcription of test_dsa_backend.py:18-37."""
    positions = np.array([0, 5, 127, 128, 200, 2175, 2176, 5000])
    rng = np.random.default_rng(0)
    topk = rng.integers(0, 1 << 20, (len(positions), TOPK)).astype(np.int32)
    width = TOPK + WINDOW
    out = merge_swa_topk(topk, positions, width, WINDOW)
    for row, pos in enumerate(positions):
        seq = pos + 1
        n, w = min(max(seq - WINDOW, 0), TOPK), min(seq, WINDOW)
        exp = np.full(width, -1, np.int32)
        exp[:n] = topk[row, :n]
        exp[n : n + w] = np.arange(seq - w, seq)
        assert np.array_equal(out[row], exp)


# ---------------------------------------------------------------- indexer prep
@pytest.mark.parametrize("num_rows", [1, 2, 5, 6, 7, 64, 129, 1026])
def test_hadamard_matches_dense(num_rows):
    """test_dsa_backend.py:73-89 bound, and exact orthonormality in fp64."""
    rng = np.random.default_rng(num_rows)
    x = bf16_round(rng.standard_normal((num_rows, 128)).astype(np.float32))
    h = oi.hadamard_matrix() / math.sqrt(128)
    ref = x.astype(np.float64) @ h
    out = oi.hadamard_rows(x)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-2
    assert np.allclose(h @ h.T, np.eye(128))


def test_partial_rope_split_cat_bit_exact():
    """test_indexer_rope.py:14-48: rotating dims 0..63 of the full head equals
    rotating the split part and concatenating; dims 64..127 untouched."""
    rng = np.random.default_rng(3)
    T, H = 7, 64
    pos = rng.integers(0, 65536, T)
    cs = oi.rope_cos_sin(pos, 64, 8e6)
    q = bf16_round(rng.standard_normal((T, H, 128)).astype(np.float32))
    full = oi.neox_partial_rope(q, cs[:, None, :], 64)
    part = oi.neox_partial_rope(q[..., :64], cs[:, None, :], 64)
    assert np.array_equal(full, np.concatenate([part, q[..., 64:]], -1))
    # rotation preserves the pair norm up to bf16 rounding
    n0 = np.hypot(q[..., :32], q[..., 32:64])
    n1 = np.hypot(full[..., :32], full[..., 32:64])
    assert np.allclose(n0, n1, rtol=2e-2, atol=1e-2)


def test_layer_norm_rows_against_fp64_torch():
    """The k_norm restatement (attention.py:912, 962) against
    torch.nn.functional.layer_norm in fp64: within one bf16 rounding."""
    rng = np.random.default_rng(41)
    x = bf16_round((rng.standard_normal((300, 128)) * rng.uniform(0.01, 30, (300, 1))
                    + rng.uniform(-5, 5, (300, 1))).astype(np.float32))
    w = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    b = (0.1 * rng.standard_normal(128)).astype(np.float32)
    got = oi.layer_norm_rows(x, w, b, 1e-6)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (128,), torch.from_numpy(w).double(),
                                         torch.from_numpy(b).double(), 1e-6).numpy()
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-5)
    assert np.array_equal(got, bf16_round(got))


def test_layer_norm_rows_closed_forms():
    """A constant row normalizes to the bias exactly; with eps = 0, scaling a
    row by a power of two leaves every output bit unchanged; the reduction
    order sums to the exact row sum within fp32 rounding."""
    rng = np.random.default_rng(42)
    w = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    b = bf16_round((0.1 * rng.standard_normal(128)).astype(np.float32))
    const = np.full((3, 128), 1.5, np.float32)
    assert np.array_equal(oi.layer_norm_rows(const, w, b, 1e-6), np.broadcast_to(b, (3, 128)))
    x = bf16_round(rng.standard_normal((50, 128)).astype(np.float32))
    base = oi.layer_norm_rows(x, w, b, 0.0)
    for k in (-3, 5, 11):
        assert np.array_equal(oi.layer_norm_rows((x * np.float32(2.0 ** k)).astype(np.float32), w, b, 0.0), base)
    s = oi._chunk_tree_sum(x)
    np.testing.assert_allclose(s, x.astype(np.float64).sum(-1), rtol=0, atol=1e-4)
    # unit weight, zero bias: every row has mean 0 and (biased) variance 1
    # up to the bf16 rounding, which averages out over 128 entries
    y = oi.layer_norm_rows(x, np.ones(128, np.float32), np.zeros(128, np.float32), 0.0).astype(np.float64)
    assert np.abs(y.mean(-1)).max() < 2e-3
    assert np.abs((y * y).mean(-1) - 1.0).max() < 2e-3


def test_indexer_prep_at_position_zero_is_norm_then_hadamard():
    """At position 0 the rotation is the identity (cos 1, sin 0), so the prep
    reduces to hadamard(k_norm(k)) and hadamard(q), bit for bit."""
    rng = np.random.default_rng(43)
    q = bf16_round(rng.standard_normal((3, 64, 128)).astype(np.float32))
    k = bf16_round(rng.standard_normal((3, 128)).astype(np.float32))
    w = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    b = (0.1 * rng.standard_normal(128)).astype(np.float32)
    cs = oi.rope_cos_sin(np.zeros(3, np.int64), 64, 8e6)
    qh, kh = oi.indexer_prep(q, k, w, b, 1e-6, cs)
    assert np.array_equal(kh, oi.hadamard_rows(oi.layer_norm_rows(k, w, b, 1e-6)))
    assert np.array_equal(qh, oi.hadamard_rows(q))


def test_q_quant_weight_fold():
    """attention.py:925, 980: w * q_scale * 128**-0.5 * 64**-0.5."""
    rng = np.random.default_rng(4)
    q = bf16_round(rng.standard_normal((3, 64, 128)).astype(np.float32) * 5)
    w = bf16_round(rng.standard_normal((3, 64)).astype(np.float32))
    codes, folded = oi.quantize_q(q, w)
    _, qs = quantize_rows(q)
    np.testing.assert_allclose(folded, w * qs / (8 * math.sqrt(128)), rtol=1e-6)


# ---------------------------------------------------------------- scoring / top-k
def test_exact_dot_equals_fp64_dot():
    """The int representation is exact: int64 dot == fp64 dot of decoded values."""
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (500, 128)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    q = rng.integers(0, 256, (64, 128)).astype(np.uint8)
    q[(q & 0x7F) == 0x7F] = 0
    d_int = oi.int_repr(codes) @ oi.int_repr(q).T
    d_f64 = decode_e4m3(codes).astype(np.float64) @ decode_e4m3(q).astype(np.float64).T
    assert np.array_equal(d_int.astype(np.float64) * 2.0 ** -18, d_f64)


def test_scores_match_fp64_formula():
    rng = np.random.default_rng(6)
    k = bf16_round(rng.standard_normal((300, 128)).astype(np.float32))
    kc, ks = quantize_rows(k)
    q = bf16_round(rng.standard_normal((64, 128)).astype(np.float32))
    w = rng.standard_normal(64).astype(np.float32)
    qc, wf = oi.quantize_q(q[None], w[None])
    s = oi.exact_scores(qc[0], wf[0], kc, ks)
    kv = decode_e4m3(kc).astype(np.float64) * ks[:, None]
    qv = decode_e4m3(qc[0]).astype(np.float64)
    ref = (np.maximum(kv @ qv.T, 0) * wf[0].astype(np.float64)).sum(1)
    np.testing.assert_allclose(s, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


def test_head_sum_order_is_pinned():
    """A planted mistake: summing heads in natural order differs from the
    kernel order on some inputs, so the pin is not vacuous."""
    rng = np.random.default_rng(7)
    p = (rng.standard_normal((2000, 64)) * np.exp2(rng.integers(-20, 20, (2000, 64)))).astype(np.float32)
    pinned = oi.head_sum_pinned(p)
    natural = np.zeros(2000, np.float32)
    for h in range(64):
        natural = (natural + p[:, h]).astype(np.float32)
    assert np.any(pinned != natural)
    np.testing.assert_allclose(pinned, p.astype(np.float64).sum(1), rtol=1e-4, atol=1e-3 * np.abs(p).max())


@pytest.mark.parametrize("n", [0, 5, 2048, 2049, 40000])
def test_topk_reduces_to_stable_sort(n):
    rng = np.random.default_rng(n)
    s = rng.standard_normal(n).astype(np.float32)
    s[rng.random(n) < 0.05] = 4.0
    got = oi.topk_ascending(s, TOPK)
    if n:
        order = torch.sort(-torch.from_numpy(s), stable=True).indices[: min(n, TOPK)].numpy()
        exp = np.sort(order)
    else:
        exp = np.zeros(0, np.int64)
    assert np.array_equal(got[: len(exp)], exp) and np.all(got[len(exp) :] == -1)


def test_topk_special_cases():
    assert np.array_equal(oi.topk_ascending(np.full(5000, 1.5, np.float32), TOPK), np.arange(TOPK))
    s = np.zeros(3000, np.float32)
    s[:1500] = -0.0
    assert np.array_equal(oi.topk_ascending(s + np.float32(0.0), TOPK), np.arange(TOPK))


def test_windowed_lengths():
    assert list(oi.windowed_lengths(np.array([0, 127, 128, 200]), 128)) == [0, 0, 1, 73]


# ---------------------------------------------------------------- compressor
def _span(rng, D=576):
    kv = bf16_round(rng.standard_normal((128, D)).astype(np.float32))
    sc = bf16_round(rng.standard_normal((128, D)).astype(np.float32))
    return kv, sc


def _fp64_compress(kv, score, ape, w, eps, cs):
    g = score.astype(np.float64) + ape
    p = np.exp(g - g.max(0))
    p /= p.sum(0)
    x = (p * kv).sum(0)
    y = x / np.sqrt((x * x).mean() + eps) * w
    D = len(y)
    x0, x1 = y[D - 64 :: 2].copy(), y[D - 63 :: 2].copy()
    y[D - 64 :: 2] = x0 * cs[:32] - x1 * cs[32:]
    y[D - 63 :: 2] = x0 * cs[32:] + x1 * cs[:32]
    return y


def test_compressor_fp64_brute_force():
    rng = np.random.default_rng(8)
    kv, sc = _span(rng)
    ape = (rng.standard_normal((128, 576)) * 0.5).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(576)).astype(np.float32)
    cs = oi.rope_cos_sin(np.array([128 * 7]), 64, 1.6e5)[0]
    got = oh.compress_span(kv, sc, ape, w, 1e-6, cs)
    ref = _fp64_compress(kv, sc, ape, w, 1e-6, cs)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_compressor_fp64_brute_force_with_moving_shift():
    """Gates that rise along the span (0 .. 60, plus noise): every row group's
    shift moves many times, and the result still matches the fp64 softmax."""
    rng = np.random.default_rng(13)
    kv, sc = _span(rng)
    ramp = np.linspace(0.0, 60.0, 128, dtype=np.float32)[:, None]
    sc = bf16_round((ramp + rng.standard_normal((128, 576))).astype(np.float32))
    ape = (rng.standard_normal((128, 576)) * 0.5).astype(np.float32)
    w = np.ones(576, np.float32)
    cs = oi.rope_cos_sin(np.array([128 * 3]), 64, 1.6e5)[0]
    got = oh.compress_span(kv, sc, ape, w, 1e-6, cs)
    ref = _fp64_compress(kv, sc, ape, w, 1e-6, cs)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_compressor_constant_gate_is_mean_and_one_hot_is_copy():
    rng = np.random.default_rng(9)
    kv, _ = _span(rng)
    zero = np.zeros((128, 576), np.float32)
    one = np.ones(576, np.float32)
    ident = np.concatenate([np.ones(32), np.zeros(32)]).astype(np.float32)
    y = oh.compress_span(kv, zero, zero, one, 0.0, ident)
    m = kv.astype(np.float64).mean(0)
    np.testing.assert_allclose(y, m / np.sqrt((m * m).mean()), rtol=1e-5, atol=1e-6)
    hot = zero.copy()
    hot[37] = 100.0
    y = oh.compress_span(kv, hot, zero, one, 0.0, ident)
    c = kv[37].astype(np.float64)
    np.testing.assert_allclose(y, c / np.sqrt((c * c).mean()), rtol=1e-5)


def test_compressor_permutation_invariance():
    rng = np.random.default_rng(10)
    kv, sc = _span(rng)
    ape = (rng.standard_normal((128, 576)) * 0.5).astype(np.float32)
    one = np.ones(576, np.float32)
    cs = oi.rope_cos_sin(np.array([0]), 64, 1.6e5)[0]
    perm = rng.permutation(128)
    a = oh.compress_span(kv, sc, ape, one, 1e-6, cs)
    b = oh.compress_span(kv[perm], sc[perm], ape[perm], one, 1e-6, cs)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("D", [512, 576])
def test_compressor_rope_is_undone_by_the_reference_inverse_rope(D):
    """The compressor's rotation of the last 64 channels is the one the
    reference's own post-attention kernel inverts: ``_vha_inv_rope_quant_kernel``
    (attention.py:166-229) maps each interleaved pair (2i, 2i+1) of the rope
    dims to ``(e cos + o sin, o cos - e sin)`` with ``cos | sin`` from the same
    table row (``:208-219``), restated as ``oracle.quant.vha_inv_rope_quant``.
    Applied at the same position to a compressed row it must give back the
    row before its rotation (the compressor run with cos = 1, sin = 0), within
    fp32 rounding.  A compressor that rotated NeoX halves (i, i + 32), or
    rotated the other way, fails this."""
    from oracle import quant as oq

    rng = np.random.default_rng(21)
    kv, sc = _span(rng, D)
    ape = (rng.standard_normal((128, D)) * 0.5).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    pos = 128 * 500
    cs = oi.rope_cos_sin(np.array([pos]), 64, 1.6e5)[0]
    ident = np.concatenate([np.ones(32, np.float32), np.zeros(32, np.float32)])
    rotated = oh.compress_span(kv, sc, ape, w, 1e-6, cs)
    plain = oh.compress_span(kv, sc, ape, w, 1e-6, ident)
    assert np.array_equal(rotated[: D - 64], plain[: D - 64])

    def inverse(row):
        # the last 512 channels as head 0 of an identity head mix, nope 448
        o = np.zeros((1, 64, 512), np.float32)
        o[0, 0] = row[D - 512:]
        table = np.zeros((pos + 1, 64), np.float32)
        table[pos] = cs
        y = oq.vha_inv_rope_quant(o, np.eye(64, dtype=np.float32), np.array([pos]), table, 1, 448, 64,
                                  quantize=False)
        return y[0, 0, 448:]

    tol = 4e-6 * np.abs(plain[D - 64:]).max()
    assert np.abs(inverse(rotated) - plain[D - 64:]).max() <= tol

    # planted mistakes in the rotation: NeoX halves, and the opposite direction
    c, s = cs[:32], cs[32:]
    r = plain[D - 64:].copy()
    neox = np.concatenate([r[:32] * c - r[32:] * s, r[:32] * s + r[32:] * c]).astype(np.float32)
    backwards = r.copy()
    backwards[0::2] = r[0::2] * c + r[1::2] * s
    backwards[1::2] = r[1::2] * c - r[0::2] * s
    for wrong in (neox, backwards):
        row = plain.copy()
        row[D - 64:] = wrong
        assert np.abs(inverse(row) - plain[D - 64:]).max() > 100 * tol


def _fma32_exact(a, b, c):
    """Correctly rounded fp32 a*b + c by exact rational arithmetic: the
    nearest of the fp32 values around the fp64 approximation, ties to the
    even significand."""
    from fractions import Fraction

    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    r = np.float32(float(exact))
    cands = [r]
    for _ in range(2):
        cands += [np.nextafter(cands[-1], np.float32(np.inf))]
    lo = r
    for _ in range(2):
        lo = np.nextafter(lo, np.float32(-np.inf))
        cands.append(lo)
    best = min(cands, key=lambda v: (abs(Fraction(float(v)) - exact), int(np.float32(v).view(np.uint32)) & 1))
    return np.float32(best)


def test_fma32_is_correctly_rounded():
    """The oracle's fp32 fused multiply-add against exact rational rounding,
    on random operands and on products that land exactly halfway between two
    fp32 values, nudged either way by a tiny addend (where rounding the fp64
    sum would round twice and pick the even neighbour wrongly)."""
    rng = np.random.default_rng(12)
    n = 3000
    a = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    c = (rng.standard_normal(n) * 2.0 ** rng.integers(-40, 20, n)).astype(np.float32)
    cases = list(zip(a, b, c))
    for m in range(12, 24):
        x = np.float32(1.0 + 2.0 ** -m)
        for scale in (1.0, 2.0 ** -30, 2.0 ** 20):
            for tiny in (0.0, 2.0 ** -60, -(2.0 ** -60), 2.0 ** -90):
                cases.append((np.float32(x * scale), x, np.float32(tiny * scale)))
    a, b, c = (np.array(v, np.float32) for v in zip(*cases))
    got = oh.fma32(a, b, c)
    want = np.array([_fma32_exact(*t) for t in cases], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the halfway case: 1 + 2^-11 + 2^-24 is a midpoint; + 2^-60 rounds up
    x = np.float32(1.0 + 2.0 ** -12)
    assert oh.fma32(x, x, np.float32(2.0 ** -60)) == np.float32(1.0 + 2.0 ** -11 + 2.0 ** -23)
    assert oh.fma32(x, x, np.float32(0.0)) == np.float32(1.0 + 2.0 ** -11)


def test_exp_ekv_accuracy():
    x = np.linspace(-60, 0, 200001).astype(np.float32)
    np.testing.assert_allclose(oh.exp_ekv(x), np.exp(x.astype(np.float64)), rtol=5e-6)
    assert oh.exp_ekv(np.float32(0.0)) == 1.0 and oh.exp_ekv(np.float32(-200.0)) == 0.0


def _remez_exp2_rel(deg=5, iters=40):
    """Minimax relative-error polynomial P of degree ``deg`` with P(0) = 1 for
    2**f on [-1/2, 1/2], by a Remez exchange: with P(f) = 1 + f Q(f) the
    relative error is |f| 2**-f (Q(f) - g(f)) up to sign, g(f) = (2**f - 1)/f,
    so Q is the weighted minimax fit of the smooth g with weight |f| 2**-f.
    Returns (coefficients [1, q0, .., q_{deg-1}], minimax error)."""
    grid = np.linspace(-0.5, 0.5, 400001)
    grid = grid[grid != 0]
    g = np.expm1(grid * math.log(2.0)) / grid
    wt = np.abs(grid) * np.exp2(-grid)
    n = deg + 1
    x = 0.5 * np.cos(np.pi * (np.arange(n)[::-1] + 0.5) / n)
    for _ in range(iters):
        wx = np.abs(x) * np.exp2(-x)
        A = np.concatenate([wx[:, None] * x[:, None] ** np.arange(deg)[None, :],
                            -((-1.0) ** np.arange(n))[:, None]], axis=1)
        sol = np.linalg.solve(A, wx * np.expm1(x * math.log(2.0)) / x)
        q, E = sol[:deg], abs(sol[deg])
        e = wt * (np.polyval(q[::-1], grid) - g)
        # one extremum per run of equal sign, then the n largest alternating
        edges = np.flatnonzero(np.diff(np.sign(e)) != 0) + 1
        idx = np.array([s[np.argmax(np.abs(e[s]))] for s in np.split(np.arange(len(grid)), edges)])
        while len(idx) > n:
            idx = idx[1:] if abs(e[idx[0]]) < abs(e[idx[-1]]) else idx[:-1]
        x = grid[idx]
        if np.abs(e).max() <= E * (1 + 1e-9):
            break
    return np.concatenate([[1.0], q]), np.abs(e).max()


def test_exp_polynomial_is_a_near_minimax_fit():
    """Provenance of EXP_C, the compressor's degree-5 polynomial for 2**f on
    [-1/2, 1/2]: re-derive the minimax relative-error fit (with P(0) = 1) by a
    Remez exchange and bound EXP_C against it.  EXP_C is within 2x of the
    optimum in exact arithmetic (it was fit to the fp32-rounded evaluation),
    its coefficients within 1e-3 of the optimum's, and its fp32 Horner-with-FMA
    evaluation -- the kernel's -- stays below the 2.2e-7 relative error the
    oracle states."""
    coef, emin = _remez_exp2_rel()
    assert 8e-8 < emin < 1e-7  # degree 5 on a unit interval: ~9.1e-8
    f = np.linspace(-0.5, 0.5, 400001)
    c = np.array([float(v) for v in oh.EXP_C])
    assert c[0] == 1.0
    rel = np.abs(np.polyval(c[::-1], f) * np.exp2(-f) - 1.0).max()
    assert emin <= rel <= 2.0 * emin
    assert np.all(np.abs(c / coef - 1.0) < 1e-3)
    # the fp32 evaluation the kernel performs
    f32 = f.astype(np.float32)
    p = np.broadcast_to(oh.EXP_C[5], f32.shape).astype(np.float32)
    for k in range(4, -1, -1):
        p = oh.fma32(p, f32, oh.EXP_C[k])
    assert np.abs(p.astype(np.float64) / np.exp2(f32.astype(np.float64)) - 1.0).max() < 2.2e-7
    # a dropped term: the best degree-4 fit is ~12x worse than the stated bound
    c4, e4 = _remez_exp2_rel(deg=4)
    assert e4 > 10 * 2.2e-7


def test_hca_rollback_recompresses_from_latest_rows():
    """Every compressed row equals the compressor over the last-written kv_score
    rows of its 128 positions, across chunked calls and a rollback."""
    rng = np.random.default_rng(11)
    D = 512
    st = oh.HcaState(num_pages=64, dim=D, num_state=1)
    bt = np.arange(16, dtype=np.int32)[None]
    cbt = np.array([[20]], np.int32)
    ring_pages = np.array([[30, 31, 32]], np.int32)
    ape = np.zeros((128, D), np.float32)
    w = np.ones(D, np.float32)
    cs = oi.rope_cos_sin(np.arange(8) * 128, 64, 1.6e5)
    latest = {}
    for p0, n in [(0, 100), (100, 30), (130, 3), (128, 3), (131, 200), (329, 3), (327, 5)]:
        pos = np.arange(p0, p0 + n)
        lat = bf16_round(rng.standard_normal((n, D)).astype(np.float32))
        kvs = bf16_round(rng.standard_normal((n, 2 * D)).astype(np.float32))
        for p, r in zip(pos, kvs):
            latest[int(p)] = r
        slots = paged.slots_from_block_table(bt, np.zeros(n, int), pos)
        oh.hca_write(st, lat, kvs, pos, np.zeros(n, np.int32), np.array([0, n]), slots, ring_pages, 192,
                     cbt, np.array([0], np.int32), ape, w, 1e-6, cs)
    top = max(latest)
    for j in range((top + 1) // 128):
        rows = np.stack([latest[128 * j + i] for i in range(128)])
        y = oh.compress_span(rows[:, :D], rows[:, D:], ape, w, 1e-6, cs[j])
        codes, scale = quantize_rows(y[None])
        got_c, got_s = paged.read_fp8_rows(st.pool, np.array([20 * 64 + j]), D)
        assert np.array_equal(got_c, codes) and np.array_equal(got_s, scale), f"span {j}"


# ---------------------------------------------------------------- decode
def test_hca_decode_indices_brute_force():
    """hca_decode_indices / ring_slot / comp_slot against an independent
    model: every position of a sequence is replayed into a simulated ring
    whose rows are taken cyclically in append order over the slots of
    ring_pages[b] listed in order, and the compressed entries fill the slots
    of comp_block_table[b] listed in order.  A decode row is the first n_c
    compressed slots, then the rows currently holding positions p-w+1..p."""
    from oracle import hca as oh

    rng = np.random.default_rng(77)
    B, ring, width = 3, 192, 3000 // 128 + 128
    perm = rng.permutation(B * (1 + 3)).astype(np.int32)
    comp_bt = perm[:B].reshape(B, 1)
    ring_pages = perm[B:].reshape(B, 3)
    positions = np.array([0, 1, 126, 127, 128, 191, 192, 193, 383, 384, 1000, 2999], np.int64)
    for b in range(B):
        req = np.full(len(positions), b, np.int32)
        got, lens = oh.hca_decode_indices(positions, req, comp_bt, ring_pages, ring, width)
        ring_slots = [int(pg) * 64 + r for pg in ring_pages[b] for r in range(64)]
        comp_slots = [int(pg) * 64 + r for pg in comp_bt[b] for r in range(64)]
        holder, cursor, done = {}, 0, 0
        for t, p in enumerate(positions):
            while done <= p:  # append positions up to p
                holder[ring_slots[cursor]] = done
                cursor = (cursor + 1) % ring
                done += 1
            where = {pos: slot for slot, pos in holder.items()}
            n_c, w = (int(p) + 1) // 128, min(int(p) + 1, 128)
            ref = comp_slots[:n_c] + [where[q] for q in range(int(p) - w + 1, int(p) + 1)]
            assert lens[t] == len(ref)
            assert got[t, : len(ref)].tolist() == ref and np.all(got[t, len(ref):] == -1)


def test_hca_decode_rows_read_back_what_the_write_wrote():
    """Data-flow pin: after chunked writes, the window slots a decode row
    names hold exactly the quantized latent rows of positions p-w+1..p, and
    its compressed slots hold the compressed rows of spans 0..n_c-1 (the
    compressor's own output, recomputed here span by span)."""
    from oracle import hca as oh
    from oracle.fp8 import quantize_rows

    rng = np.random.default_rng(78)
    D, B, ring = 512, 2, 192
    lp, cp, rp = 8, 1, 3
    perm = rng.permutation(B * (lp + cp + rp)).astype(np.int32)
    bt = perm[: B * lp].reshape(B, lp)
    comp_bt = perm[B * lp: B * (lp + cp)].reshape(B, cp)
    ring_pages = perm[B * (lp + cp):].reshape(B, rp)
    st = oh.HcaState(len(perm), D, B)
    ape = (rng.standard_normal((128, D)) * 0.5).astype(np.float32)
    norm_w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    cos_sin = oi.rope_cos_sin(np.arange(8) * 128, 64, 1.6e5)
    state_slot = np.arange(B, dtype=np.int32)
    lat_all = {b: [] for b in range(B)}
    kvs_all = {b: [] for b in range(B)}
    pos0 = [0, 0]
    for counts in ([200, 130], [3, 3], [150, 300]):
        positions, token_seq, qsl = [], [], [0]
        for b, n in enumerate(counts):
            positions += list(range(pos0[b], pos0[b] + n))
            token_seq += [b] * n
            qsl.append(qsl[-1] + n)
        positions = np.array(positions, np.int64)
        token_seq = np.array(token_seq, np.int32)
        T = len(positions)
        latent = bf16_round(rng.standard_normal((T, D)).astype(np.float32))
        kv_score = bf16_round(rng.standard_normal((T, 2 * D)).astype(np.float32))
        slots = paged.slots_from_block_table(bt, token_seq, positions)
        oh.hca_write(st, latent, kv_score, positions, token_seq, np.array(qsl, np.int32), slots, ring_pages, ring,
                     comp_bt, state_slot, ape, norm_w, 1e-6, cos_sin)
        for t in range(T):
            lat_all[int(token_seq[t])].append(latent[t])
            kvs_all[int(token_seq[t])].append(kv_score[t])
        for b, n in enumerate(counts):
            pos0[b] += n
    for b in range(B):
        p = pos0[b] - 1
        idx, lens = oh.hca_decode_indices(np.array([p]), np.array([b], np.int32), comp_bt, ring_pages, ring, 200)
        n_c, w = (p + 1) // 128, min(p + 1, 128)
        codes, scales = paged.read_fp8_rows(st.pool, idx[0, :lens[0]], D)
        lat = np.stack(lat_all[b])
        kvs = np.stack(kvs_all[b])
        wc, ws = quantize_rows(lat[p - w + 1: p + 1])
        assert np.array_equal(codes[n_c:], wc) and np.array_equal(scales[n_c:], ws)
        for j in range(n_c):
            y = oh.compress_span(kvs[128 * j: 128 * j + 128, :D], kvs[128 * j: 128 * j + 128, D:], ape, norm_w,
                                 1e-6, cos_sin[j])
            cc, cs = quantize_rows(y[None, :])
            assert np.array_equal(codes[j], cc[0]) and scales[j] == cs[0]


def test_decode_matches_softmax_with_sink_logit():
    """Independent formulation: the sink is one more logit whose value row is 0."""
    rng = np.random.default_rng(12)
    T, H, D, n = 2, 16, 576, 50
    q = rng.standard_normal((T, H, D))
    rows = rng.standard_normal((200, D))
    idx = rng.integers(0, 200, (T, n)).astype(np.int32)
    idx[1, 10:] = -1
    sinks = rng.standard_normal(H)
    sinks[3] = -np.inf
    out, lse = od.sparse_mla_decode(q, lambda s: rows[s], idx, 0.0625, 512, sinks)
    for t in range(T):
        valid = idx[t][idx[t] >= 0]
        kv = rows[valid]
        s = q[t] @ kv.T * 0.0625
        logits = np.concatenate([s, sinks[:, None]], 1)
        p = np.exp(logits - logits.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        np.testing.assert_allclose(out[t], p[:, :-1] @ kv[:, :512], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(lse[t], np.log(np.exp(s).sum(1)), rtol=1e-12)


def test_decode_empty_row():
    out, lse = od.sparse_mla_decode(np.ones((1, 16, 576)), lambda s: None, np.full((1, 4), -1), 0.1, 512,
                                    np.zeros(16))
    assert not out.any() and np.all(np.isneginf(lse))
