"""Pins of the post-attention quant oracle (CPU): the packed-scale unpacking
of the reference's test, torch's bf16 `x * sigmoid(gate)`, and closed forms
of the VHA mix / inverse RoPE / quant."""

import numpy as np
import torch

from oracle import indexer as oi
from oracle import quant as oq
from oracle.fp8 import bf16_round, decode_e4m3, quantize_rows


def test_unpack_matches_reference_rule():
    """``exp2(((scale >> 8k) & 0xff) - 127)`` per byte (test_vha_quant.py:16-20)."""
    packed = np.array([[0x7F7E8081, 0x01FE0000]], np.uint32).view(np.int32)
    s = oq.unpack_scales(packed)
    assert s.shape == (1, 8)
    np.testing.assert_array_equal(s[0, :4], [2.0 ** 2, 2.0 ** 1, 2.0 ** -1, 1.0])
    np.testing.assert_array_equal(s[0, 4:], [2.0 ** -127, 2.0 ** -127, 2.0 ** 127, 2.0 ** -126])


def test_sigmoid_mul_matches_torch_bf16_expression():
    """The oracle's y = bf16(x * bf16(sigmoid(g))) against torch's
    `x * torch.sigmoid(gate)` on bf16 CPU tensors: equal except where torch's
    fp32 sigmoid sits one ulp from the correctly rounded one across a bf16
    rounding boundary (rare, and then one bf16 ulp apart)."""
    rng = np.random.default_rng(0)
    x = bf16_round((rng.standard_normal((64, 8192)) * 3).astype(np.float32))
    g = bf16_round((rng.standard_normal((64, 8192)) * 4).astype(np.float32))
    xt, gt = torch.from_numpy(x).bfloat16(), torch.from_numpy(g).bfloat16()
    ref = (xt * torch.sigmoid(gt)).float().numpy()
    s = torch.sigmoid(gt).float().numpy()
    mine = bf16_round((x.astype(np.float64) * oq.sigmoid_bf16(g)).astype(np.float32))
    diff = mine != ref
    assert diff.mean() < 1e-4, diff.mean()
    ulp = np.abs(ref) * 2.0 ** -7
    assert np.all(np.abs(mine - ref)[diff] <= ulp[diff] * 1.01)
    sig_diff = oq.sigmoid_bf16(g) != s
    assert sig_diff.mean() < 1e-4


def test_sigmoid_mul_quant_groups_and_packing():
    """Each 128-group is quantize_rows of its y; pack p holds groups 4p..4p+3
    in bytes 0..3."""
    rng = np.random.default_rng(1)
    x = bf16_round((rng.standard_normal((3, 1024)) * 3).astype(np.float32))
    g = bf16_round((rng.standard_normal((3, 1024)) * 4).astype(np.float32))
    x[1, :128] = 0.0  # an all-zero group: the 1e-10 floor
    codes, packed = oq.sigmoid_mul_quant(x, g)
    y = bf16_round((x.astype(np.float64) * oq.sigmoid_bf16(g)).astype(np.float32))
    c2, s2 = quantize_rows(y.reshape(-1, 128))
    np.testing.assert_array_equal(codes.reshape(-1, 128), c2)
    np.testing.assert_array_equal(oq.unpack_scales(packed).reshape(-1), s2.astype(np.float64))
    deq = decode_e4m3(codes).astype(np.float64) * np.repeat(oq.unpack_scales(packed), 128, axis=1)
    assert np.all(np.abs(deq - y) <= np.repeat(oq.unpack_scales(packed), 128, axis=1) * 16 + 1e-30)


def test_vha_identity_mix_at_position_zero_is_plain_quant():
    """mix = I and cos = 1, sin = 0: the rows pass through unchanged, so the
    output is the per-(head, 128) quant of o itself."""
    rng = np.random.default_rng(2)
    T, H, D = 3, 64, 512
    o = bf16_round(rng.standard_normal((T, H, D)).astype(np.float32))
    cs = oi.rope_cos_sin(np.arange(8), 64, 1e4)
    codes, exps = oq.vha_inv_rope_quant(o, np.eye(H), np.zeros(T, np.int64), cs, 8, 448, 64)
    c2, s2 = quantize_rows(o.reshape(-1, 128))
    np.testing.assert_array_equal(codes.reshape(8, T, 8, 4, 128).transpose(1, 0, 2, 3, 4).reshape(-1, 128), c2)
    e2 = ((s2.view(np.uint32) >> 23) & 0xFF).reshape(T, 8, 8, 4).transpose(1, 2, 0, 3)
    np.testing.assert_array_equal(exps, e2)


def test_vha_inverse_rope_undoes_forward_rope():
    """Rotating the interleaved pairs forward by position p, then through the
    VHA path with mix = I at p, returns the rows (fp32 rounding aside); the
    nope channels are untouched."""
    rng = np.random.default_rng(3)
    T, H, D, nope = 4, 64, 512, 448
    o = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.array([0, 5, 1000, 4095])
    cs = oi.rope_cos_sin(np.arange(4096), 64, 1e4)
    c, s = cs[pos][:, None, :32].astype(np.float64), cs[pos][:, None, 32:].astype(np.float64)
    f = o.astype(np.float64).copy()
    e, od = f[..., nope::2].copy(), f[..., nope + 1::2].copy()
    f[..., nope::2] = e * c - od * s
    f[..., nope + 1::2] = e * s + od * c
    y = oq.vha_inv_rope_quant(f.astype(np.float32), np.eye(H), pos, cs, 8, nope, 64, quantize=False)
    np.testing.assert_allclose(y, o, rtol=0, atol=1e-5)
    np.testing.assert_array_equal(y[..., :nope], f.astype(np.float32)[..., :nope])
