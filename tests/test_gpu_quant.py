"""GPU parity of the post-attention fused quant kernels against the oracle:
sigmoid_mul_quant_fp8 bit-exact (codes and packed scales; the reference pins
its kernel bitwise against the unfused path, test_vha_quant.py:82-102), and
vha_inv_rope_fp8_quant within the reference's own criteria
(test_vha_quant.py:31-78): the head mix's fp32 accumulation order is the
kernel's, so a scale exponent at a power-of-two boundary or one fp8 step may
differ; the fused result is at least as close to the fp32 mix as the unfused
bf16 path."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, randn_bf16, to_dev
from oracle import indexer as oi
from oracle import quant as oq
from oracle.fp8 import bf16_round, decode_e4m3, quantize_rows

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hidden", [8192, 16384])
@pytest.mark.parametrize("num_rows", [1, 5, 1000])
def test_sigmoid_mul_quant_exact(dev, num_rows, hidden):
    from ernie_kv import attention as A
    from ernie_kv import ops

    rng = np.random.default_rng(num_rows + hidden)
    x = randn_bf16(rng, (num_rows, hidden), 3.0)
    g = randn_bf16(rng, (num_rows, hidden), 4.0)
    x[0, :128] = 0.0  # a zero group (the 1e-10 floor)
    q, s = A.sigmoid_mul_quant_fp8(bf16_tensor(x, dev), bf16_tensor(g, dev))
    aligned = ops.tma_aligned_rows(num_rows)
    assert q.dtype == torch.float8_e4m3fn and q.shape == (num_rows, hidden)
    assert s.shape == (num_rows, hidden // 512) and s.stride() == (1, aligned)
    codes, packed = oq.sigmoid_mul_quant(x, g)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), codes)
    assert np.array_equal(s.cpu().numpy(), packed)


@pytest.mark.parametrize("num_tokens", [1, 7, 300])
def test_vha_inv_rope_fp8_quant(dev, num_tokens):
    from ernie_kv import attention as A

    rng = np.random.default_rng(num_tokens)
    heads, groups, head_dim, rope_dim, rank = 64, 8, 512, 64, 16
    nope = head_dim - rope_dim
    o_padded = randn_bf16(rng, (num_tokens, 128, head_dim))  # the FlashMLA output buffer's padded head axis
    o = o_padded[:, :heads]
    u = rng.standard_normal((heads, rank)) / 8
    v = rng.standard_normal((heads, rank)) / 8
    mix = bf16_round((np.eye(heads) + v @ u.T).astype(np.float32))
    positions = rng.integers(0, 4096, num_tokens).astype(np.int64)
    cs = oi.rope_cos_sin(np.arange(4096), rope_dim, 1e4)
    o_t = bf16_tensor(o_padded, dev)[:, :heads]
    got = A.vha_inv_rope_fp8_quant(o_t, bf16_tensor(mix, dev), to_dev(positions, dev), to_dev(cs, dev), groups, nope,
                                   rope_dim)
    hpg = heads // groups
    assert got.data.shape == (num_tokens, groups, hpg * head_dim) and got.scale.shape == (num_tokens, groups, hpg)
    codes = got.data.view(torch.uint8).transpose(0, 1).contiguous().cpu().numpy()  # [G, T, hpg * 512]
    sc = got.scale.contiguous().cpu().numpy()  # [T, G, hpg] int32
    exps = np.stack([(sc.astype(np.int64) >> (8 * c)) & 0xFF for c in range(4)], -1).astype(np.uint8)
    exps = exps.transpose(1, 2, 0, 3)  # [G, hpg, T, 4]
    ref_codes, ref_exps = oq.vha_inv_rope_quant(o, mix, positions, cs, groups, nope, rope_dim)
    assert (exps != ref_exps).mean() < 0.01, f"scale exponents differ on {(exps != ref_exps).mean():.4f}"

    def dequant(cd, ex):  # -> [T, 64, 512]
        v = decode_e4m3(cd).astype(np.float64).reshape(groups, num_tokens, hpg, 4, 128)
        s = np.exp2(ex.astype(np.float64) - 127).transpose(0, 2, 1, 3)[..., None]  # [G, T, hpg, 4, 1]
        return (v * s).transpose(1, 0, 2, 3, 4).reshape(num_tokens, heads, head_dim)

    d_got, d_ref = dequant(codes, exps), dequant(ref_codes, ref_exps)
    # where the scale agrees, codes are at most one fp8 step apart: 2^-3 of
    # the value (3 mantissa bits), or the subnormal step scale * 2^-9
    same = (exps == ref_exps).transpose(2, 0, 1, 3).reshape(num_tokens, heads, 4).repeat(128, -1)
    ref_scale = np.exp2(ref_exps.astype(np.float64) - 127).transpose(2, 0, 1, 3).reshape(num_tokens, heads, 4)
    step = np.maximum(np.abs(d_ref) * 2.0 ** -3, ref_scale.repeat(128, -1) * 2.0 ** -9)
    assert np.all(np.abs(d_got - d_ref)[same] <= step[same] * 1.001), "codes more than one fp8 step apart"
    assert np.linalg.norm(d_got - d_ref) / np.linalg.norm(d_ref) < 0.03
    exact = oq.vha_inv_rope_quant(o, mix, positions, cs, groups, nope, rope_dim, quantize=False)
    y16 = bf16_round(np.einsum("hg,tgd->thd", mix.astype(np.float64), o.astype(np.float64)).astype(np.float32))
    unf_c, unf_e = oq.vha_inv_rope_quant(y16, np.eye(heads), positions, cs, groups, nope, rope_dim)
    err = np.linalg.norm(d_got - exact) / np.linalg.norm(exact)
    err_unfused = np.linalg.norm(dequant(unf_c, unf_e) - exact) / np.linalg.norm(exact)
    assert err <= err_unfused * 1.05, (err, err_unfused)
    # the scale buffer's padding rows are zero
    aligned = (num_tokens + 3) // 4 * 4
    full = torch.empty(0, dtype=torch.int32, device=dev).set_(got.scale.untyped_storage()).view(groups, hpg, aligned)
    assert (full[..., num_tokens:] == 0).all()
