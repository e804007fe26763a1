"""Post-attention fused quantization (oracle, test-only).

* ``sigmoid_mul_quant`` -- ``sigmoid_mul_quant_fp8`` of
  ``src/vllm_ernie/models/ernie5_5/nvidia/attention.py:288-361``: with bf16
  values ``x`` and ``gate``, ``s = bf16(fp32(sigmoid(gate)))`` and
  ``y = bf16(x * s)`` (the roundings of torch's ``x * torch.sigmoid(gate)``,
  ``:322``), then per 1 x 128 group the UE8M0 quant of ``:324-331``; the four
  biased exponents of a 512-column pack in the bytes of one int32 (``:333-336``).
  The fp32 sigmoid is taken correctly rounded (evaluated in fp64); torch's own
  fp32 sigmoid can sit one ulp away, which moves a bf16 result for about one
  element in 10^4-10^5 (pinned against torch in tests/test_oracle_quant.py).
* ``vha_inv_rope_quant`` -- ``vha_inv_rope_fp8_quant`` (``:166-285``): the head
  mix ``y = mix @ o`` (exact products summed in fp64, rounded once to fp32; the
  reference accumulates in fp32 in an unspecified order), the inverse rotation
  of the interleaved rope pairs ``(e, o) -> (e cos + o sin, o cos - e sin)``
  (``:211-219``) in fp32 with separate roundings, and the per-(head, 128)
  UE8M0 quant (``:221-224``).  The reference's own test pins this kernel only
  within tolerance (``test_vha_quant.py:31-78``), and so does this build.
"""

from __future__ import annotations

import numpy as np

from .fp8 import bf16_round, quantize_rows


def sigmoid_bf16(gate: np.ndarray) -> np.ndarray:
    g = np.asarray(gate, np.float64)
    return bf16_round((1.0 / (1.0 + np.exp(-g))).astype(np.float32))


def sigmoid_mul_quant(x: np.ndarray, gate: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(codes uint8 [N, hidden], packed int32 [N, hidden / 512])."""
    x = np.asarray(x, np.float32)
    n, hidden = x.shape
    y = bf16_round((x.astype(np.float64) * sigmoid_bf16(gate)).astype(np.float32))
    codes, scale = quantize_rows(y.reshape(-1, 128))
    exps = ((scale.view(np.uint32) >> 23) & 0xFF).astype(np.uint32).reshape(n, hidden // 512, 4)
    packed = (exps[..., 0] | (exps[..., 1] << 8) | (exps[..., 2] << 16) | (exps[..., 3] << 24)).view(np.int32)
    return codes.reshape(n, hidden), packed


def unpack_scales(packed: np.ndarray) -> np.ndarray:
    """``[..., P]`` packed int32 exponents -> ``[..., 4 P]`` fp32 scales
    ``2^(byte - 127)`` (the unpacking of test_vha_quant.py:16-20)."""
    u = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    exps = np.stack([(u >> (8 * k)) & 0xFF for k in range(4)], axis=-1)
    return np.exp2(exps.reshape(*u.shape[:-1], -1).astype(np.float64) - 127)


def vha_inv_rope_quant(o: np.ndarray, mix: np.ndarray, positions: np.ndarray, cos_sin: np.ndarray, n_groups: int,
                       nope_dim: int, rope_dim: int, quantize: bool = True):
    """o [T, 64, 512] and mix [64, 64] (bf16 values), cos_sin [P, >= rope_dim]
    (cos | sin).  Returns (codes uint8 [G, T, hpg * 512], exponent bytes uint8
    [G, hpg, T, 4]), or with ``quantize=False`` the fp32 rows y [T, 64, 512]
    before the quant."""
    o = np.asarray(o, np.float64)
    T, H, D = o.shape
    y = np.einsum("hg,tgd->thd", np.asarray(mix, np.float64), o).astype(np.float32)
    half = rope_dim // 2
    cs = np.asarray(cos_sin, np.float32)[np.asarray(positions, np.int64)]
    c, s = cs[:, None, :half], cs[:, None, half:rope_dim]
    ev, od = y[..., nope_dim::2].copy(), y[..., nope_dim + 1::2].copy()
    y[..., nope_dim::2] = ((ev * c).astype(np.float32) + (od * s).astype(np.float32)).astype(np.float32)
    y[..., nope_dim + 1::2] = ((od * c).astype(np.float32) - (ev * s).astype(np.float32)).astype(np.float32)
    if not quantize:
        return y
    hpg = H // n_groups
    codes, scale = quantize_rows(y.reshape(-1, 128))
    codes = codes.reshape(T, n_groups, hpg, D).transpose(1, 0, 2, 3).reshape(n_groups, T, hpg * D)
    exps = ((scale.view(np.uint32) >> 23) & 0xFF).astype(np.uint8).reshape(T, n_groups, hpg, 4).transpose(1, 2, 0, 3)
    return np.ascontiguousarray(codes), np.ascontiguousarray(exps)
