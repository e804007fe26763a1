"""OCP fp8 e4m3fn codec and the UE8M0 per-token scale rule (oracle, test-only).

Reference rule (``src/vllm_ernie/models/ernie5_5/nvidia/attention.py:221-227``
and ``:317-319``)::

    amax  = max(max|x|, 1e-10)
    scale = exp2(ceil(log2(amax * (1/448))))
    q     = clamp(x / scale, -448, 448).to(float8_e4m3fn)

and the UE8M0 byte is ``exponent + 127`` (``attention.py:326``;
``tests/models/ernie5_5/test_vha_quant.py:16-20`` unpacks it as
``2**(byte - 127)``).

Two choices are fixed here and mirrored bit for bit by the HIP kernels:

* ``r = fl32(amax * fl32(1/448))`` is formed in fp32, as the Triton kernels do
  (a constexpr float times an fp32 tensor), and ``ceil(log2(r))`` is taken
  *exactly* from r's binary exponent, not from an approximate ``log2``;
* the cast rounds to nearest, ties to even, after the clamp (torch's own cast
  does not saturate, so the clamp comes first, ``attention.py:224``).

``encode_e4m3`` is pinned against ``torch.Tensor.to(torch.float8_e4m3fn)`` and
the decode table against the e4m3fn definition in ``tests/test_oracle_fp8.py``.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
AMAX_FLOOR = np.float32(1e-10)
INV_E4M3_MAX = np.float32(1.0 / 448.0)


def decode_table() -> np.ndarray:
    """float32 value of each of the 256 e4m3fn codes (NaN for 0x7f/0xff)."""
    codes = np.arange(256, dtype=np.int64)
    sign = np.where(codes >> 7, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = codes & 0x7
    mag = np.where(exp == 0, man * 2.0**-9, (8 + man) * np.exp2(exp - 10.0))
    val = sign * mag
    val[(exp == 15) & (man == 7)] = np.nan
    return val.astype(np.float32)


_DECODE = decode_table()


def decode_e4m3(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values."""
    return _DECODE[np.asarray(codes, dtype=np.uint8)]


def encode_e4m3(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn codes, round to nearest even; requires |x| <= 448."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    if np.any(~(a <= E4M3_MAX)):
        raise ValueError("encode_e4m3 expects finite inputs clamped to +-448")
    sign = (x.view(np.uint32) >> 31).astype(np.uint8) << 7
    frac, ex = np.frexp(a)  # a = frac * 2**ex, frac in [0.5, 1)
    e = ex.astype(np.int64) - 1  # a = (2*frac) * 2**e
    normal = a >= 2.0**-6
    m8 = np.rint((2.0 * frac - 1.0) * 8.0)  # 3-bit mantissa, ties to even
    carry = m8 >= 8.0
    e = np.where(carry, e + 1, e)
    m8 = np.where(carry, 0.0, m8)
    code_n = ((e + 7) << 3) | m8.astype(np.int64)
    code_s = np.rint(a * 512.0).astype(np.int64)  # multiples of 2**-9; 8 -> 0x08
    code = np.where(normal, code_n, code_s)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def ue8m0_exponent(amax: np.ndarray) -> np.ndarray:
    """Exponent e of the power-of-two scale 2**e for each amax (int32)."""
    amax = np.maximum(np.asarray(amax, dtype=np.float32), AMAX_FLOOR)
    r = (amax * INV_E4M3_MAX).astype(np.float32)
    frac, ex = np.frexp(r.astype(np.float64))
    e = np.where(frac == 0.5, ex - 1, ex)
    return e.astype(np.int32)


def quantize_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row UE8M0 fp8 quant of ``x [..., D]`` (any float dtype).

    Returns ``(codes uint8 [..., D], scale float32 [...])`` where scale is the
    power of two ``2**e`` stored as fp32.
    """
    xf = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(xf), axis=-1)
    e = ue8m0_exponent(amax)
    scale = np.ldexp(np.float32(1.0), e).astype(np.float32)
    y = xf * np.ldexp(np.float32(1.0), -e)[..., None].astype(np.float32)
    y = np.clip(y, -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return encode_e4m3(y), scale


def dequantize_rows(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Inverse of ``quantize_rows`` up to the fp8 rounding: float32 rows."""
    return (decode_e4m3(codes) * np.asarray(scale, np.float32)[..., None]).astype(
        np.float32
    )


def ue8m0_byte(scale: np.ndarray) -> np.ndarray:
    """UE8M0 byte ``exponent + 127`` of a power-of-two fp32 scale."""
    bits = np.asarray(scale, dtype=np.float32).view(np.uint32)
    return ((bits >> 23) & 0xFF).astype(np.uint8)


def ue8m0_unpack(byte: np.ndarray) -> np.ndarray:
    """``2**(byte - 127)`` as float32 (``test_vha_quant.py:16-20``)."""
    return np.exp2(np.asarray(byte, dtype=np.float64) - 127.0).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even); float32 result."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return rounded.astype(np.uint32).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), ties to even."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32."""
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)
