"""MXFP4 lightning-indexer keys (oracle; test infrastructure only).

Reference call sites (``src/vllm_ernie/models/ernie5_5/nvidia/attention.py``):

* ``_quantize_fp4`` -- ``:986-1025``: q and k rows (128 values, after the
  Hadamard) go through ``downcast_to_mxfp(x, axis=-1, BLOCK_QUANT_DIM=128)``;
  q comes back as ``values [T, 64, 64]`` uint8 and ``scales [T, 64]`` (four
  UE8M0 bytes viewed as one int32, ``:1024-1025``);
* the weights are not folded with any q scale on this path:
  ``w = fl32(weights * 128**-0.5 * 64**-0.5)`` (``:970-974``);
* ``_store_indexer_fp4`` -- ``:831-860``: row of slot ``s`` goes to page
  ``s // 64``; its 64 packed bytes at ``page_base + (s % 64) * 64``, its four
  scale bytes at ``page_base + 64 * 64 + (s % 64) * 4``; negative slots are
  skipped.  Pinned by the known-answer test ``test_indexer_fp4.py:71-90``
  (two rows into a 9216-byte page filled with 173).
* row bytes ``128 / 2 + 128 / 32 = 68`` (``:929-935``).

Quantization (``downcast_to_mxfp`` lives in triton_kernels, an upstream
dependency of vLLM 0.32.0 that is not in this container; restated from its
published algorithm, DequantScaleRoundingMode.ROUND_UP):

1. per group of 32 values: ``amax = max |x|`` (fp32);
2. ``scale = 2**ceil(log2(amax / 6))`` -- the fp32 quotient ``amax / 6``
   rounded up to a power of two by adding ``0x7FFFFF`` to its bits and
   keeping the exponent field; stored as the E8M0 byte (the exponent field,
   ``0`` when ``amax == 0``);
3. ``y = x * (1 / scale)`` (exact: a power of two), ``|y| <= 6``;
4. ``y`` to e2m1 (values 0, 0.5, 1, 1.5, 2, 3, 4, 6) by nearest, with a tie
   going to the larger magnitude (the upstream bit recipe adds one below the
   kept bits and shifts; 0.25, 1.25, 2.5 and 5 therefore go up, where
   round-to-nearest-even would go down); the sign bit is kept, so a small
   negative value becomes code 8 (-0);
5. two codes per byte, the even element in the low nibble.

Parity: the layout is pinned by the reference KAT; the e2m1 encoding off
ties is pinned by ``triton.tools.mxfp.MXFP4Tensor`` (round-to-nearest-even);
the scale by its closed form; the tie rule and the fp32 quotient (upstream
Triton's ``/`` may be the approximate division, which could move the scale
of a group whose amax is exactly ``6 * 2**k``) are **parity unpinned**
against upstream.

Exact scoring contract (mirrored bit for bit by the HIP kernels): with
``Iq, Ik`` the integers ``2 * e2m1 value`` (|I| <= 12) and ``sq, sk`` the
E8M0 bytes of block ``b`` (32 dims),

1. ``D_b = sum_{d in b} Iq[h, d] * Ik[s, d]`` exactly;
2. ``T_b = fl32(D_b * 2**(sq[h, b] + sk[s, b] - 256))``;
3. ``dot = fl32(fl32(fl32(T_0 + T_1) + T_2) + T_3)``;
4. ``p_h = fl32(w[t, h] * max(dot, 0))``, heads summed in the fixed order of
   ``oracle.indexer.head_sum_pinned``; ``score = acc + 0.0``.
Upstream's DeepGEMM FP4 logits kernel is not available; its accumulation
order is unpinned.
"""

from __future__ import annotations

import numpy as np

from .indexer import INDEX_HEAD_DIM, WEIGHTS_SCALE, head_sum_pinned, topk_ascending
from .paged import PAGE_TOKENS

MXFP4_BLOCK = 32  # values per E8M0 scale
FP4_VALUE_BYTES = INDEX_HEAD_DIM // 2  # 64
FP4_SCALE_BYTES = INDEX_HEAD_DIM // MXFP4_BLOCK  # 4
FP4_ROW_BYTES = FP4_VALUE_BYTES + FP4_SCALE_BYTES  # 68
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)


def e2m1_encode(y: np.ndarray) -> np.ndarray:
    """fp32 ``y`` (|y| <= 6 expected) -> e2m1 codes (uint8, one per value),
    by the upstream bit recipe (nearest, ties to the larger magnitude,
    saturating at 6)."""
    u = np.asarray(y, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (u >> 31) & 1
    e = (u >> 23) & 0xFF
    m = u & 0x7FFFFF
    adj = 126 - e  # right shift that aligns a value below 1 to the e2m1 subnormal
    sub = (0x400000 | (m >> 1)) >> np.clip(adj, 0, 63)
    m2 = np.where(e < 127, np.where(adj < 32, sub, 0), m)
    e2 = np.maximum(e, 126) - 126
    code = np.minimum((((e2 << 2) | (m2 >> 21)) + 1) >> 1, 7)
    return ((sign << 3) | code).astype(np.uint8)


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    """e2m1 codes (low nibble) -> fp32 values."""
    c = np.asarray(codes, dtype=np.uint8)
    v = E2M1_VALUES[c & 7]
    return np.where(c & 8, -v, v).astype(np.float32)


def scale_bytes(amax: np.ndarray) -> np.ndarray:
    """E8M0 byte of each group's ``amax`` (fp32): the exponent field of
    ``amax / 6`` rounded up to a power of two."""
    q = (np.asarray(amax, dtype=np.float32) / np.float32(6.0)).astype(np.float32)
    bits = q.view(np.uint32).astype(np.uint64)
    return (((bits + 0x7FFFFF) & 0x7F800000) >> 23).astype(np.uint8)


def quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``x [..., D]`` (D a multiple of 32; any float dtype, taken as fp32) ->
    ``(values uint8 [..., D/2], scales uint8 [..., D/32])``."""
    xf = np.asarray(x, dtype=np.float32)
    D = xf.shape[-1]
    assert D % MXFP4_BLOCK == 0
    g = xf.reshape(*xf.shape[:-1], D // MXFP4_BLOCK, MXFP4_BLOCK)
    amax = np.max(np.abs(g), axis=-1)
    sb = scale_bytes(amax)
    scale = (sb.astype(np.uint32) << 23).view(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(scale == 0, np.float32(0.0), np.float32(1.0) / scale).astype(np.float32)
    y = (g * inv[..., None]).astype(np.float32)
    codes = e2m1_encode(y).reshape(*xf.shape[:-1], D)
    values = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    return values, sb


def unpack(values: np.ndarray) -> np.ndarray:
    """Packed bytes ``[..., D/2]`` -> codes ``[..., D]`` (even element low)."""
    v = np.asarray(values, dtype=np.uint8)
    out = np.empty(v.shape[:-1] + (2 * v.shape[-1],), dtype=np.uint8)
    out[..., 0::2] = v & 0xF
    out[..., 1::2] = v >> 4
    return out


def dequantize(values: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Packed values and E8M0 bytes -> fp32 ``[..., D]`` (float64 for the
    power of two, so scale bytes 0 and 255 stay finite here)."""
    c = unpack(values)
    D = c.shape[-1]
    v = e2m1_decode(c).astype(np.float64).reshape(*c.shape[:-1], D // MXFP4_BLOCK, MXFP4_BLOCK)
    p = np.ldexp(1.0, np.asarray(scales, dtype=np.int64) - 127)
    return (v * p[..., None]).reshape(*c.shape[:-1], D)


def int2(values: np.ndarray) -> np.ndarray:
    """Packed values -> the exact integers ``2 * e2m1 value`` (int64)."""
    return np.rint(2.0 * e2m1_decode(unpack(values))).astype(np.int64)


def quantize_q(q: np.ndarray, weights: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``q [T, 64, 128]``, ``weights [T, 64]`` -> ``(values [T, 64, 64],
    scales uint8 [T, 64, 4], w fp32 [T, 64])``; ``w = fl32(weights * WS)``
    (``attention.py:970-974``)."""
    values, scales = quantize(q)
    w = (np.asarray(weights, dtype=np.float32) * WEIGHTS_SCALE).astype(np.float32)
    return values, scales, w


def page_bytes() -> int:
    return PAGE_TOKENS * FP4_ROW_BYTES


def store(kcache: np.ndarray, values: np.ndarray, scales: np.ndarray, slots: np.ndarray) -> None:
    """``_store_indexer_fp4`` (``attention.py:831-860``) on ``kcache [pages,
    stride]`` uint8: rows applied in order, negative slots skipped."""
    flat = kcache.reshape(kcache.shape[0], -1)
    for r, s in enumerate(np.asarray(slots, dtype=np.int64)):
        if s < 0:
            continue
        page, off = int(s) // PAGE_TOKENS, int(s) % PAGE_TOKENS
        flat[page, off * FP4_VALUE_BYTES:(off + 1) * FP4_VALUE_BYTES] = values[r]
        base = PAGE_TOKENS * FP4_VALUE_BYTES + off * FP4_SCALE_BYTES
        flat[page, base:base + FP4_SCALE_BYTES] = scales[r]


def k_insert(kcache: np.ndarray, k: np.ndarray, slots: np.ndarray) -> None:
    """Quantize ``k [T, 128]`` and store it by slot (``attention.py:1001-1021``)."""
    values, scales = quantize(k)
    store(kcache, values, scales, slots)


def read_rows(kcache: np.ndarray, slots: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``(values [S, 64], scales [S, 4])`` of the given slots."""
    flat = kcache.reshape(kcache.shape[0], -1)
    s = np.asarray(slots, dtype=np.int64)
    page, off = s // PAGE_TOKENS, s % PAGE_TOKENS
    vidx = (off * FP4_VALUE_BYTES)[:, None] + np.arange(FP4_VALUE_BYTES)[None, :]
    sidx = (PAGE_TOKENS * FP4_VALUE_BYTES + off * FP4_SCALE_BYTES)[:, None] + np.arange(FP4_SCALE_BYTES)[None, :]
    return flat[page[:, None], vidx], flat[page[:, None], sidx]


def exact_scores(q_values: np.ndarray, q_scales: np.ndarray, w: np.ndarray, k_values: np.ndarray,
                 k_scales: np.ndarray) -> np.ndarray:
    """Scores of one query row (``q_values [64, 64]``, ``q_scales [64, 4]``,
    ``w [64]``) against keys ``k_values [S, 64]``, ``k_scales [S, 4]``."""
    iq = int2(q_values).reshape(-1, 4, MXFP4_BLOCK).astype(np.float64)  # [64, 4, 32]
    ik = int2(k_values).reshape(-1, 4, MXFP4_BLOCK).astype(np.float64)  # [S, 4, 32]
    # block dot products: integers below 2**13, exact in float64 matmuls
    d = np.stack([ik[:, b, :] @ iq[:, b, :].T for b in range(4)], axis=-1)  # [S, 64, 4]
    e = (np.asarray(k_scales, np.int64)[:, None, :] + np.asarray(q_scales, np.int64)[None, :, :] - 256)
    with np.errstate(over="ignore"):
        tb = np.ldexp(d, e).astype(np.float32)
        dot = (tb[..., 0] + tb[..., 1]).astype(np.float32)
        dot = (dot + tb[..., 2]).astype(np.float32)
        dot = (dot + tb[..., 3]).astype(np.float32)
    r = np.maximum(dot, np.float32(0.0))
    p = (np.asarray(w, np.float32)[None, :] * r).astype(np.float32)
    return (head_sum_pinned(p) + np.float32(0.0)).astype(np.float32)


def indexer_topk(q_values: np.ndarray, q_scales: np.ndarray, w: np.ndarray, kcache: np.ndarray,
                 block_table: np.ndarray, req_ids: np.ndarray, lengths: np.ndarray,
                 k: int) -> tuple[np.ndarray, list[np.ndarray]]:
    """Per query row t: exact scores over ``s < lengths[t]`` of request
    ``req_ids[t]`` and the top-k.  Returns ``(topk [T, k], scores per row)``."""
    T = q_values.shape[0]
    out = np.full((T, k), -1, dtype=np.int32)
    all_scores = []
    for t in range(T):
        n = int(lengths[t])
        s = np.arange(n, dtype=np.int64)
        bt = np.asarray(block_table, dtype=np.int64)[int(req_ids[t])]
        slots = bt[s // PAGE_TOKENS] * PAGE_TOKENS + s % PAGE_TOKENS
        kv, ks = read_rows(kcache, slots)
        sc = exact_scores(q_values[t], q_scales[t], w[t], kv, ks)
        all_scores.append(sc)
        out[t] = topk_ascending(sc, k)
    return out, all_scores
