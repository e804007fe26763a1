"""Lightning-indexer path: prep, K insert, exact scoring, exact top-k (oracle).

Reference call sites (``src/vllm_ernie/models/ernie5_5/nvidia/attention.py``):

* ``hadamard_rows`` -- ``:102-108`` (orthonormal Sylvester Walsh-Hadamard per
  128-wide row; pinned by ``test_dsa_backend.py:73-89``);
* partial NeoX RoPE on dims 0..63 of each 128-d head -- ``:913-922, 965``
  (pinned structurally by ``test_indexer_rope.py:14-48``);
* q quant with a per-(token, head) UE8M0 scale folded into the head weights,
  ``weights * q_scale * 128**-0.5 * 64**-0.5`` -- ``:925, 976-980``;
* K insert: 128 fp8 + fp32 scale per token, values-then-scales pages --
  ``:929-935, 942-953`` (byte parity with upstream DeepGEMM pages unpinned);
* scoring ``score[t, s] = sum_h w[t, h] * relu(q[t, h] . k[s])`` over
  ``s < pos + 1 - window`` -- ``:644-691, 982-984`` (windowed lengths);
* top-k with the lowest-index tie-break -- ``:942-953`` (upstream tie-break is
  unspecified; the build contract is lowest index first).

Exact scoring contract (mirrored bit for bit by the HIP kernels):

1. ``D = sum_d Iq[h, d] * Ik[s, d]`` exactly, where ``I = fp8 value * 2**9`` is
   an integer (|I| < 2**18), so D is an exact int64;
2. ``dot = fl32(D * 2**-18)`` -- one rounding;
3. ``p_h = fl32(w[t, h] * max(dot, 0))``;
4. heads summed in fp32 in the kernel's fixed order: lane group
   ``g = 0..3`` adds ``p[16*hb + 4*g + i]`` for ``hb = 0..3, i = 0..3`` starting
   from +0, then ``(acc0 + acc1) + (acc2 + acc3)``;
5. ``score = fl32(acc * kscale[s]) + 0.0`` (the + 0 turns -0 into +0).

Selection orders candidates by (score descending, index ascending) and writes
the chosen indices in ascending order, padded with -1.
"""

from __future__ import annotations

import math

import numpy as np

from .fp8 import bf16_round, decode_e4m3, quantize_rows
from .paged import PAGE_TOKENS, fp8_page_bytes, read_fp8_rows, write_fp8_rows

INDEX_HEAD_DIM = 128
INDEX_N_HEADS = 64
INDEXER_QUANT_BLOCK = 128  # attention.py:99


def hadamard_matrix(n: int = 128) -> np.ndarray:
    """Sylvester Hadamard matrix (unnormalized), as built in test_dsa_backend.py:82-85."""
    h = np.ones((1, 1), dtype=np.float64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def hadamard_rows(x: np.ndarray) -> np.ndarray:
    """FWHT of each 128-wide row in fp32, times fl32(128**-0.5), rounded to bf16.

    Butterfly order: spans h = 1, 2, 4, ..., 64; ``(a, b) -> (a + b, a - b)``.
    Returns float32 values that are exactly bf16-representable.
    """
    y = np.asarray(x, dtype=np.float32).copy()
    n = y.shape[-1]
    h = 1
    while h < n:
        y = y.reshape(*y.shape[:-1], n // (2 * h), 2, h)
        a = y[..., 0, :].copy()
        b = y[..., 1, :].copy()
        y[..., 0, :] = (a + b).astype(np.float32)
        y[..., 1, :] = (a - b).astype(np.float32)
        y = y.reshape(*y.shape[:-3], n)
        h *= 2
    return bf16_round((y * np.float32(1.0 / math.sqrt(n))).astype(np.float32))


def rope_cos_sin(positions: np.ndarray, rot_dim: int, theta: float) -> np.ndarray:
    """fp32 ``[len(positions), rot_dim]`` table: cos of the rot_dim/2 freqs, then sin.

    ``inv_freq_i = theta ** (-2i / rot_dim)``, angles in fp64, rounded to fp32.
    """
    half = rot_dim // 2
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / rot_dim)
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


def yarn_cos_sin(positions: np.ndarray, rot_dim: int, theta: float, factor: float = 16.0,
                 original_max_position: int = 4096, beta_fast: float = 32.0, beta_slow: float = 1.0) -> np.ndarray:
    """YaRN cos | sin table (Peng et al., "YaRN: Efficient Context Window
    Extension of Large Language Models", 2023): per frequency, a linear ramp
    between the original (extrapolated) and the 1/factor (interpolated) inverse
    frequency over the dims whose wavelengths lie between the ones that turn
    beta_fast and beta_slow times in the original context, and the attention
    factor mscale = 0.1 ln(factor) + 1 multiplied into cos and sin.

    The HCA layers' RoPE is YaRN at ``compress_rope_theta``
    (src/vllm_ernie/models/ernie5_5/config.py:187-188); its parameters come
    from the checkpoint's ``rope_scaling``, so the ones here are
    representative.  The table is an input of the compressor (cos_sin), not
    computed by the path itself."""
    half = rot_dim // 2
    inv_extra = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / rot_dim)
    inv_inter = inv_extra / factor

    def corr_dim(turns):
        return rot_dim * math.log(original_max_position / (turns * 2 * math.pi)) / (2 * math.log(theta))

    low = max(math.floor(corr_dim(beta_fast)), 0)
    high = min(math.ceil(corr_dim(beta_slow)), rot_dim - 1)
    ramp = np.clip((np.arange(half, dtype=np.float64) - low) / max(high - low, 1e-3), 0.0, 1.0)
    inv = inv_inter * ramp + inv_extra * (1.0 - ramp)
    mscale = 0.1 * math.log(factor) + 1.0
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv[None, :]
    return (np.concatenate([np.cos(ang), np.sin(ang)], axis=-1) * mscale).astype(np.float32)


def neox_partial_rope(x: np.ndarray, cos_sin: np.ndarray, rot_dim: int) -> np.ndarray:
    """NeoX rotation of dims ``[0, rot_dim)`` of the last axis; the rest untouched.

    ``x [..., D]`` bf16 values (float32 container), ``cos_sin [..., rot_dim]``
    broadcast over the leading axes.  Each output is
    ``bf16(fl32(x1*c) - fl32(x2*s))`` / ``bf16(fl32(x2*c) + fl32(x1*s))``.
    """
    x = np.asarray(x, dtype=np.float32)
    half = rot_dim // 2
    c = cos_sin[..., :half].astype(np.float32)
    s = cos_sin[..., half:rot_dim].astype(np.float32)
    x1 = x[..., :half]
    x2 = x[..., half:rot_dim]
    o1 = ((x1 * c).astype(np.float32) - (x2 * s).astype(np.float32)).astype(np.float32)
    o2 = ((x2 * c).astype(np.float32) + (x1 * s).astype(np.float32)).astype(np.float32)
    out = x.copy()
    out[..., :half] = bf16_round(o1)
    out[..., half:rot_dim] = bf16_round(o2)
    return out


def _chunk_tree_sum(v: np.ndarray) -> np.ndarray:
    """Sum of each 128-wide row in the kernel's fp32 order: per 8-element
    chunk ((v0+v1)+(v2+v3))+((v4+v5)+(v6+v7)), then a butterfly over the 16
    chunks (partners at distance 1, 2, 4, 8), which leaves every chunk with
    the same balanced-tree total."""
    f32 = np.float32
    c = v.reshape(*v.shape[:-1], 16, 8).astype(f32)
    p = [(c[..., 2 * i] + c[..., 2 * i + 1]).astype(f32) for i in range(4)]
    s = (((p[0] + p[1]).astype(f32)) + ((p[2] + p[3]).astype(f32))).astype(f32)
    idx = np.arange(16)
    for off in (1, 2, 4, 8):
        s = (s + s[..., idx ^ off]).astype(f32)
    return s[..., 0]


def layer_norm_rows(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    """LayerNorm of each 128-wide row (the indexer's ``k_norm``,
    nvidia/attention.py:912, 962), in fp32 with the sums in
    ``_chunk_tree_sum``'s order::

        mean = fl32(S(x) / 128);  d = fl32(x - mean);  var = fl32(S(fl32(d*d)) / 128)
        rstd = fl32(1 / sqrt_rn(fl32(var + eps)));  y = bf16(fl32(fl32(fl32(d * rstd) * w) + b))

    Returns float32 values that are exactly bf16-representable."""
    f32 = np.float32
    x = np.asarray(x, f32)
    n = f32(x.shape[-1])
    mean = (_chunk_tree_sum(x) / n).astype(f32)
    d = (x - mean[..., None]).astype(f32)
    var = (_chunk_tree_sum((d * d).astype(f32)) / n).astype(f32)
    rstd = (f32(1.0) / np.sqrt((var + f32(eps)).astype(f32))).astype(f32)
    y = ((((d * rstd[..., None]).astype(f32)) * np.asarray(w, f32)).astype(f32) + np.asarray(b, f32)).astype(f32)
    return bf16_round(y)


def indexer_prep(q: np.ndarray, k: np.ndarray, ln_w: np.ndarray, ln_b: np.ndarray, eps: float,
                 cos_sin: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``Ernie5_5Indexer.forward`` up to the quantization (nvidia/attention.py:
    955-969): ``k = hadamard(rope(k_norm(k)))``, ``q = hadamard(rope(q))``, the
    NeoX rotation on dims 0..63.  ``q [T, 64, 128]``, ``k [T, 128]`` bf16 values,
    ``cos_sin [T, 64]`` (the rows of the tokens' positions)."""
    cs = np.asarray(cos_sin, np.float32)
    k1 = neox_partial_rope(layer_norm_rows(k, ln_w, ln_b, eps), cs, 64)
    q1 = neox_partial_rope(np.asarray(q, np.float32), cs[:, None, :], 64)
    return hadamard_rows(q1), hadamard_rows(k1)


WEIGHTS_SCALE = np.float32(INDEX_HEAD_DIM**-0.5 * INDEX_N_HEADS**-0.5)  # attention.py:925


def quantize_q(q: np.ndarray, weights: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``q [T, H, 128]`` -> fp8 codes with per-(t, h) UE8M0 scales folded into weights.

    Returns ``(q_codes uint8 [T, H, 128], w_folded f32 [T, H])`` with
    ``w_folded = fl32(fl32(w * q_scale) * WEIGHTS_SCALE)`` (``attention.py:980``).
    """
    codes, qscale = quantize_rows(q)
    w = np.asarray(weights, dtype=np.float32)
    folded = ((w * qscale).astype(np.float32) * WEIGHTS_SCALE).astype(np.float32)
    return codes, folded


def k_insert(kcache: np.ndarray, k: np.ndarray, slots: np.ndarray) -> None:
    """Quantize ``k [T, 128]`` per token and scatter into the indexer K pages."""
    codes, scale = quantize_rows(k)
    write_fp8_rows(kcache, slots, codes, scale, INDEX_HEAD_DIM)


def int_repr(codes: np.ndarray) -> np.ndarray:
    """Exact integer ``fp8 value * 2**9`` of each code (int64)."""
    v = decode_e4m3(codes).astype(np.float64)
    return np.rint(np.nan_to_num(v) * 512.0).astype(np.int64)


def head_sum_pinned(p: np.ndarray) -> np.ndarray:
    """Sum ``p [..., 64]`` over heads in the scoring kernel's fp32 order."""
    p = np.asarray(p, dtype=np.float32)
    accs = []
    for g in range(4):
        acc = np.zeros(p.shape[:-1], dtype=np.float32)
        for hb in range(4):
            for i in range(4):
                acc = (acc + p[..., 16 * hb + 4 * g + i]).astype(np.float32)
        accs.append(acc)
    a01 = (accs[0] + accs[1]).astype(np.float32)
    a23 = (accs[2] + accs[3]).astype(np.float32)
    return (a01 + a23).astype(np.float32)


def exact_scores(
    q_codes: np.ndarray, w: np.ndarray, k_codes: np.ndarray, k_scale: np.ndarray
) -> np.ndarray:
    """Scores of one query row ``q_codes [64, 128]`` against ``k_codes [S, 128]``."""
    iq = int_repr(q_codes)  # [64, 128]
    ik = int_repr(k_codes)  # [S, 128]
    d = ik @ iq.T  # [S, 64] exact int64
    dot = (d.astype(np.float64) * 2.0**-18).astype(np.float32)
    r = np.maximum(dot, np.float32(0.0))
    p = (np.asarray(w, np.float32)[None, :] * r).astype(np.float32)
    acc = head_sum_pinned(p)
    s = (acc * np.asarray(k_scale, np.float32)).astype(np.float32)
    return (s + np.float32(0.0)).astype(np.float32)


def score_keys(scores: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 keys of fp32 scores (larger score -> larger key)."""
    u = np.asarray(scores, dtype=np.float32).view(np.uint32)
    return np.where(u >> 31, ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def topk_ascending(scores: np.ndarray, k: int) -> np.ndarray:
    """Top-k indices by (score desc, index asc), returned ascending, -1 padded."""
    n = len(scores)
    out = np.full(k, -1, dtype=np.int32)
    if n == 0:
        return out
    keys = score_keys(scores).astype(np.int64)
    order = np.argsort(-keys, kind="stable")[: min(k, n)]
    sel = np.sort(order)
    out[: len(sel)] = sel
    return out


def kcache_pages(num_pages: int, stride: int | None = None) -> np.ndarray:
    stride = fp8_page_bytes(INDEX_HEAD_DIM) if stride is None else stride
    return np.zeros((num_pages, stride), dtype=np.uint8)


def indexer_topk(
    q_codes: np.ndarray,
    w: np.ndarray,
    kcache: np.ndarray,
    block_table: np.ndarray,
    req_ids: np.ndarray,
    lengths: np.ndarray,
    k: int,
) -> tuple[np.ndarray, list[np.ndarray]]:
    """Per query row t: exact scores over ``s < lengths[t]`` of request
    ``req_ids[t]`` and its top-k.  Returns ``(topk [T, k], scores per row)``."""
    T = q_codes.shape[0]
    out = np.full((T, k), -1, dtype=np.int32)
    all_scores = []
    for t in range(T):
        n = int(lengths[t])
        s = np.arange(n, dtype=np.int64)
        bt = np.asarray(block_table, dtype=np.int64)[int(req_ids[t])]
        slots = bt[s // PAGE_TOKENS] * PAGE_TOKENS + s % PAGE_TOKENS
        codes, scale = read_fp8_rows(kcache, slots, INDEX_HEAD_DIM)
        sc = exact_scores(q_codes[t], w[t], codes, scale)
        all_scores.append(sc)
        out[t] = topk_ascending(sc, k)
    return out, all_scores


def windowed_lengths(positions: np.ndarray, window: int) -> np.ndarray:
    """Indexer candidate count per query row: ``max(pos + 1 - window, 0)``
    (``attention.py:669-675`` for decode; the per-row causal form of it)."""
    return np.maximum(np.asarray(positions, np.int64) + 1 - window, 0).astype(np.int32)
