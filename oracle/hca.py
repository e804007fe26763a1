"""HCA write path: append + fp8 quant, 128->1 span compressor, window ring (oracle).

Reference: the HCA layer (``src/vllm_ernie/models/ernie5_5/nvidia/attention.py``
``:398-408, 471-539``) hands the projected compressor input ``kv_score`` (the
``compressor.fused_wkv_wgate`` output, ``nvidia/model.py:684-685``) and the
per-token latent to upstream ``DeepseekV4Attention._prepare_and_attn_fn``,
which appends the latent by ``slot_mapping`` and runs ``DeepseekCompressor``
(state cache + ``c128_boundary``).  vLLM 0.32.0 is absent, so the compressor
below is a restatement of the DeepSeek-V4 compressor as described by its call
sites -- **parity unpinned** against upstream; it is pinned against closed
forms (constant gate -> mean, one-hot gate -> copy, permutation invariance) and
an fp64 brute force in ``tests/test_oracle_hca.py``.

Compressor of span j (positions 128j .. 128j+127), per channel c < D::

    g_i = fl32(score_i[c] + ape[i, c]);   m = max_i g_i
    e_i = exp_ekv(fl32(g_i - m))
    Z, N = 0, 0;  for i in 0..127:  Z = fl32(Z + e_i);  N = fl32(N + fl32(e_i * kv_i[c]))
    x_c = fl32(N / Z)
    RMSNorm over D (eps from rms_norm_eps), sums in the kernel's order
    RoPE (interleaved pairs) on channels D-64..D-1 at position 128j
    UE8M0 fp8 quant -> compressed row j

``exp_ekv`` is this build's own exp: ``2**n * P(f)`` with ``n = rint(x*log2 e)``,
``f = x*log2 e - n`` and ``P`` the degree-6 Taylor polynomial of ``2**f``
evaluated by Horner in fp32 (no fused multiply-add), flushing to 0 below
``2**-125``.  The kernel evaluates the same operations.

State: the kv_score rows of a sequence's most recent 256 positions live in a
ring ``state[state_slot, pos % 256]`` so a span that completes in a later call
(or is re-completed after an MTP rollback) can be recompressed.
Window ring: the fp8 rows of the most recent ``R`` positions (``R`` a multiple
of 64, >= 128 + draft tokens) in pages named by ``ring_pages[seq]``.
"""

from __future__ import annotations

import math

import numpy as np

from .fp8 import bf16_round, quantize_rows
from .paged import PAGE_TOKENS, write_fp8_rows

SPAN = 128
STATE_RING = 256
WINDOW = 128

LOG2E = np.float32(1.0 / math.log(2.0))
EXP_C = [np.float32(math.log(2.0) ** k / math.factorial(k)) for k in range(7)]


def exp_ekv(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    t = (x * LOG2E).astype(np.float32)
    n = np.rint(t).astype(np.float32)
    f = (t - n).astype(np.float32)
    p = EXP_C[6]
    for k in range(5, -1, -1):
        p = ((p * f).astype(np.float32) + EXP_C[k]).astype(np.float32)
    out = np.ldexp(p, np.clip(n, -200, 200).astype(np.int32)).astype(np.float32)
    return np.where(t < np.float32(-125.0), np.float32(0.0), out).astype(np.float32)


def compress_span(
    kv: np.ndarray,
    score: np.ndarray,
    ape: np.ndarray,
    norm_w: np.ndarray,
    eps: float,
    cos_sin: np.ndarray,
) -> np.ndarray:
    """One compressed row (fp32 before quant) from ``kv, score [128, D]`` (bf16 values)."""
    kv = np.asarray(kv, np.float32)
    D = kv.shape[1]
    g = (np.asarray(score, np.float32) + np.asarray(ape, np.float32)).astype(np.float32)
    m = g.max(axis=0)
    e = exp_ekv((g - m[None, :]).astype(np.float32))
    Z = np.zeros(D, np.float32)
    N = np.zeros(D, np.float32)
    for i in range(SPAN):
        Z = (Z + e[i]).astype(np.float32)
        N = (N + (e[i] * kv[i]).astype(np.float32)).astype(np.float32)
    x = (N / Z).astype(np.float32)
    sq = (x * x).astype(np.float32).reshape(D // 4, 4)
    part = np.zeros(D // 4, np.float32)
    for k in range(4):
        part = (part + sq[:, k]).astype(np.float32)
    S = np.float32(0.0)
    for v in part:
        S = np.float32(S + v)
    ms = np.float32(S / np.float32(D))
    r = np.float32(np.float32(1.0) / np.sqrt(np.float32(ms + np.float32(eps))))
    y = ((x * r).astype(np.float32) * np.asarray(norm_w, np.float32)).astype(np.float32)
    cs = np.asarray(cos_sin, np.float32)
    x0 = y[D - 64 :: 2].copy()
    x1 = y[D - 63 :: 2].copy()
    c, s = cs[:32], cs[32:64]
    y[D - 64 :: 2] = ((x0 * c).astype(np.float32) - (x1 * s).astype(np.float32)).astype(np.float32)
    y[D - 63 :: 2] = ((x0 * s).astype(np.float32) + (x1 * c).astype(np.float32)).astype(np.float32)
    return y


def ring_slot(ring_pages: np.ndarray, seq: int, pos: int, ring: int) -> int:
    r = pos % ring
    return int(ring_pages[seq, r // PAGE_TOKENS]) * PAGE_TOKENS + r % PAGE_TOKENS


def comp_slot(comp_block_table: np.ndarray, seq: int, j: int) -> int:
    return int(comp_block_table[seq, j // PAGE_TOKENS]) * PAGE_TOKENS + j % PAGE_TOKENS


class HcaState:
    """Numpy model of every buffer the HCA write path touches."""

    def __init__(self, num_pages: int, dim: int, num_state: int, stride: int | None = None):
        self.dim = dim
        stride = PAGE_TOKENS * (dim + 4) if stride is None else stride
        self.pool = np.zeros((num_pages, stride), dtype=np.uint8)
        self.state = np.zeros((num_state, STATE_RING, 2 * dim), dtype=np.float32)


def hca_write(
    st: HcaState,
    latent: np.ndarray,
    kv_score: np.ndarray,
    positions: np.ndarray,
    token_seq: np.ndarray,
    qsl: np.ndarray,
    slot_mapping: np.ndarray,
    ring_pages: np.ndarray | None,
    ring: int,
    comp_block_table: np.ndarray | None,
    state_slot: np.ndarray,
    ape: np.ndarray,
    norm_w: np.ndarray,
    eps: float,
    comp_cos_sin: np.ndarray,
) -> None:
    """Apply one call: compress completed spans (from the pre-call state and
    this call's rows), then append, update the ring and the state ring."""
    D = st.dim
    positions = np.asarray(positions, np.int64)
    B = len(qsl) - 1
    if comp_block_table is not None:
        for b in range(B):
            t0, t1 = int(qsl[b]), int(qsl[b + 1])
            if t1 <= t0:
                continue
            p0, pl = int(positions[t0]), int(positions[t0]) + (t1 - t0) - 1
            for j in range(p0 // SPAN, (pl + 1) // SPAN):
                rows = np.empty((SPAN, 2 * D), np.float32)
                for i in range(SPAN):
                    p = SPAN * j + i
                    if p >= p0:
                        rows[i] = kv_score[t0 + p - p0]
                    else:
                        rows[i] = st.state[int(state_slot[b]), p % STATE_RING]
                y = compress_span(rows[:, :D], rows[:, D:], ape, norm_w, eps, comp_cos_sin[j])
                codes, scale = quantize_rows(y[None, :])
                write_fp8_rows(st.pool, [comp_slot(comp_block_table, b, j)], codes, scale, D)
    codes, scale = quantize_rows(latent)
    write_fp8_rows(st.pool, slot_mapping, codes, scale, D)
    for b in range(B):
        t0, t1 = int(qsl[b]), int(qsl[b + 1])
        if t1 <= t0:
            continue
        p0 = int(positions[t0])
        pl = p0 + (t1 - t0) - 1
        for t in range(t0, t1):
            p = p0 + (t - t0)
            if ring_pages is not None and p > pl - ring:
                write_fp8_rows(st.pool, [ring_slot(ring_pages, b, p, ring)], codes[t : t + 1], scale[t : t + 1], D)
            if comp_block_table is not None and p > pl - STATE_RING:
                st.state[int(state_slot[b]), p % STATE_RING] = kv_score[t]


def hca_decode_indices(
    positions: np.ndarray,
    req_ids: np.ndarray,
    comp_block_table: np.ndarray,
    ring_pages: np.ndarray,
    ring: int,
    width: int,
    window: int = WINDOW,
) -> tuple[np.ndarray, np.ndarray]:
    """Global slots ``[comp 0..n_c-1 | window p-w+1..p | -1...]`` and lengths."""
    T = len(positions)
    out = np.full((T, width), -1, dtype=np.int32)
    lens = np.zeros(T, dtype=np.int32)
    for t in range(T):
        p = int(positions[t])
        b = int(req_ids[t])
        n_c = (p + 1) // SPAN
        w = min(p + 1, window)
        assert n_c + w <= width
        for j in range(n_c):
            out[t, j] = comp_slot(comp_block_table, b, j)
        for i in range(w):
            out[t, n_c + i] = ring_slot(ring_pages, b, p - w + 1 + i, ring)
        lens[t] = n_c + w
    return out, lens


def bf16_values(x: np.ndarray) -> np.ndarray:
    return bf16_round(np.asarray(x, np.float32))
