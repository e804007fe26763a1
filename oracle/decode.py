"""Sparse MLA decode with an attention sink (oracle, test-only; fp64 math).

Follows ``src/vllm_ernie/models/ernie5_5/nvidia/attention.py:701-790``: per query
row and head, attention over the gathered latent rows named by the index row
(``-1`` entries skipped), keys are the full D-wide rows, values their first
``dv`` (512) columns, the softmax scale is ``qk_head_dim**-0.5`` (``:1156``),
and the per-head sink enters the denominator only (``:701-706``)::

    m   = max(max_j s_j, sink)
    out = sum_j exp(s_j - m) v_j / (sum_j exp(s_j - m) + exp(sink - m))
    lse = log(sum_j exp(s_j))          # natural log, sink excluded

A ``-inf`` sink is a no-op (``:717-720``).  Rows with no valid index give
``out = 0`` and ``lse = -inf``.  The lse convention (natural log, sink
excluded) is this build's contract: upstream FlashMLA's is unpinned here.
"""

from __future__ import annotations

import numpy as np

from .fp8 import decode_e4m3
from .paged import PAGE_TOKENS


def gather_rows_fp8(cache: np.ndarray, slots: np.ndarray, dim: int) -> np.ndarray:
    """Dequantized fp64 rows ``[n, dim]`` of the fp8 paged cache."""
    flat = cache.reshape(cache.shape[0], -1)
    slots = np.asarray(slots, dtype=np.int64)
    page, row = slots // PAGE_TOKENS, slots % PAGE_TOKENS
    codes = flat[page[:, None], row[:, None] * dim + np.arange(dim)[None, :]]
    scol = PAGE_TOKENS * dim + row[:, None] * 4 + np.arange(4)[None, :]
    scale = np.ascontiguousarray(flat[page[:, None], scol]).view(np.float32)[:, 0]
    return decode_e4m3(codes).astype(np.float64) * scale.astype(np.float64)[:, None]


def gather_rows_bf16(cache_f32: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """Rows of a bf16 cache (given as float32 values), viewed as flat rows."""
    flat = cache_f32.reshape(-1, cache_f32.shape[-1])
    return flat[np.asarray(slots, dtype=np.int64)].astype(np.float64)


def sparse_mla_decode(
    q: np.ndarray,
    rows_of: "callable",
    indices: np.ndarray,
    scale: float,
    dv: int,
    sinks: np.ndarray | None = None,
    lengths: np.ndarray | None = None,
):
    """``q [T, H, D]``; ``rows_of(slots) -> [n, D]`` fp64; returns (out, lse)."""
    q = np.asarray(q, dtype=np.float64)
    T, H, _ = q.shape
    out = np.zeros((T, H, dv), dtype=np.float64)
    lse = np.full((T, H), -np.inf, dtype=np.float64)
    sink = None if sinks is None else np.asarray(sinks, dtype=np.float64)
    for t in range(T):
        idx = np.asarray(indices[t], dtype=np.int64)
        if lengths is not None:
            idx = idx[: int(lengths[t])]
        idx = idx[idx >= 0]
        if len(idx) == 0:
            continue
        kv = rows_of(idx)  # [n, D]
        s = (q[t] @ kv.T) * scale  # [H, n]
        m = s.max(axis=1)
        if sink is not None:
            m = np.maximum(m, sink)
        e = np.exp(s - m[:, None])
        den = e.sum(axis=1)
        lse[t] = m + np.log(den)
        if sink is not None:
            den = den + np.exp(sink - m)
        out[t] = (e @ kv[:, :dv]) / den[:, None]
    return out, lse
