"""Window merge and logical->global index conversion (oracle, test-only).

``merge_swa_topk`` follows ``src/vllm_ernie/models/ernie5_5/nvidia/attention.py``
lines 582-641: each output row is ``[topk[:n] | seq-w .. seq-1 | -1 ...]`` with
``seq = pos + 1``, ``n = min(max(seq - window, 0), topk)``, ``w = min(seq,
window)``.  Pinned by the known-answer test ``test_dsa_backend.py:18-37``
(transcribed in ``tests/test_oracle_paths.py::test_merge_swa_topk_known_answer``
and, on the GPU, ``tests/test_gpu_indexer.py::test_merge_swa_topk_known_answer``).

The logical->global conversion is the paged-slot closed form applied to a
request-local index (the FlashMLA fp8 path receives global indices and a dummy
block table, ``attention.py:737-748``); ``-1`` stays ``-1``.
"""

from __future__ import annotations

import numpy as np

from .paged import PAGE_TOKENS


def merge_swa_topk(
    topk: np.ndarray, positions: np.ndarray, width: int, window: int
) -> np.ndarray:
    topk = np.asarray(topk, dtype=np.int32)
    num_tokens, k = topk.shape
    assert width >= k + window
    out = np.full((num_tokens, width), -1, dtype=np.int32)
    for r, pos in enumerate(np.asarray(positions, dtype=np.int64)):
        seq = int(pos) + 1
        n = min(max(seq - window, 0), k)
        w = min(seq, window)
        out[r, :n] = topk[r, :n]
        out[r, n : n + w] = np.arange(seq - w, seq, dtype=np.int32)
    return out


def logical_to_global(
    indices: np.ndarray, req_ids: np.ndarray, block_table: np.ndarray
) -> np.ndarray:
    idx = np.asarray(indices, dtype=np.int64)
    bt = np.asarray(block_table, dtype=np.int64)
    req = np.asarray(req_ids, dtype=np.int64)[:, None]
    safe = np.maximum(idx, 0)
    glob = bt[req, safe // PAGE_TOKENS] * PAGE_TOKENS + safe % PAGE_TOKENS
    return np.where(idx >= 0, glob, -1).astype(np.int32)
