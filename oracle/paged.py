"""Slot math and paged page layouts (oracle, test-only).

Slot contract (the vLLM paged-KV convention the plugin relies on, and the
closed form in ``src/vllm_ernie/models/ernie5_5/nvidia/attention.py:845-849``)::

    slot = block_table[seq, pos // 64] * 64 + pos % 64      # slot < 0 -> skip
    page = slot // 64,  row = slot % 64

Page layout of every fp8 cache on the path (latent rows of D bytes, indexer K
rows of 128 bytes): all value rows first, then all fp32 scales -- the layout
``_store_indexer_fp4`` writes (``attention.py:852-860``: values at
``page*stride + off*VALUE_BYTES``, scales at
``page*stride + PAGE*VALUE_BYTES + off*SCALE_BYTES``).  One page of D-byte rows
is ``64*D + 64*4`` bytes; the page stride may be larger (it is a multiple of
``packed_block_stride_alignment``, ``attention.py:561-571``).
"""

from __future__ import annotations

import numpy as np

PAGE_TOKENS = 64  # DSA_BLOCK_SIZE, attention.py:97-98


def slots_from_block_table(
    block_table: np.ndarray, seq_ids: np.ndarray, positions: np.ndarray
) -> np.ndarray:
    """Global slots of tokens ``(seq_ids[i], positions[i])``; int64."""
    bt = np.asarray(block_table, dtype=np.int64)
    seq = np.asarray(seq_ids, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64)
    return bt[seq, pos // PAGE_TOKENS] * PAGE_TOKENS + pos % PAGE_TOKENS


def fp8_page_bytes(dim: int) -> int:
    """Bytes of one page of ``dim``-byte fp8 rows plus fp32 scales."""
    return PAGE_TOKENS * (dim + 4)


def write_fp8_rows(
    cache: np.ndarray,
    slots: np.ndarray,
    codes: np.ndarray,
    scales: np.ndarray,
    dim: int,
) -> None:
    """Scatter fp8 rows and their fp32 scales into ``cache [pages, stride]``.

    Rows whose slot is negative are skipped (``attention.py:845-847``).  When a
    slot repeats, the last row wins (rows are applied in order).
    """
    flat = cache.reshape(cache.shape[0], -1)
    scale_bytes = np.asarray(scales, dtype=np.float32).view(np.uint8).reshape(-1, 4)
    for i, slot in enumerate(np.asarray(slots, dtype=np.int64)):
        if slot < 0:
            continue
        page, row = divmod(int(slot), PAGE_TOKENS)
        flat[page, row * dim : (row + 1) * dim] = codes[i]
        off = PAGE_TOKENS * dim + row * 4
        flat[page, off : off + 4] = scale_bytes[i]


def read_fp8_rows(
    cache: np.ndarray, slots: np.ndarray, dim: int
) -> tuple[np.ndarray, np.ndarray]:
    """Gather ``(codes [n, dim] uint8, scales [n] f32)`` for non-negative slots."""
    flat = cache.reshape(cache.shape[0], -1)
    slots = np.asarray(slots, dtype=np.int64)
    page, row = slots // PAGE_TOKENS, slots % PAGE_TOKENS
    cols = row[:, None] * dim + np.arange(dim)[None, :]
    codes = flat[page[:, None], cols]
    scol = PAGE_TOKENS * dim + row[:, None] * 4 + np.arange(4)[None, :]
    scales = np.ascontiguousarray(flat[page[:, None], scol]).view(np.float32)[:, 0]
    return codes, scales


def write_bf16_rows(cache_bits: np.ndarray, slots: np.ndarray, rows_bits: np.ndarray) -> None:
    """bf16 cache viewed as flat rows ``[-1, D]`` (``attention.py:761-763``)."""
    flat = cache_bits.reshape(-1, cache_bits.shape[-1])
    for i, slot in enumerate(np.asarray(slots, dtype=np.int64)):
        if slot >= 0:
            flat[slot] = rows_bits[i]
