"""Torch-facing wrappers of the C ABI (``include/ernie_kv.h``).

Tensors are device memory and the current HIP stream is passed through; torch
is plumbing here, every byte of the path is computed by the HIP library.  All
outputs are caller-provided (written in place), as in the reference layers.
Caches are ``uint8`` tensors ``[num_pages, page_stride_bytes]``.
"""

from __future__ import annotations

import math

import torch

from . import _lib

PAGE_TOKENS = 64  # DSA_BLOCK_SIZE (attention.py:97-98)
INDEX_HEAD_DIM = 128


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _rs(t: torch.Tensor) -> int:
    """Row stride of a 2-D+ tensor; a size-1 leading dim may carry stride 0
    (e.g. a numpy ``[None]`` view), which would read as zero columns, and an
    empty one has no row to measure (the row's element count stands in)."""
    if t.shape[0] > 1:
        return t.stride(0)
    return t[0].numel() if t.shape[0] == 1 else math.prod(t.shape[1:])


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check_dev(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("ERNIE KV ops take device tensors (no CPU path)")


def fp8_page_bytes(dim: int) -> int:
    return PAGE_TOKENS * (dim + 4)


def _bits16(t: torch.Tensor) -> torch.Tensor:
    _need(t.dtype == torch.bfloat16, f"expected bfloat16, got {t.dtype}")
    return t


# --------------------------------------------------------------------------- writes
def kv_append_quant(rows: torch.Tensor, slot_mapping: torch.Tensor, cache: torch.Tensor) -> None:
    """Quantize bf16 rows ``[T, D]`` to fp8 + fp32 scale into ``cache`` slots."""
    _check_dev(rows, slot_mapping, cache)
    _bits16(rows)
    T, D = rows.shape
    _need(rows.stride(1) == 1, "rows must be row-contiguous")
    _need(slot_mapping.dtype == torch.int64 and slot_mapping.numel() >= T, "slot_mapping int64 [T]")
    _need(cache.dtype == torch.uint8 and cache.dim() == 2 and cache.stride(1) == 1, "cache uint8 [pages, bytes]")
    _lib.call(
        "ekv_kv_append_quant", rows.data_ptr(), _rs(rows), T, D, slot_mapping.data_ptr(),
        cache.data_ptr(), _rs(cache), cache.shape[0], _stream(),
    )


def indexer_k_insert(k: torch.Tensor, slot_mapping: torch.Tensor, kcache: torch.Tensor) -> None:
    """Indexer K rows ``[T, 128]`` bf16 -> 132-byte fp8 rows in ``kcache``."""
    _check_dev(k, slot_mapping, kcache)
    _bits16(k)
    _need(k.shape[1] == INDEX_HEAD_DIM and k.stride(1) == 1, "k must be [T, 128] row-contiguous")
    _need(slot_mapping.dtype == torch.int64, "slot_mapping must be int64")
    _lib.call(
        "ekv_indexer_k_insert", k.data_ptr(), _rs(k), k.shape[0], slot_mapping.data_ptr(),
        kcache.data_ptr(), _rs(kcache), kcache.shape[0], _stream(),
    )


def hca_compress(
    kv_score: torch.Tensor,
    positions: torch.Tensor,
    qsl: torch.Tensor,
    max_query_len: int,
    state: torch.Tensor | None,
    state_slot: torch.Tensor | None,
    ape: torch.Tensor,
    norm_w: torch.Tensor,
    eps: float,
    cos_sin: torch.Tensor,
    comp_block_table: torch.Tensor,
    pool: torch.Tensor,
) -> None:
    _check_dev(kv_score, positions, qsl, state, state_slot, ape, norm_w, cos_sin, comp_block_table, pool)
    _bits16(kv_score)
    D = ape.shape[1]
    _need(kv_score.shape[1] >= 2 * D and kv_score.stride(1) == 1, "kv_score must be [T, 2D]")
    _need(ape.shape == (128, D) and ape.dtype == torch.float32 and ape.is_contiguous(), "ape fp32 [128, D]")
    _need(norm_w.shape == (D,) and norm_w.dtype == torch.float32, "norm_w fp32 [D]")
    _need(cos_sin.dtype == torch.float32 and cos_sin.shape[1] == 64 and cos_sin.is_contiguous(), "cos_sin fp32 [S, 64]")
    _need(comp_block_table.dtype == torch.int32 and comp_block_table.stride(1) == 1, "comp_block_table int32")
    _need(positions.dtype == torch.int64 and qsl.dtype == torch.int32, "positions int64, qsl int32")
    if state is not None:
        _bits16(state)
        _need(state_slot is not None and state_slot.dtype == torch.int32, "state_slot int32")
    _lib.call(
        "ekv_hca_compress", kv_score.data_ptr(), _rs(kv_score), positions.data_ptr(), qsl.data_ptr(),
        qsl.numel() - 1, int(max_query_len), D, _ptr(state), _ptr(state_slot),
        0 if state is None else state.shape[0], ape.data_ptr(), norm_w.data_ptr(), float(eps),
        cos_sin.data_ptr(), cos_sin.shape[0], comp_block_table.data_ptr(), _rs(comp_block_table),
        pool.data_ptr(), _rs(pool), pool.shape[0], _stream(),
    )


def hca_append(
    latent: torch.Tensor,
    kv_score: torch.Tensor | None,
    slot_mapping: torch.Tensor,
    positions: torch.Tensor,
    token_seq: torch.Tensor,
    qsl: torch.Tensor,
    pool: torch.Tensor,
    ring_pages: torch.Tensor | None,
    ring: int,
    state: torch.Tensor | None,
    state_slot: torch.Tensor | None,
) -> None:
    _check_dev(latent, kv_score, slot_mapping, positions, token_seq, qsl, pool, ring_pages, state, state_slot)
    _bits16(latent)
    T, D = latent.shape
    _need(latent.stride(1) == 1, "latent must be row-contiguous")
    _need(slot_mapping.dtype == torch.int64 and positions.dtype == torch.int64, "slot_mapping/positions int64")
    _need(token_seq.dtype == torch.int32 and qsl.dtype == torch.int32, "token_seq/qsl int32")
    if ring_pages is not None:
        _need(ring_pages.dtype == torch.int32 and ring_pages.stride(1) == 1, "ring_pages int32 [B, R/64]")
    if pool.dtype == torch.bfloat16:  # bf16 rows: the flat [-1, D] view, 64 rows a page
        _need(pool.is_contiguous() and pool.numel() % (PAGE_TOKENS * D) == 0, "bf16 pool: contiguous rows of D")
        name, page_stride, num_pages = "ekv_hca_append_bf16", PAGE_TOKENS * D * 2, pool.numel() // (PAGE_TOKENS * D)
    else:
        name, page_stride, num_pages = "ekv_hca_append", _rs(pool), pool.shape[0]
    _lib.call(
        name, latent.data_ptr(), _rs(latent), _ptr(kv_score),
        0 if kv_score is None else _rs(kv_score), T, D, slot_mapping.data_ptr(), positions.data_ptr(),
        token_seq.data_ptr(), qsl.data_ptr(), qsl.numel() - 1, pool.data_ptr(), page_stride, num_pages,
        _ptr(ring_pages), 0 if ring_pages is None else _rs(ring_pages), int(ring), _ptr(state),
        _ptr(state_slot), 0 if state is None else state.shape[0], _stream(),
    )


def _hca_write_args(latent, kv_score, slot_mapping, positions, token_seq, qsl, max_query_len, state, state_slot,
                    ape, norm_w, eps, cos_sin, comp_block_table, ring_pages, ring, pool, workspace) -> list:
    _check_dev(latent, kv_score, slot_mapping, positions, token_seq, qsl, state, state_slot, ape, norm_w, cos_sin,
               comp_block_table, ring_pages, pool, workspace)
    _bits16(latent)
    _bits16(kv_score)
    T, D = latent.shape
    _need(latent.stride(1) == 1, "latent must be row-contiguous")
    _need(kv_score.shape[1] >= 2 * D and kv_score.stride(1) == 1, "kv_score must be [T, 2D]")
    _need(ape.shape == (128, D) and ape.dtype == torch.float32 and ape.is_contiguous(), "ape fp32 [128, D]")
    _need(norm_w.shape == (D,) and norm_w.dtype == torch.float32, "norm_w fp32 [D]")
    _need(cos_sin.dtype == torch.float32 and cos_sin.shape[1] == 64 and cos_sin.is_contiguous(), "cos_sin fp32 [S, 64]")
    _need(comp_block_table.dtype == torch.int32 and comp_block_table.stride(1) == 1, "comp_block_table int32")
    _need(slot_mapping.dtype == torch.int64 and positions.dtype == torch.int64, "slot_mapping/positions int64")
    _need(token_seq.dtype == torch.int32 and qsl.dtype == torch.int32, "token_seq/qsl int32")
    if ring_pages is not None:
        _need(ring_pages.dtype == torch.int32 and ring_pages.stride(1) == 1, "ring_pages int32 [B, R/64]")
    if state is not None:
        _bits16(state)
        _need(state_slot is not None and state_slot.dtype == torch.int32, "state_slot int32")
    if workspace is not None:
        _need(workspace.dtype == torch.uint8 and workspace.is_contiguous(), "workspace: a uint8 hca_write_workspace")
    if pool.dtype == torch.bfloat16:  # bf16 rows: the flat [-1, D] view, 64 rows a page
        _need(pool.is_contiguous() and pool.numel() % (PAGE_TOKENS * D) == 0, "bf16 pool: contiguous rows of D")
        page_stride, num_pages = PAGE_TOKENS * D * 2, pool.numel() // (PAGE_TOKENS * D)
    else:
        _need(pool.dtype == torch.uint8 and pool.dim() == 2 and pool.stride(1) == 1, "fp8 pool uint8 [pages, bytes]")
        page_stride, num_pages = _rs(pool), pool.shape[0]
    return [
        latent.data_ptr(), _rs(latent), kv_score.data_ptr(), _rs(kv_score), T, D,
        slot_mapping.data_ptr(), positions.data_ptr(), token_seq.data_ptr(), qsl.data_ptr(), qsl.numel() - 1,
        int(max_query_len), _ptr(state), _ptr(state_slot), 0 if state is None else state.shape[0],
        ape.data_ptr(), norm_w.data_ptr(), float(eps), cos_sin.data_ptr(), cos_sin.shape[0],
        comp_block_table.data_ptr(), _rs(comp_block_table), _ptr(ring_pages),
        0 if ring_pages is None else _rs(ring_pages), int(ring), pool.data_ptr(), page_stride, num_pages,
        _ptr(workspace), 0 if workspace is None else workspace.numel(),
    ]


def hca_write(
    latent: torch.Tensor,
    kv_score: torch.Tensor,
    slot_mapping: torch.Tensor,
    positions: torch.Tensor,
    token_seq: torch.Tensor,
    qsl: torch.Tensor,
    max_query_len: int,
    state: torch.Tensor | None,
    state_slot: torch.Tensor | None,
    ape: torch.Tensor,
    norm_w: torch.Tensor,
    eps: float,
    cos_sin: torch.Tensor,
    comp_block_table: torch.Tensor,
    ring_pages: torch.Tensor | None,
    ring: int,
    pool: torch.Tensor,
    workspace: torch.Tensor | None = None,
) -> None:
    """``hca_compress`` then ``hca_append`` (same arguments, same result) in
    one call.  With ``workspace`` (``hca_write_workspace``) decode-sized calls
    compress each completed span with ``dim / 64`` workgroups, and longer calls whose
    workspace was sized for their ``max_query_len`` with ``dim / 64`` (same
    bytes).  A bf16 ``pool`` (rows of D bf16 values, 64 a page) takes the
    rows as they are and the compressed rows rounded to bf16; a uint8 pool
    holds fp8 rows with per-token scales."""
    args = _hca_write_args(latent, kv_score, slot_mapping, positions, token_seq, qsl, max_query_len, state, state_slot,
                           ape, norm_w, eps, cos_sin, comp_block_table, ring_pages, ring, pool, workspace)
    _lib.call("ekv_hca_write_bf16" if pool.dtype == torch.bfloat16 else "ekv_hca_write", *args, _stream())


def hca_write_step(
    latent: torch.Tensor,
    kv_score: torch.Tensor,
    slot_mapping: torch.Tensor,
    positions: torch.Tensor,
    token_seq: torch.Tensor,
    qsl: torch.Tensor,
    max_query_len: int,
    state: torch.Tensor | None,
    state_slot: torch.Tensor | None,
    ape: torch.Tensor,
    norm_w: torch.Tensor,
    eps: float,
    cos_sin: torch.Tensor,
    comp_block_table: torch.Tensor,
    ring_pages: torch.Tensor,
    ring: int,
    pool: torch.Tensor,
    window: int,
    out: torch.Tensor,
    lengths: torch.Tensor,
    workspace: torch.Tensor | None = None,
) -> None:
    """``hca_write`` then ``hca_decode_indices(positions, token_seq, ...,
    query_start_loc=qsl, slot_mapping=slot_mapping)`` into ``out`` /
    ``lengths``, same results; decode-sized calls build the index rows in the
    write's launch."""
    _need(ring_pages is not None, "ring_pages is needed for the index rows")
    _check_dev(out, lengths)
    _need(out.dtype == torch.int32 and out.dim() == 2 and out.stride(1) == 1, "out must be int32 [T, width]")
    _need(lengths.dtype == torch.int32 and lengths.numel() >= latent.shape[0], "lengths must be int32 [T]")
    args = _hca_write_args(latent, kv_score, slot_mapping, positions, token_seq, qsl, max_query_len, state, state_slot,
                           ape, norm_w, eps, cos_sin, comp_block_table, ring_pages, ring, pool, workspace)
    name = "ekv_hca_write_step_bf16" if pool.dtype == torch.bfloat16 else "ekv_hca_write_step"
    _lib.call(name, *args, int(window), out.data_ptr(), out.stride(0), out.shape[1], lengths.data_ptr(), _stream())


def hca_write_workspace(num_seqs: int, dim: int, device, max_query_len: int = 0) -> torch.Tensor:
    """Zero-filled workspace of ``hca_write`` for calls of up to ``num_seqs``
    sequences of width ``dim`` (every call leaves it zero again).  Sized for
    ``max_query_len`` rows per sequence it also holds a slot per span of
    such calls, which then compress each span with ``dim / 64`` workgroups."""
    spans = int(num_seqs) * (max(int(max_query_len), 0) // 128 + 1)
    n = int(_lib.load().ekv_hca_write_workspace_size(spans, int(dim)))
    return torch.zeros(max(n, 16), dtype=torch.uint8, device=device)


def hca_decode_indices(
    positions: torch.Tensor,
    req_ids: torch.Tensor,
    comp_block_table: torch.Tensor,
    ring_pages: torch.Tensor,
    ring: int,
    out: torch.Tensor,
    lengths: torch.Tensor,
    window: int = 128,
    query_start_loc: torch.Tensor | None = None,
    slot_mapping: torch.Tensor | None = None,
) -> None:
    """Index rows [compressed entries | window | -1 ...] and their lengths.
    With ``query_start_loc`` and ``slot_mapping`` (the call's), window
    positions inside the call use the call's slots, older ones the ring."""
    _check_dev(positions, req_ids, comp_block_table, ring_pages, out, lengths, query_start_loc, slot_mapping)
    _need(out.dtype == torch.int32 and out.stride(1) == 1, "out int32 [T, W]")
    _need((query_start_loc is None) == (slot_mapping is None), "query_start_loc and slot_mapping go together")
    if slot_mapping is not None:
        _need(slot_mapping.dtype == torch.int64 and query_start_loc.dtype == torch.int32,
              "slot_mapping int64, query_start_loc int32")
    _lib.call(
        "ekv_hca_decode_indices", positions.data_ptr(), req_ids.data_ptr(), positions.numel(),
        comp_block_table.data_ptr(), _rs(comp_block_table), ring_pages.data_ptr(), _rs(ring_pages),
        int(ring), int(window), _ptr(query_start_loc), _ptr(slot_mapping), out.data_ptr(), _rs(out), out.shape[1],
        lengths.data_ptr(), _stream(),
    )


# --------------------------------------------------------------------------- indexer
def merge_swa_topk(topk_indices: torch.Tensor, out: torch.Tensor, positions: torch.Tensor, window: int) -> None:
    """Reference signature and semantics (attention.py:606-641)."""
    num_tokens = positions.shape[0]
    if num_tokens == 0:
        return
    topk, width = topk_indices.shape[1], out.shape[1]
    assert width >= topk + window
    _check_dev(topk_indices, out, positions)
    _need(topk_indices.dtype == torch.int32 and out.dtype == torch.int32, "int32 index buffers")
    _need(topk_indices.stride(1) == 1 and out.stride(1) == 1, "rows must be contiguous")
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    _lib.call(
        "ekv_merge_swa_topk", topk_indices.data_ptr(), _rs(topk_indices), out.data_ptr(), _rs(out),
        pos.data_ptr(), num_tokens, topk, width, int(window), _stream(),
    )


def indexer_prep(
    q: torch.Tensor,
    k: torch.Tensor,
    ln_w: torch.Tensor,
    ln_b: torch.Tensor,
    eps: float,
    cos_sin: torch.Tensor,
    positions: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``Ernie5_5Indexer.forward`` before the quantization (attention.py:
    955-969): ``(hadamard(rope(q)), hadamard(rope(k_norm(k))))`` for
    ``q [T, H, 128]``, ``k [T, 128]`` bf16; NeoX rope on dims 0..63 by the rows
    ``cos_sin[positions]`` of an fp32 ``[N, 64]`` table (cos | sin)."""
    _check_dev(q, k, ln_w, ln_b, cos_sin, positions)
    _bits16(q)
    _bits16(k)
    T, H, D = q.shape
    _need(D == 128 and q.stride(2) == 1 and k.shape == (T, 128) and k.stride(1) == 1, "q [T, H, 128], k [T, 128]")
    _need(ln_w.shape == (128,) and ln_b.shape == (128,) and ln_w.dtype == torch.float32 and ln_b.dtype == torch.float32,
          "ln_w, ln_b fp32 [128]")
    _need(cos_sin.dtype == torch.float32 and cos_sin.shape[1] == 64 and cos_sin.is_contiguous(), "cos_sin fp32 [N, 64]")
    _need(positions.dtype == torch.int64 and positions.numel() == T, "positions int64 [T]")
    q_out = torch.empty((T, H, 128), dtype=q.dtype, device=q.device)
    k_out = torch.empty((T, 128), dtype=k.dtype, device=k.device)
    _lib.call(
        "ekv_indexer_prep", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), _rs(k), T, H,
        ln_w.contiguous().data_ptr(), ln_b.contiguous().data_ptr(), float(eps), cos_sin.data_ptr(), cos_sin.shape[0],
        positions.data_ptr(), q_out.data_ptr(), k_out.data_ptr(), _stream(),
    )
    return q_out, k_out


def hadamard_rows(x: torch.Tensor) -> torch.Tensor:
    """Reference semantics of ``hadamard_rows`` (attention.py:102-108)."""
    _check_dev(x)
    _bits16(x)
    _need(x.dim() == 2 and x.shape[1] == 128 and x.stride(1) == 1, "x must be [n, 128] row-contiguous")
    y = torch.empty_like(x, memory_format=torch.contiguous_format)
    _lib.call("ekv_hadamard_rows", x.data_ptr(), _rs(x), y.data_ptr(), _rs(y), x.shape[0], 128, _stream())
    return y


def indexer_q_quant(
    q: torch.Tensor, weights: torch.Tensor, with_digits: bool = True
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """``q [T, H, 128]`` bf16 -> (q fp8 [T,H,128] uint8, folded weights fp32 [T,H],
    int8 digit planes [T,3,H,128])."""
    _check_dev(q, weights)
    _bits16(q)
    T, H, Dh = q.shape
    _need(Dh == 128 and q.stride(2) == 1, "q must be [T, H, 128] with unit last stride")
    _need(weights.shape[:2] == (T, H) and weights.stride(1) == 1, "weights [T, H]")
    _need(weights.dtype in (torch.bfloat16, torch.float32), "weights bf16 or fp32")
    q_fp8 = torch.empty((T, H, 128), dtype=torch.uint8, device=q.device)
    w_out = torch.empty((T, H), dtype=torch.float32, device=q.device)
    digits = torch.empty((T, 3, H, 128), dtype=torch.int8, device=q.device) if with_digits else None
    _lib.call(
        "ekv_indexer_q_quant", q.data_ptr(), _rs(q), q.stride(1), weights.data_ptr(),
        int(weights.dtype == torch.bfloat16), _rs(weights), T, H, q_fp8.data_ptr(), w_out.data_ptr(),
        _ptr(digits), _stream(),
    )
    return q_fp8, w_out, digits


def dsa_decode_prologue(
    k: torch.Tensor,
    kcache: torch.Tensor,
    latent: torch.Tensor,
    cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    q: torch.Tensor,
    weights: torch.Tensor,
    positions: torch.Tensor,
    window: int,
    lengths: torch.Tensor,
    prep: tuple | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One launch doing ``indexer_k_insert(k, slot_mapping, kcache)``,
    ``kv_append_quant(latent, slot_mapping, cache)``, ``indexer_q_quant(q,
    weights)`` (returned) and ``indexer_windowed_lengths(positions, window,
    lengths)``.  With ``prep = (ln_w, ln_b, eps, cos_sin)``, q and k are the
    raw indexer projections and ``indexer_prep`` runs on them first, in the
    same launch."""
    _check_dev(k, kcache, latent, cache, slot_mapping, q, weights, positions, lengths)
    ln_w = ln_b = cos_sin = None
    eps = 0.0
    if prep is not None:
        ln_w, ln_b, eps, cos_sin = prep
        _check_dev(ln_w, ln_b, cos_sin)
        _need(ln_w.shape == (128,) and ln_b.shape == (128,) and ln_w.dtype == torch.float32
              and ln_b.dtype == torch.float32 and ln_w.is_contiguous() and ln_b.is_contiguous(), "ln_w, ln_b fp32 [128]")
        _need(cos_sin.dtype == torch.float32 and cos_sin.shape[1] == 64 and cos_sin.is_contiguous(),
              "cos_sin fp32 [N, 64]")
    _bits16(k)
    _bits16(latent)
    _bits16(q)
    T = k.shape[0]
    _need(k.shape == (T, 128) and k.stride(1) == 1, "k must be [T, 128] row-contiguous")
    _need(latent.dim() == 2 and latent.shape[0] == T and latent.stride(1) == 1, "latent must be [T, D] row-contiguous")
    _need(slot_mapping.dtype == torch.int64 and slot_mapping.numel() >= T, "slot_mapping int64 [T]")
    for c in (kcache, cache):
        _need(c.dtype == torch.uint8 and c.dim() == 2 and c.stride(1) == 1, "caches uint8 [pages, bytes]")
    _need(q.dim() == 3 and q.shape[0] == T and q.shape[2] == 128 and q.stride(2) == 1, "q must be [T, H, 128]")
    H = q.shape[1]
    _need(weights.shape[:2] == (T, H) and weights.stride(1) == 1, "weights [T, H]")
    _need(weights.dtype in (torch.bfloat16, torch.float32), "weights bf16 or fp32")
    _need(positions.dtype == torch.int64 and lengths.dtype == torch.int32, "positions int64, lengths int32")
    q_fp8 = torch.empty((T, H, 128), dtype=torch.uint8, device=q.device)
    w_out = torch.empty((T, H), dtype=torch.float32, device=q.device)
    digits = torch.empty((T, 3, H, 128), dtype=torch.int8, device=q.device)
    _lib.call(
        "ekv_dsa_decode_prologue", k.data_ptr(), _rs(k), kcache.data_ptr(), _rs(kcache), kcache.shape[0],
        latent.data_ptr(), _rs(latent), latent.shape[1], cache.data_ptr(), _rs(cache), cache.shape[0],
        slot_mapping.data_ptr(), T, q.data_ptr(), _rs(q), q.stride(1), weights.data_ptr(),
        int(weights.dtype == torch.bfloat16), _rs(weights), H, q_fp8.data_ptr(), w_out.data_ptr(), digits.data_ptr(),
        positions.data_ptr(), int(window), lengths.data_ptr(), _ptr(ln_w), _ptr(ln_b), float(eps), _ptr(cos_sin),
        0 if cos_sin is None else cos_sin.shape[0], _stream(),
    )
    return q_fp8, w_out, digits


def dsa_decode_prologue_fp4(
    k: torch.Tensor,
    kcache: torch.Tensor,
    latent: torch.Tensor,
    cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    q: torch.Tensor,
    weights: torch.Tensor,
    positions: torch.Tensor,
    window: int,
    lengths: torch.Tensor,
    prep: tuple | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The MXFP4 ``dsa_decode_prologue``, one launch: with ``prep = (ln_w,
    ln_b, eps, cos_sin)`` ``indexer_prep`` of q and k first, then
    ``indexer_k_insert_fp4(k, slot_mapping, kcache)``, ``indexer_q_quant_fp4(q,
    weights)`` (returned: values, scale words, folded weights),
    ``kv_append_quant(latent, slot_mapping, cache)`` and
    ``indexer_windowed_lengths(positions, window, lengths)``."""
    _check_dev(k, kcache, latent, cache, slot_mapping, q, weights, positions, lengths)
    ln_w = ln_b = cos_sin = None
    eps = 0.0
    if prep is not None:
        ln_w, ln_b, eps, cos_sin = prep
        _check_dev(ln_w, ln_b, cos_sin)
        _need(ln_w.shape == (128,) and ln_b.shape == (128,) and ln_w.dtype == torch.float32
              and ln_b.dtype == torch.float32 and ln_w.is_contiguous() and ln_b.is_contiguous(), "ln_w, ln_b fp32 [128]")
        _need(cos_sin.dtype == torch.float32 and cos_sin.shape[1] == 64 and cos_sin.is_contiguous(),
              "cos_sin fp32 [N, 64]")
    _bits16(k)
    _bits16(latent)
    _bits16(q)
    T = k.shape[0]
    _need(k.shape == (T, 128) and k.stride(1) == 1, "k must be [T, 128] row-contiguous")
    _need(latent.dim() == 2 and latent.shape[0] == T and latent.stride(1) == 1, "latent must be [T, D] row-contiguous")
    _need(slot_mapping.dtype == torch.int64 and slot_mapping.numel() >= T, "slot_mapping int64 [T]")
    for c in (kcache, cache):
        _need(c.dtype == torch.uint8 and c.dim() == 2 and c.stride(1) == 1, "caches uint8 [pages, bytes]")
    _need(q.dim() == 3 and q.shape[0] == T and q.shape[2] == 128 and q.stride(2) == 1, "q must be [T, H, 128]")
    H = q.shape[1]
    _need(weights.shape[:2] == (T, H) and weights.stride(1) == 1, "weights [T, H]")
    _need(weights.dtype in (torch.bfloat16, torch.float32), "weights bf16 or fp32")
    _need(positions.dtype == torch.int64 and lengths.dtype == torch.int32, "positions int64, lengths int32")
    values = torch.empty((T, H, 64), dtype=torch.uint8, device=q.device)
    scales = torch.empty((T, H), dtype=torch.int32, device=q.device)
    w_out = torch.empty((T, H), dtype=torch.float32, device=q.device)
    _lib.call(
        "ekv_dsa_decode_prologue_fp4", k.data_ptr(), _rs(k), kcache.data_ptr(), _rs(kcache), kcache.shape[0],
        latent.data_ptr(), _rs(latent), latent.shape[1], cache.data_ptr(), _rs(cache), cache.shape[0],
        slot_mapping.data_ptr(), T, q.data_ptr(), _rs(q), q.stride(1), weights.data_ptr(),
        int(weights.dtype == torch.bfloat16), _rs(weights), H, values.data_ptr(), scales.data_ptr(), w_out.data_ptr(),
        positions.data_ptr(), int(window), lengths.data_ptr(), _ptr(ln_w), _ptr(ln_b), float(eps), _ptr(cos_sin),
        0 if cos_sin is None else cos_sin.shape[0], _stream(),
    )
    return values, scales, w_out


def indexer_windowed_lengths(positions: torch.Tensor, window: int, out: torch.Tensor) -> None:
    _check_dev(positions, out)
    _need(positions.dtype == torch.int64 and out.dtype == torch.int32, "positions int64, out int32")
    _lib.call("ekv_indexer_windowed_lengths", positions.data_ptr(), positions.numel(), int(window), out.data_ptr(), _stream())


def indexer_score(
    q_digits: torch.Tensor,
    w: torch.Tensor,
    kcache: torch.Tensor,
    block_table: torch.Tensor,
    req_ids: torch.Tensor,
    lengths: torch.Tensor,
    max_len: int,
    scores: torch.Tensor,
) -> None:
    _check_dev(q_digits, w, kcache, block_table, req_ids, lengths, scores)
    T = q_digits.shape[0]
    _need(q_digits.shape[1:] == (3, 64, 128) and q_digits.is_contiguous(), "q_digits [T, 3, 64, 128]")
    _need(w.shape == (T, 64) and w.dtype == torch.float32 and w.is_contiguous(), "w fp32 [T, 64]")
    _need(block_table.dtype == torch.int32 and block_table.stride(1) == 1, "block_table int32")
    _need(scores.dtype == torch.float32 and scores.stride(1) == 1 and scores.shape[1] >= max_len, "scores")
    _lib.call(
        "ekv_indexer_score", q_digits.data_ptr(), w.data_ptr(), kcache.data_ptr(), _rs(kcache),
        kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(), lengths.data_ptr(),
        T, int(max_len), scores.data_ptr(), _rs(scores), _stream(),
    )


def topk_select(scores: torch.Tensor, lengths: torch.Tensor, k: int, out: torch.Tensor) -> None:
    _check_dev(scores, lengths, out)
    _need(scores.dtype == torch.float32 and scores.stride(1) == 1, "scores fp32 rows")
    _need(out.dtype == torch.int32 and out.stride(1) == 1 and out.shape[1] >= k, "out int32 [T, >=k]")
    _lib.call(
        "ekv_topk_select", scores.data_ptr(), _rs(scores), lengths.data_ptr(), scores.shape[0],
        scores.shape[1], out.data_ptr(), _rs(out), int(k), _stream(),
    )


def indexer_filter_dots(q_codes: torch.Tensor, k_codes: torch.Tensor) -> torch.Tensor:
    """The indexer filter's fp8-MFMA dot products ``[S, 64]`` of e4m3fn codes
    ``q_codes [64, 128]`` and ``k_codes [S, 128]`` (S a multiple of 16), by
    the filter's own MFMA call (a diagnostic of its error bound)."""
    _check_dev(q_codes, k_codes)
    _need(q_codes.shape == (64, 128) and q_codes.dtype == torch.uint8 and q_codes.is_contiguous(), "q_codes [64, 128]")
    _need(k_codes.dim() == 2 and k_codes.shape[1] == 128 and k_codes.dtype == torch.uint8 and k_codes.is_contiguous(),
          "k_codes [S, 128] uint8")
    _need(k_codes.shape[0] % 16 == 0, "S must be a multiple of 16")
    out = torch.empty((k_codes.shape[0], 64), dtype=torch.float32, device=k_codes.device)
    _lib.call("ekv_indexer_filter_dots", q_codes.data_ptr(), k_codes.data_ptr(), k_codes.shape[0], out.data_ptr(),
              _stream())
    return out


def indexer_topk_workspace(num_tokens: int, max_len: int, device) -> torch.Tensor:
    """Zero-filled workspace for the indexer top-k calls of up to
    ``num_tokens`` rows of ``max_len`` tokens (the calls keep its counters
    zero, so it is reused as is)."""
    need = _lib.load().ekv_indexer_topk_workspace_size(int(num_tokens), int(max_len))
    return torch.zeros(max(need, 1), dtype=torch.uint8, device=device)


def _topk_common(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, T):
    _check_dev(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths)
    if q_fp8 is not None:
        _need(q_fp8.shape == (T, 64, 128) and q_fp8.dtype == torch.uint8 and q_fp8.is_contiguous(), "q_fp8 [T, 64, 128]")
    if q_digits is not None:
        _need(q_digits.shape == (T, 3, 64, 128) and q_digits.is_contiguous(), "q_digits [T, 3, 64, 128]")
    _need(w.shape == (T, 64) and w.dtype == torch.float32 and w.is_contiguous(), "w fp32 [T, 64]")
    _need(block_table.dtype == torch.int32 and block_table.stride(1) == 1, "block_table int32")
    _need(lengths.dtype == torch.int32 and req_ids.dtype == torch.int32, "lengths/req_ids int32")


def indexer_filter(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, max_len: int,
                   workspace: torch.Tensor, k: int = 2048) -> None:
    """Stage 1: fp8-MFMA filter, candidate bound and (when it fits one launch)
    the candidates' exact scores, into ``workspace``."""
    T = q_fp8.shape[0]
    _topk_common(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, T)
    _lib.call(
        "ekv_indexer_filter", q_fp8.data_ptr(), q_digits.data_ptr(), w.data_ptr(), kcache.data_ptr(), _rs(kcache),
        kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(), lengths.data_ptr(), T,
        int(max_len), int(k), workspace.data_ptr(), workspace.numel(), _stream(),
    )


def _merged_args(merged, positions, window, topk_out, T):
    """(pointer, row stride, width, positions pointer) of an optional merged output."""
    if merged is None:
        return 0, 0, 0, 0
    _need(positions is not None, "merged output needs positions")
    _check_dev(merged, positions)
    _need(merged.dtype == torch.int32 and merged.stride(1) == 1 and merged.shape[0] == T, "merged int32 [T, W]")
    _need(positions.dtype == torch.int64 and positions.shape[0] == T, "positions int64 [T]")
    _need(merged.shape[1] >= topk_out.shape[1] + window, "merged width must be >= k + window")
    return merged.data_ptr(), _rs(merged), merged.shape[1], positions.data_ptr()


def indexer_select(q_digits, w, kcache, block_table, req_ids, lengths, max_len: int, topk_out: torch.Tensor,
                   workspace: torch.Tensor, merged: torch.Tensor | None = None,
                   positions: torch.Tensor | None = None, window: int = 128, merged_slots: bool = False) -> None:
    """Stage 2: the candidates' exact scores (if stage 1 left them), exact top-k
    (ascending, -1 padded).  With ``merged`` (and ``positions``) it also writes
    ``merge_swa_topk(topk_out, merged, positions, window)`` in the same launch;
    ``merged_slots`` turns those entries into cache slots through the block
    table (-1 when unmapped)."""
    T = q_digits.shape[0]
    _topk_common(None, q_digits, w, kcache, block_table, req_ids, lengths, T)
    _need(topk_out.dtype == torch.int32 and topk_out.stride(1) == 1, "topk_out int32 [T, K]")
    m_ptr, m_stride, m_width, p_ptr = 0, 0, 0, 0
    if merged is not None:
        _need(positions is not None, "merged output needs positions")
        _check_dev(merged, positions)
        _need(merged.dtype == torch.int32 and merged.stride(1) == 1 and merged.shape[0] == T, "merged int32 [T, W]")
        _need(positions.dtype == torch.int64 and positions.shape[0] == T, "positions int64 [T]")
        _need(merged.shape[1] >= topk_out.shape[1] + window, "merged width must be >= k + window")
        m_ptr, m_stride, m_width, p_ptr = merged.data_ptr(), _rs(merged), merged.shape[1], positions.data_ptr()
    _lib.call(
        "ekv_indexer_select", q_digits.data_ptr(), w.data_ptr(), kcache.data_ptr(), _rs(kcache), kcache.shape[0],
        block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(), lengths.data_ptr(), T, int(max_len),
        topk_out.data_ptr(), _rs(topk_out), topk_out.shape[1], workspace.data_ptr(), workspace.numel(),
        m_ptr, m_stride, m_width, p_ptr, int(window), int(bool(merged_slots)), _stream(),
    )


def indexer_topk(
    q_fp8: torch.Tensor,
    q_digits: torch.Tensor,
    w: torch.Tensor,
    kcache: torch.Tensor,
    block_table: torch.Tensor,
    req_ids: torch.Tensor,
    lengths: torch.Tensor,
    max_len: int,
    topk_out: torch.Tensor,
    workspace: torch.Tensor | None = None,
) -> None:
    """Exact top-k over ``s < lengths[t]`` (filter + exact rescoring), ascending, -1 padded."""
    T = q_fp8.shape[0]
    _topk_common(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, T)
    _need(topk_out.dtype == torch.int32 and topk_out.stride(1) == 1, "topk_out int32 [T, K]")
    if workspace is None:
        workspace = indexer_topk_workspace(T, max_len, q_fp8.device)
    _lib.call(
        "ekv_indexer_topk", q_fp8.data_ptr(), q_digits.data_ptr(), w.data_ptr(), kcache.data_ptr(), _rs(kcache),
        kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(), lengths.data_ptr(),
        T, int(max_len), topk_out.data_ptr(), _rs(topk_out), topk_out.shape[1], workspace.data_ptr(),
        workspace.numel(), _stream(),
    )


def indexer_topk_merged(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, max_len: int,
                        topk_out: torch.Tensor, workspace: torch.Tensor, merged: torch.Tensor | None = None,
                        positions: torch.Tensor | None = None, window: int = 128,
                        merged_slots: bool = False) -> None:
    """``indexer_topk`` with ``indexer_select``'s merged output, in one call
    (one launch when the filter fits one: its workgroups then also select)."""
    T = q_fp8.shape[0]
    _topk_common(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, T)
    _need(topk_out.dtype == torch.int32 and topk_out.stride(1) == 1, "topk_out int32 [T, K]")
    m_ptr, m_stride, m_width, p_ptr = _merged_args(merged, positions, window, topk_out, T)
    _lib.call(
        "ekv_indexer_topk_merged", q_fp8.data_ptr(), q_digits.data_ptr(), w.data_ptr(), kcache.data_ptr(),
        _rs(kcache), kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(),
        lengths.data_ptr(), T, int(max_len), topk_out.data_ptr(), _rs(topk_out), topk_out.shape[1],
        workspace.data_ptr(), workspace.numel(), m_ptr, m_stride, m_width, p_ptr, int(window),
        int(bool(merged_slots)), _stream(),
    )


def dsa_decode_prologue_folds(num_tokens: int, max_len: int) -> bool:
    """Whether ``dsa_decode_prologue_topk_merged`` of ``num_tokens`` rows of
    at most ``max_len`` keys runs as one launch on the current device."""
    return bool(_lib.load().ekv_dsa_decode_prologue_folds(int(num_tokens), int(max_len)))


def dsa_decode_prologue_topk_merged(
    k: torch.Tensor,
    kcache: torch.Tensor,
    latent: torch.Tensor,
    cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    q: torch.Tensor,
    weights: torch.Tensor,
    positions: torch.Tensor,
    window: int,
    lengths: torch.Tensor,
    block_table: torch.Tensor,
    req_ids: torch.Tensor,
    max_len: int,
    topk_out: torch.Tensor,
    workspace: torch.Tensor,
    merged: torch.Tensor,
    merged_slots: bool = False,
    prep: tuple | None = None,
    max_new_rows: int = 1,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``dsa_decode_prologue(k, kcache, latent, cache, slot_mapping, q,
    weights, positions, window, lengths, prep)`` then ``indexer_topk_merged``
    of its outputs over ``kcache`` (the top-k, the merged rows), in one call.
    ``max_new_rows`` is the most query rows any one sequence has in the call
    (its newest positions; 1 for plain decode): with ``1 <= max_new_rows <=
    window`` no row scores a key the call appends, and the prologue runs in
    the top-k's launch when that is one launch.  Returns the prologue's
    ``(q_fp8, w, q_digits)``."""
    _check_dev(k, kcache, latent, cache, slot_mapping, q, weights, positions, lengths, block_table, req_ids,
               topk_out, workspace, merged)
    ln_w = ln_b = cos_sin = None
    eps = 0.0
    if prep is not None:
        ln_w, ln_b, eps, cos_sin = prep
        _check_dev(ln_w, ln_b, cos_sin)
        _need(ln_w.shape == (128,) and ln_b.shape == (128,) and ln_w.dtype == torch.float32
              and ln_b.dtype == torch.float32 and ln_w.is_contiguous() and ln_b.is_contiguous(), "ln_w, ln_b fp32 [128]")
        _need(cos_sin.dtype == torch.float32 and cos_sin.shape[1] == 64 and cos_sin.is_contiguous(),
              "cos_sin fp32 [N, 64]")
    _bits16(k)
    _bits16(latent)
    _bits16(q)
    T = k.shape[0]
    _need(k.shape == (T, 128) and k.stride(1) == 1, "k must be [T, 128] row-contiguous")
    _need(latent.dim() == 2 and latent.shape[0] == T and latent.stride(1) == 1, "latent must be [T, D] row-contiguous")
    _need(slot_mapping.dtype == torch.int64 and slot_mapping.numel() >= T, "slot_mapping int64 [T]")
    for c in (kcache, cache):
        _need(c.dtype == torch.uint8 and c.dim() == 2 and c.stride(1) == 1, "caches uint8 [pages, bytes]")
    _need(q.dim() == 3 and q.shape[0] == T and q.shape[2] == 128 and q.stride(2) == 1, "q must be [T, H, 128]")
    H = q.shape[1]
    _need(weights.shape[:2] == (T, H) and weights.stride(1) == 1, "weights [T, H]")
    _need(weights.dtype in (torch.bfloat16, torch.float32), "weights bf16 or fp32")
    _need(positions.dtype == torch.int64 and lengths.dtype == torch.int32, "positions int64, lengths int32")
    _need(block_table.dtype == torch.int32 and block_table.stride(1) == 1, "block_table int32")
    _need(req_ids.dtype == torch.int32, "req_ids int32")
    _need(topk_out.dtype == torch.int32 and topk_out.stride(1) == 1, "topk_out int32 [T, K]")
    m_ptr, m_stride, m_width, p_ptr = _merged_args(merged, positions, window, topk_out, T)
    q_fp8 = torch.empty((T, H, 128), dtype=torch.uint8, device=q.device)
    w_out = torch.empty((T, H), dtype=torch.float32, device=q.device)
    digits = torch.empty((T, 3, H, 128), dtype=torch.int8, device=q.device)
    _lib.call(
        "ekv_dsa_decode_prologue_topk_merged", k.data_ptr(), _rs(k), kcache.data_ptr(), _rs(kcache), kcache.shape[0],
        latent.data_ptr(), _rs(latent), latent.shape[1], cache.data_ptr(), _rs(cache), cache.shape[0],
        slot_mapping.data_ptr(), T, q.data_ptr(), _rs(q), q.stride(1), weights.data_ptr(),
        int(weights.dtype == torch.bfloat16), _rs(weights), H, q_fp8.data_ptr(), w_out.data_ptr(), digits.data_ptr(),
        p_ptr, int(window), int(max_new_rows), lengths.data_ptr(), _ptr(ln_w), _ptr(ln_b), float(eps), _ptr(cos_sin),
        0 if cos_sin is None else cos_sin.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(),
        int(max_len), topk_out.data_ptr(), _rs(topk_out), topk_out.shape[1], workspace.data_ptr(), workspace.numel(),
        m_ptr, m_stride, m_width, int(bool(merged_slots)), _stream(),
    )
    return q_fp8, w_out, digits


def indexer_topk_counter_bytes() -> int:
    """Bytes at the front of a top-k workspace holding the one-launch path's
    per-row counters (zero between calls)."""
    return int(_lib.load().ekv_indexer_topk_counter_bytes())


def indexer_set_spin_limit(polls: int) -> int:
    """Test hook: polls a one-launch top-k workgroup waits for the rest of its
    row before it gives up (the row's last workgroup then selects alone);
    ``polls < 0`` restores the default.  Returns the previous value."""
    return int(_lib.load().ekv_indexer_set_spin_limit(int(polls)))


# --------------------------------------------------------------------------- MXFP4 indexer
FP4_ROW_BYTES = INDEX_HEAD_DIM // 2 + INDEX_HEAD_DIM // 32  # 68 (attention.py:929-932)


def fp4_page_bytes() -> int:
    return PAGE_TOKENS * FP4_ROW_BYTES


def mxfp4_quant(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``downcast_to_mxfp(x, axis=-1)`` of bf16 ``x [..., D]`` (D a multiple of
    32): ``(values uint8 [..., D/2], scales uint8 [..., D/32])``."""
    _check_dev(x)
    _bits16(x)
    D = x.shape[-1]
    _need(D % 32 == 0, "last dim must be a multiple of 32")
    x2 = x.reshape(-1, D)
    _need(x2.stride(1) == 1, "x must have a unit last stride")
    rows = x2.shape[0]
    values = torch.empty((rows, D // 2), dtype=torch.uint8, device=x.device)
    scales = torch.empty((rows, D // 32), dtype=torch.uint8, device=x.device)
    _lib.call("ekv_mxfp4_quant", x2.data_ptr(), _rs(x2), 0, rows, 1, D, values.data_ptr(), _rs(values),
              scales.data_ptr(), _rs(scales), _stream())
    return values.view(*x.shape[:-1], D // 2), scales.view(*x.shape[:-1], D // 32)


def indexer_q_quant_fp4(q: torch.Tensor, weights: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``q [T, H, 128]`` bf16 -> (values uint8 [T, H, 64], scales int32 [T, H],
    w fp32 [T, H] = weights * 128**-0.5 * 64**-0.5)."""
    _check_dev(q, weights)
    _bits16(q)
    T, H, Dh = q.shape
    _need(Dh == 128 and q.stride(2) == 1, "q must be [T, H, 128] with unit last stride")
    _need(weights.shape[:2] == (T, H) and weights.stride(1) == 1, "weights [T, H]")
    _need(weights.dtype in (torch.bfloat16, torch.float32), "weights bf16 or fp32")
    values = torch.empty((T, H, 64), dtype=torch.uint8, device=q.device)
    scales = torch.empty((T, H), dtype=torch.int32, device=q.device)
    w_out = torch.empty((T, H), dtype=torch.float32, device=q.device)
    _lib.call(
        "ekv_indexer_q_quant_fp4", q.data_ptr(), _rs(q), q.stride(1), weights.data_ptr(),
        int(weights.dtype == torch.bfloat16), _rs(weights), T, H, values.data_ptr(), scales.data_ptr(),
        w_out.data_ptr(), _stream(),
    )
    return values, scales, w_out


def indexer_k_insert_fp4(k: torch.Tensor, slot_mapping: torch.Tensor, kcache: torch.Tensor) -> None:
    """Indexer K rows ``[T, 128]`` bf16 -> 68-byte MXFP4 rows in ``kcache``."""
    _check_dev(k, slot_mapping, kcache)
    _bits16(k)
    _need(k.shape[1] == INDEX_HEAD_DIM and k.stride(1) == 1, "k must be [T, 128] row-contiguous")
    _need(slot_mapping.dtype == torch.int64, "slot_mapping must be int64")
    _lib.call(
        "ekv_indexer_k_insert_fp4", k.data_ptr(), _rs(k), k.shape[0], slot_mapping.data_ptr(),
        kcache.data_ptr(), _rs(kcache), kcache.shape[0], _stream(),
    )


def indexer_store_fp4(values: torch.Tensor, scales: torch.Tensor, slot_mapping: torch.Tensor,
                      kcache: torch.Tensor) -> None:
    """``_store_indexer_fp4``: quantized rows (values ``[T, 64]``, scales
    ``[T, 4]`` uint8) to their slots in ``kcache``."""
    _check_dev(values, scales, slot_mapping, kcache)
    _need(values.dtype == torch.uint8 and values.shape[1] == 64 and values.stride(1) == 1, "values uint8 [T, 64]")
    _need(scales.dtype == torch.uint8 and scales.shape[1] == 4 and scales.stride(1) == 1, "scales uint8 [T, 4]")
    _need(slot_mapping.dtype == torch.int64, "slot_mapping must be int64")
    _lib.call(
        "ekv_indexer_store_fp4", values.data_ptr(), _rs(values), scales.data_ptr(), _rs(scales), values.shape[0],
        slot_mapping.data_ptr(), kcache.data_ptr(), _rs(kcache), kcache.shape[0], _stream(),
    )


def _fp4_common(q_values, q_scales, w, kcache, block_table, req_ids, lengths):
    _check_dev(q_values, q_scales, w, kcache, block_table, req_ids, lengths)
    T = q_values.shape[0]
    _need(q_values.shape == (T, 64, 64) and q_values.dtype == torch.uint8 and q_values.is_contiguous(),
          "q_values uint8 [T, 64, 64]")
    _need(q_scales.shape == (T, 64) and q_scales.dtype == torch.int32 and q_scales.is_contiguous(),
          "q_scales int32 [T, 64]")
    _need(w.shape == (T, 64) and w.dtype == torch.float32 and w.is_contiguous(), "w fp32 [T, 64]")
    _need(block_table.dtype == torch.int32 and block_table.stride(1) == 1, "block_table int32")
    _need(lengths.dtype == torch.int32 and req_ids.dtype == torch.int32, "lengths/req_ids int32")
    return T


def indexer_score_fp4(q_values, q_scales, w, kcache, block_table, req_ids, lengths, max_len: int,
                      scores: torch.Tensor) -> None:
    """Exact MXFP4 indexer scores of every token ``s < lengths[t]``."""
    T = _fp4_common(q_values, q_scales, w, kcache, block_table, req_ids, lengths)
    _check_dev(scores)
    _need(scores.dtype == torch.float32 and scores.stride(1) == 1 and scores.shape[1] >= max_len, "scores")
    _lib.call(
        "ekv_indexer_score_fp4", q_values.data_ptr(), q_scales.data_ptr(), w.data_ptr(), kcache.data_ptr(),
        _rs(kcache), kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(),
        lengths.data_ptr(), T, int(max_len), scores.data_ptr(), _rs(scores), _stream(),
    )


def indexer_filter_fp4(q_values, q_scales, w, kcache, block_table, req_ids, lengths, max_len: int,
                       workspace: torch.Tensor, k: int = 2048) -> None:
    """Stage 1 of the MXFP4 top-k (as ``indexer_filter``)."""
    T = _fp4_common(q_values, q_scales, w, kcache, block_table, req_ids, lengths)
    _lib.call(
        "ekv_indexer_filter_fp4", q_values.data_ptr(), q_scales.data_ptr(), w.data_ptr(), kcache.data_ptr(),
        _rs(kcache), kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(),
        lengths.data_ptr(), T, int(max_len), int(k), workspace.data_ptr(), workspace.numel(), _stream(),
    )


def indexer_select_fp4(q_values, q_scales, w, kcache, block_table, req_ids, lengths, max_len: int,
                       topk_out: torch.Tensor, workspace: torch.Tensor, merged: torch.Tensor | None = None,
                       positions: torch.Tensor | None = None, window: int = 128, merged_slots: bool = False) -> None:
    """Stage 2 of the MXFP4 top-k (as ``indexer_select``)."""
    T = _fp4_common(q_values, q_scales, w, kcache, block_table, req_ids, lengths)
    _need(topk_out.dtype == torch.int32 and topk_out.stride(1) == 1, "topk_out int32 [T, K]")
    m_ptr, m_stride, m_width, p_ptr = 0, 0, 0, 0
    if merged is not None:
        _need(positions is not None, "merged output needs positions")
        _check_dev(merged, positions)
        _need(merged.dtype == torch.int32 and merged.stride(1) == 1 and merged.shape[0] == T, "merged int32 [T, W]")
        _need(positions.dtype == torch.int64 and positions.shape[0] == T, "positions int64 [T]")
        _need(merged.shape[1] >= topk_out.shape[1] + window, "merged width must be >= k + window")
        m_ptr, m_stride, m_width, p_ptr = merged.data_ptr(), _rs(merged), merged.shape[1], positions.data_ptr()
    _lib.call(
        "ekv_indexer_select_fp4", q_values.data_ptr(), q_scales.data_ptr(), w.data_ptr(), kcache.data_ptr(),
        _rs(kcache), kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(),
        lengths.data_ptr(), T, int(max_len), topk_out.data_ptr(), _rs(topk_out), topk_out.shape[1],
        workspace.data_ptr(), workspace.numel(), m_ptr, m_stride, m_width, p_ptr, int(window),
        int(bool(merged_slots)), _stream(),
    )


def indexer_topk_fp4(q_values, q_scales, w, kcache, block_table, req_ids, lengths, max_len: int,
                     topk_out: torch.Tensor, workspace: torch.Tensor | None = None) -> None:
    """Exact MXFP4 top-k over ``s < lengths[t]``, ascending, -1 padded."""
    T = _fp4_common(q_values, q_scales, w, kcache, block_table, req_ids, lengths)
    _need(topk_out.dtype == torch.int32 and topk_out.stride(1) == 1, "topk_out int32 [T, K]")
    if workspace is None:
        workspace = indexer_topk_workspace(T, max_len, q_values.device)
    _lib.call(
        "ekv_indexer_topk_fp4", q_values.data_ptr(), q_scales.data_ptr(), w.data_ptr(), kcache.data_ptr(),
        _rs(kcache), kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(),
        lengths.data_ptr(), T, int(max_len), topk_out.data_ptr(), _rs(topk_out), topk_out.shape[1],
        workspace.data_ptr(), workspace.numel(), _stream(),
    )


def indexer_topk_merged_fp4(q_values, q_scales, w, kcache, block_table, req_ids, lengths, max_len: int,
                            topk_out: torch.Tensor, workspace: torch.Tensor, merged: torch.Tensor | None = None,
                            positions: torch.Tensor | None = None, window: int = 128,
                            merged_slots: bool = False) -> None:
    """MXFP4 ``indexer_topk_merged``."""
    T = _fp4_common(q_values, q_scales, w, kcache, block_table, req_ids, lengths)
    _need(topk_out.dtype == torch.int32 and topk_out.stride(1) == 1, "topk_out int32 [T, K]")
    m_ptr, m_stride, m_width, p_ptr = _merged_args(merged, positions, window, topk_out, T)
    _lib.call(
        "ekv_indexer_topk_merged_fp4", q_values.data_ptr(), q_scales.data_ptr(), w.data_ptr(), kcache.data_ptr(),
        _rs(kcache), kcache.shape[0], block_table.data_ptr(), _rs(block_table), req_ids.data_ptr(),
        lengths.data_ptr(), T, int(max_len), topk_out.data_ptr(), _rs(topk_out), topk_out.shape[1],
        workspace.data_ptr(), workspace.numel(), m_ptr, m_stride, m_width, p_ptr, int(window),
        int(bool(merged_slots)), _stream(),
    )


def indexer_filter_dots_fp4(q_values: torch.Tensor, q_scales: torch.Tensor, k_values: torch.Tensor,
                            k_scales: torch.Tensor) -> torch.Tensor:
    """The MXFP4 filter's MFMA dot products ``[S, 64]`` (a diagnostic of its
    error bound): q ``[64, 64]`` uint8 + ``[64]`` int32, k ``[S, 64]`` + ``[S]``."""
    _check_dev(q_values, q_scales, k_values, k_scales)
    _need(q_values.shape == (64, 64) and q_values.dtype == torch.uint8 and q_values.is_contiguous(), "q_values [64, 64]")
    _need(q_scales.shape == (64,) and q_scales.dtype == torch.int32, "q_scales int32 [64]")
    S = k_values.shape[0]
    _need(k_values.shape == (S, 64) and k_values.dtype == torch.uint8 and k_values.is_contiguous(), "k_values [S, 64]")
    _need(k_scales.shape == (S,) and k_scales.dtype == torch.int32, "k_scales int32 [S]")
    _need(S % 16 == 0, "S must be a multiple of 16")
    out = torch.empty((S, 64), dtype=torch.float32, device=k_values.device)
    _lib.call("ekv_indexer_filter_dots_fp4", q_values.data_ptr(), q_scales.data_ptr(), k_values.data_ptr(),
              k_scales.data_ptr(), S, out.data_ptr(), _stream())
    return out


# --------------------------------------------------------------------------- upstream page format
DS_MLA_ROW_BYTES = 656  # 512 fp8 + 4 fp32 tile scales + 64 bf16


def ds_mla_page_stride() -> int:
    """64 fp8_ds_mla rows rounded up to the packed block alignment (9216 B)."""
    return -(-PAGE_TOKENS * DS_MLA_ROW_BYTES // 9216) * 9216


def export_fp8_ds_mla_pages(cache: torch.Tensor, src_pages: torch.Tensor, out: torch.Tensor,
                            dst_pages: torch.Tensor | None = None) -> None:
    """This library's 576-wide latent pages ``src_pages`` of ``cache`` ->
    fp8_ds_mla pages of ``out`` (``dst_pages``, default 0..n-1); lossless."""
    _check_dev(cache, src_pages, out, dst_pages)
    _need(src_pages.dtype == torch.int32 and (dst_pages is None or dst_pages.dtype == torch.int32),
          "page ids must be int32")
    _need(dst_pages is None or dst_pages.numel() == src_pages.numel(), "dst_pages must match src_pages")
    _lib.call("ekv_export_fp8_ds_mla_pages", cache.data_ptr(), _rs(cache), cache.shape[0], src_pages.data_ptr(),
              src_pages.numel(), out.data_ptr(), _rs(out), out.shape[0], _ptr(dst_pages), _stream())


def import_fp8_ds_mla_pages(src: torch.Tensor, src_pages: torch.Tensor, cache: torch.Tensor,
                            dst_pages: torch.Tensor | None = None) -> None:
    """fp8_ds_mla pages ``src_pages`` of ``src`` -> this library's latent
    pages of ``cache`` (``dst_pages``, default 0..n-1), requantized per row."""
    _check_dev(src, src_pages, cache, dst_pages)
    _need(src_pages.dtype == torch.int32 and (dst_pages is None or dst_pages.dtype == torch.int32),
          "page ids must be int32")
    _need(dst_pages is None or dst_pages.numel() == src_pages.numel(), "dst_pages must match src_pages")
    _lib.call("ekv_import_fp8_ds_mla_pages", src.data_ptr(), _rs(src), src.shape[0], src_pages.data_ptr(),
              src_pages.numel(), cache.data_ptr(), _rs(cache), cache.shape[0], _ptr(dst_pages), _stream())


# --------------------------------------------------------------------------- decode
def decode_workspace(num_tokens: int, heads: int, width: int, device) -> torch.Tensor:
    """Workspace for every ``sparse_mla_decode`` call of at most ``num_tokens``
    rows, ``heads`` heads and ``width`` index entries (the split partials:
    O / l and (m, l) in fp32 per split and head, and each row's split
    range).  A call given a smaller workspace raises; none allocates."""
    need = _lib.load().ekv_sparse_mla_decode_workspace_size(num_tokens, heads, width)
    return torch.empty(max(need, 1), dtype=torch.uint8, device=device)


def sparse_mla_decode(
    q: torch.Tensor,
    cache: torch.Tensor,
    indices: torch.Tensor,
    scale: float,
    out: torch.Tensor,
    lse: torch.Tensor | None = None,
    sinks: torch.Tensor | None = None,
    lengths: torch.Tensor | None = None,
    block_table: torch.Tensor | None = None,
    req_ids: torch.Tensor | None = None,
    cache_bf16: bool = False,
    workspace: torch.Tensor | None = None,
) -> None:
    """Sparse MLA decode (attention.py:701-790): q [T, H, D] bf16 -> out [T, H, 512]."""
    _check_dev(q, cache, indices, out, lse, sinks, lengths, block_table, req_ids)
    _bits16(q)
    T, H, D = q.shape
    _need(q.stride(2) == 1, "q last dim must be contiguous")
    _need(indices.dtype == torch.int32 and indices.stride(-1) == 1, "indices int32 [T, W]")
    idx = indices.reshape(T, -1) if indices.dim() != 2 else indices
    _need(out.dtype == torch.bfloat16 and out.shape[0] == T and out.shape[1] >= H and out.shape[2] == 512, "out bf16 [T, H, 512]")
    if cache_bf16:
        _need(cache.dtype == torch.bfloat16, "bf16 cache expected")
        num_pages = cache.numel() // (PAGE_TOKENS * D)
        page_stride = PAGE_TOKENS * D * 2
    else:
        _need(cache.dtype == torch.uint8 and cache.dim() == 2, "fp8 cache must be uint8 [pages, bytes]")
        num_pages, page_stride = cache.shape[0], _rs(cache)
    if sinks is not None:
        _need(sinks.dtype == torch.float32 and sinks.numel() >= H, "sinks fp32 [H]")
    if workspace is None:
        workspace = decode_workspace(T, H, idx.shape[1], q.device)
    else:
        need = _lib.load().ekv_sparse_mla_decode_workspace_size(T, H, idx.shape[1])
        _need(workspace.dtype == torch.uint8 and workspace.is_contiguous() and workspace.numel() >= need,
              f"decode workspace too small: {workspace.numel()} < {need} bytes")
    _lib.call(
        "ekv_sparse_mla_decode", q.data_ptr(), _rs(q), q.stride(1), T, H, D, cache.data_ptr(),
        int(cache_bf16), page_stride, num_pages, idx.data_ptr(), _rs(idx), idx.shape[1], _ptr(lengths),
        _ptr(block_table), 0 if block_table is None else _rs(block_table), _ptr(req_ids), _ptr(sinks),
        float(scale), out.data_ptr(), _rs(out), out.stride(1), _ptr(lse),
        0 if lse is None else _rs(lse), workspace.data_ptr(), workspace.numel(), _stream(),
    )


# --------------------------------------------------------------------------- post-attention quant
def tma_aligned_rows(n: int) -> int:
    """Rows of a 4-byte scale buffer padded to 16 bytes (the TMA alignment
    the reference's packed scale buffers use)."""
    return (n + 3) // 4 * 4


def sigmoid_mul_quant_fp8(x: torch.Tensor, gate: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``x * sigmoid(gate)`` as 1x128 UE8M0 fp8 with packed scales
    (attention.py:340-361): returns (out fp8 [N, hidden], scale int32
    [N, hidden / 512] with strides (1, tma_aligned_rows(N)))."""
    _check_dev(x, gate)
    _bits16(x)
    _bits16(gate)
    N, hidden = x.shape
    _need(gate.shape == x.shape and hidden % 512 == 0, "gate like x, hidden a multiple of 512")
    _need(x.stride(-1) == 1 and gate.stride(-1) == 1, "rows must be contiguous")
    out = torch.empty((N, hidden), dtype=torch.float8_e4m3fn, device=x.device)
    packs = hidden // 512
    aligned = tma_aligned_rows(N)
    scale = torch.empty_strided((N, packs), (1, aligned), dtype=torch.int32, device=x.device)
    if N:
        _lib.call("ekv_sigmoid_mul_quant_fp8", x.data_ptr(), _rs(x), gate.data_ptr(), _rs(gate), N, hidden,
                  out.data_ptr(), hidden, scale.data_ptr(), aligned, _stream())
    return out, scale


def vha_inv_rope_fp8_quant(o: torch.Tensor, mix: torch.Tensor, positions: torch.Tensor,
                           cos_sin_cache: torch.Tensor, n_groups: int, nope_dim: int,
                           rope_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """VHA head mixing + inverse RoPE + fp8 quant (attention.py:232-285).
    Returns (data fp8 [T, n_groups, hpg * 512] -- a transposed view of a
    [n_groups, T, hpg * 512] buffer -- and scale int32 [T, n_groups, hpg] --
    a view of [n_groups, hpg, tma_aligned_rows(T)] -- with chunk c's biased
    exponent in byte c), the layouts of the reference."""
    _check_dev(o, mix, positions, cos_sin_cache)
    _bits16(o)
    _bits16(mix)
    T, H, D = o.shape
    _need(H == 64 and D == 512 and o.stride(-1) == 1, "o [T, 64, 512] with unit channel stride")
    _need(mix.shape == (64, 64) and mix.is_contiguous(), "mix [64, 64] contiguous")
    _need(positions.dtype == torch.int64 and positions.numel() >= T, "positions int64 [T]")
    _need(cos_sin_cache.dtype == torch.float32 and cos_sin_cache.stride(-1) == 1, "cos_sin_cache fp32 rows")
    hpg = H // n_groups
    out = torch.empty((n_groups, T, hpg * D), dtype=torch.float8_e4m3fn, device=o.device)
    aligned = tma_aligned_rows(T)
    scale = torch.empty((n_groups, hpg, aligned), dtype=torch.int32, device=o.device)
    if aligned:
        _lib.call("ekv_vha_inv_rope_fp8_quant", o.data_ptr(), o.stride(0), o.stride(1), T, H,
                  mix.data_ptr(), positions.data_ptr(), cos_sin_cache.data_ptr(), cos_sin_cache.stride(0),
                  int(n_groups), int(nope_dim), int(rope_dim), out.data_ptr(), scale.data_ptr(), aligned, _stream())
    return out.transpose(0, 1), scale.permute(2, 0, 1)[:T]
