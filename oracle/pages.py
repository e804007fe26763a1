"""Upstream KV page formats at the connector boundary (oracle; test
infrastructure only).

``fp8_ds_mla`` is the fp8 KV-cache dtype of vLLM's FlashMLA sparse backend,
the cache the reference's DSA layers (and its FlashMLA HCA class) run on
(``src/vllm_ernie/models/ernie5_5/nvidia/attention.py:551-558, 792-795``).
A 576-wide latent row (512 nope + 64 rope dims) is 656 bytes, token-major in
the page:

* bytes ``[0, 512)``: e4m3fn codes of dims 0..511;
* bytes ``[512, 528)``: four fp32 scales, scale ``t`` for dims
  ``128 t .. 128 t + 127`` (value = code * scale);
* bytes ``[528, 656)``: dims 512..575 as bf16, not quantized.

(the layout FlashMLA documents for its FP8 sparse decode).  Pages hold 64
such rows; the page stride is a multiple of the packed block alignment
``lcm(512, 1024, 1152) = 9216`` (``attention.py:561-571``): 46080 bytes.

This build's own latent page is 64 rows of 576 codes followed by 64 fp32
per-row power-of-two scales (580 bytes a row).  The transcoders:

* export (own -> fp8_ds_mla): codes 0..511 unchanged, the row scale in all
  four tile slots, dims 512..575 dequantized to bf16 -- lossless (a code
  times a power of two is exact in bf16);
* import (fp8_ds_mla -> own): the row dequantized in fp32
  (``fl32(code * scale_t)``, the bf16 rope dims as they are), then the
  build's row quantization (``oracle.fp8.quantize_rows``) -- one rounding,
  none when the tile scales are equal powers of two; a page export wrote comes
  back with the same values (same bytes, except rows whose largest code is
  224, requantized to half the scale with doubled codes).

The indexer pages need no transcoder: this build already stores them as
DeepGEMM's paged-MQA layout (all 128-byte fp8 rows of the page, then all
fp32 scales; ``attention.py:852`` states the values-then-scales order).
Parity: the 656-byte layout follows the public FlashMLA format; the scale
rule upstream's ``concat_and_cache_ds_mla`` applies when it writes such rows
is not available here (parity unpinned) -- import accepts any fp32 scales.
"""

from __future__ import annotations

import numpy as np

from .fp8 import bf16_bits, bf16_from_bits, decode_e4m3, quantize_rows
from .paged import PAGE_TOKENS

DS_MLA_ROW = 656
DS_MLA_NOPE = 512
DS_MLA_ROPE = 64
OWN_DIM = 576
BLOCK_ALIGN = 9216


def ds_mla_page_stride() -> int:
    """64 rows of 656 bytes rounded up to the packed block alignment."""
    return -(-PAGE_TOKENS * DS_MLA_ROW // BLOCK_ALIGN) * BLOCK_ALIGN


def own_page_rows(page: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``(codes [64, 576], scales [64] f32)`` of one own-format page."""
    codes = page[: PAGE_TOKENS * OWN_DIM].reshape(PAGE_TOKENS, OWN_DIM)
    scales = np.ascontiguousarray(page[PAGE_TOKENS * OWN_DIM: PAGE_TOKENS * (OWN_DIM + 4)]).view(np.float32)
    return codes, scales


def export_page(page: np.ndarray, out: np.ndarray) -> None:
    """One own-format page -> one fp8_ds_mla page (``out`` bytes beyond the 64
    rows are left as they are)."""
    codes, scales = own_page_rows(page)
    rows = out[: PAGE_TOKENS * DS_MLA_ROW].reshape(PAGE_TOKENS, DS_MLA_ROW)
    rows[:, :DS_MLA_NOPE] = codes[:, :DS_MLA_NOPE]
    rows[:, DS_MLA_NOPE:DS_MLA_NOPE + 16] = np.repeat(scales[:, None], 4, axis=1).astype(np.float32).view(np.uint8)
    rope = (decode_e4m3(codes[:, DS_MLA_NOPE:]) * scales[:, None]).astype(np.float32)
    rows[:, DS_MLA_NOPE + 16:] = bf16_bits(rope).view(np.uint8).reshape(PAGE_TOKENS, 2 * DS_MLA_ROPE)


def dequant_ds_mla_page(page: np.ndarray) -> np.ndarray:
    """fp32 rows ``[64, 576]`` of one fp8_ds_mla page."""
    rows = page[: PAGE_TOKENS * DS_MLA_ROW].reshape(PAGE_TOKENS, DS_MLA_ROW)
    tile = np.ascontiguousarray(rows[:, DS_MLA_NOPE:DS_MLA_NOPE + 16]).view(np.float32)  # [64, 4]
    nope = (decode_e4m3(rows[:, :DS_MLA_NOPE]) * np.repeat(tile, 128, axis=1)).astype(np.float32)
    rope = bf16_from_bits(np.ascontiguousarray(rows[:, DS_MLA_NOPE + 16:]).view(np.uint16))
    return np.concatenate([nope, rope.astype(np.float32)], axis=1)


def import_page(page: np.ndarray, out: np.ndarray) -> None:
    """One fp8_ds_mla page -> one own-format page (requantized per row)."""
    codes, scales = quantize_rows(dequant_ds_mla_page(page))
    out[: PAGE_TOKENS * OWN_DIM] = codes.reshape(-1)
    out[PAGE_TOKENS * OWN_DIM: PAGE_TOKENS * (OWN_DIM + 4)] = scales.astype(np.float32).view(np.uint8)


def export_pages(cache: np.ndarray, src_pages, out: np.ndarray, dst_pages=None) -> None:
    """Pages ``src_pages[i]`` of ``cache`` to pages ``dst_pages[i]`` (default i)
    of ``out``; negative or out-of-range page ids are skipped."""
    for i, p in enumerate(np.asarray(src_pages, np.int64)):
        d = i if dst_pages is None else int(dst_pages[i])
        if 0 <= p < cache.shape[0] and 0 <= d < out.shape[0]:
            export_page(cache[p], out[d])


def import_pages(src: np.ndarray, src_pages, cache: np.ndarray, dst_pages=None) -> None:
    for i, p in enumerate(np.asarray(src_pages, np.int64)):
        d = i if dst_pages is None else int(dst_pages[i])
        if 0 <= p < src.shape[0] and 0 <= d < cache.shape[0]:
            import_page(src[p], cache[d])
