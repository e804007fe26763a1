"""ctypes binding of ``libernie_kv.so`` (declared in ``include/ernie_kv.h``).

The library is loaded lazily on first use.  There is no fallback: if the
compiled library is missing or fails to load, every op raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libernie_kv.so"

P = c_void_p
I32 = c_int32
I64 = c_int64
F32 = c_float

# name -> (restype, argtypes); mirrors include/ernie_kv.h
SIGNATURES: dict[str, tuple] = {
    "ekv_abi_version": (I32, []),
    "ekv_kv_append_quant": (I32, [P, I64, I32, I32, P, P, I64, I64, P]),
    "ekv_indexer_k_insert": (I32, [P, I64, I32, P, P, I64, I64, P]),
    "ekv_hca_compress": (
        I32,
        [P, I64, P, P, I32, I32, I32, P, P, I32, P, P, F32, P, I32, P, I32, P, I64, I64, P],
    ),
    "ekv_hca_append": (
        I32,
        [P, I64, P, I64, I32, I32, P, P, P, P, I32, P, I64, I64, P, I32, I32, P, P, I32, P],
    ),
    "ekv_hca_append_bf16": (
        I32,
        [P, I64, P, I64, I32, I32, P, P, P, P, I32, P, I64, I64, P, I32, I32, P, P, I32, P],
    ),
    "ekv_hca_write": (
        I32,
        [P, I64, P, I64, I32, I32, P, P, P, P, I32, I32, P, P, I32, P, P, F32, P, I32, P, I32, P, I32, I32, P, I64,
         I64, P, I64, P],
    ),
    "ekv_hca_write_workspace_size": (I64, [I32, I32]),
    "ekv_hca_write_step": (
        I32,
        [P, I64, P, I64, I32, I32, P, P, P, P, I32, I32, P, P, I32, P, P, F32, P, I32, P, I32, P, I32, I32, P, I64,
         I64, P, I64, I32, P, I64, I32, P, P],
    ),
    "ekv_hca_write_bf16": (
        I32,
        [P, I64, P, I64, I32, I32, P, P, P, P, I32, I32, P, P, I32, P, P, F32, P, I32, P, I32, P, I32, I32, P, I64,
         I64, P, I64, P],
    ),
    "ekv_hca_write_step_bf16": (
        I32,
        [P, I64, P, I64, I32, I32, P, P, P, P, I32, I32, P, P, I32, P, P, F32, P, I32, P, I32, P, I32, I32, P, I64,
         I64, P, I64, I32, P, I64, I32, P, P],
    ),
    "ekv_hca_decode_indices": (I32, [P, P, I32, P, I32, P, I32, I32, I32, P, P, P, I64, I32, P, P]),
    "ekv_merge_swa_topk": (I32, [P, I64, P, I64, P, I32, I32, I32, I32, P]),
    "ekv_hadamard_rows": (I32, [P, I64, P, I64, I32, I32, P]),
    "ekv_indexer_prep": (I32, [P, I64, I64, P, I64, I32, I32, P, P, F32, P, I32, P, P, P, P]),
    "ekv_indexer_q_quant": (I32, [P, I64, I64, P, I32, I64, I32, I32, P, P, P, P]),
    "ekv_indexer_windowed_lengths": (I32, [P, I32, I32, P, P]),
    "ekv_dsa_decode_prologue": (I32, [P, I64, P, I64, I64, P, I64, I32, P, I64, I64, P, I32, P, I64, I64, P, I32,
                                      I64, I32, P, P, P, P, I32, P, P, P, F32, P, I32, P]),
    "ekv_indexer_score": (I32, [P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, P]),
    "ekv_topk_select": (I32, [P, I64, P, I32, I32, P, I64, I32, P]),
    "ekv_indexer_topk_workspace_size": (I64, [I32, I32]),
    "ekv_indexer_filter": (I32, [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, I32, P, I64, P]),
    "ekv_indexer_select": (I32, [P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, I32, P, I64, P, I64, I32, P, I32, I32, P]),
    "ekv_indexer_topk": (I32, [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, I32, P, I64, P]),
    "ekv_indexer_topk_merged": (
        I32,
        [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, I32, P, I64, P, I64, I32, P, I32, I32, P],
    ),
    "ekv_dsa_decode_prologue_folds": (I32, [I32, I32]),
    "ekv_dsa_decode_prologue_topk_merged": (
        I32,
        [P, I64, P, I64, I64, P, I64, I32, P, I64, I64, P, I32, P, I64, I64, P, I32, I64, I32, P, P, P, P, I32, I32, P,
         P, P, F32, P, I32, P, I64, P, I32, P, I64, I32, P, I64, P, I64, I32, I32, P],
    ),
    "ekv_indexer_topk_counter_bytes": (I64, []),
    "ekv_indexer_set_spin_limit": (I32, [I32]),
    "ekv_sparse_mla_decode_workspace_size": (I64, [I32, I32, I32]),
    "ekv_sparse_mla_decode": (
        I32,
        [P, I64, I64, I32, I32, I32, P, I32, I64, I64, P, I64, I32, P, P, I64, P, P, F32, P, I64, I64, P, I64, P, I64, P],
    ),
    "ekv_fp8_digit_table": (I32, [P, P]),
    "ekv_sparse_mla_decode_noalloc": (
        I32,
        [P, I64, I64, I32, I32, I32, P, I32, I64, I64, P, I64, I32, P, P, I64, P, P, F32, P, I64, I64, P, I64, P],
    ),
    "ekv_indexer_filter_dots": (I32, [P, P, I32, P, P]),
    "ekv_sigmoid_mul_quant_fp8": (I32, [P, I64, P, I64, I32, I32, P, I64, P, I64, P]),
    "ekv_vha_inv_rope_fp8_quant": (I32, [P, I64, I64, I32, I32, P, P, P, I64, I32, I32, I32, P, P, I32, P]),
    "ekv_mxfp4_quant": (I32, [P, I64, I64, I32, I32, I32, P, I64, P, I64, P]),
    "ekv_indexer_q_quant_fp4": (I32, [P, I64, I64, P, I32, I64, I32, I32, P, P, P, P]),
    "ekv_indexer_k_insert_fp4": (I32, [P, I64, I32, P, P, I64, I64, P]),
    "ekv_indexer_store_fp4": (I32, [P, I64, P, I64, I32, P, P, I64, I64, P]),
    "ekv_dsa_decode_prologue_fp4": (I32, [P, I64, P, I64, I64, P, I64, I32, P, I64, I64, P, I32, P, I64, I64, P, I32,
                                          I64, I32, P, P, P, P, I32, P, P, P, F32, P, I32, P]),
    "ekv_indexer_score_fp4": (I32, [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, P]),
    "ekv_indexer_filter_fp4": (I32, [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, I32, P, I64, P]),
    "ekv_indexer_select_fp4": (
        I32,
        [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, I32, P, I64, P, I64, I32, P, I32, I32, P],
    ),
    "ekv_indexer_topk_fp4": (I32, [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, I32, P, I64, P]),
    "ekv_indexer_topk_merged_fp4": (
        I32,
        [P, P, P, P, I64, I64, P, I64, P, P, I32, I32, P, I64, I32, P, I64, P, I64, I32, P, I32, I32, P],
    ),
    "ekv_indexer_filter_dots_fp4": (I32, [P, P, P, P, I32, P, P]),
    "ekv_export_fp8_ds_mla_pages": (I32, [P, I64, I64, P, I32, P, I64, I64, P, P]),
    "ekv_import_fp8_ds_mla_pages": (I32, [P, I64, I64, P, I32, P, I64, I64, P, P]),
}

_lib = None


class EkvError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the library (once) and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise EkvError(
            f"{LIB_PATH} is missing: build it with `python -m ernie_kv.build` "
            "(the KV-cache ops have no CPU fallback)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    lib.ekv_last_error.restype = ctypes.c_char_p
    lib.ekv_last_error.argtypes = []
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call an entry point and raise on a nonzero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.ekv_last_error().decode(errors="replace")
        raise EkvError(f"{name} failed ({rc}): {msg}")


def exported_symbols() -> list[str]:
    return sorted([*SIGNATURES, "ekv_last_error"])
