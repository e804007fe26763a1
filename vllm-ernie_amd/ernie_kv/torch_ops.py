"""The path's ops as ``torch.ops.ernie_kv.*`` (``import ernie_kv.torch_ops``).

The plugin's adapters call the KV-path kernels as torch operators: the
latent append, the HCA cache write (append, window ring, compressor state,
every completed 128-token span compressed), the indexer K insert, the
indexer top-k, the window merge and the sparse MLA decode with the sink.
Each operator here is a ``torch.library.custom_op`` over the same
``ernie_kv.ops`` wrapper the layers call: the caller owns every output,
the operator writes it in place on the current stream and returns nothing,
and the schema names the tensors it writes, so the dispatcher (and
``torch.compile``, through each operator's fake implementation) sees the
mutation.  Registration needs no GPU; calling needs the HIP library, which
fails loudly when it is missing.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import ops

_NS = "ernie_kv"


@torch.library.custom_op(f"{_NS}::kv_append_quant", mutates_args=("cache",))
def kv_append_quant(rows: torch.Tensor, slot_mapping: torch.Tensor, cache: torch.Tensor) -> None:
    """Latent rows [T, D] bf16 -> fp8 page rows at slot_mapping (negative: skipped)."""
    ops.kv_append_quant(rows, slot_mapping, cache)


@torch.library.custom_op(f"{_NS}::indexer_k_insert", mutates_args=("kcache",))
def indexer_k_insert(k: torch.Tensor, slot_mapping: torch.Tensor, kcache: torch.Tensor) -> None:
    """Indexer keys [T, 128] bf16 -> 132-byte fp8 rows (values, then the fp32 scale) of their pages."""
    ops.indexer_k_insert(k, slot_mapping, kcache)


@torch.library.custom_op(f"{_NS}::hca_write", mutates_args=("pool", "state", "workspace"))
def hca_write(latent: torch.Tensor, kv_score: torch.Tensor, slot_mapping: torch.Tensor, positions: torch.Tensor,
              token_seq: torch.Tensor, qsl: torch.Tensor, max_query_len: int, state: Optional[torch.Tensor],
              state_slot: Optional[torch.Tensor], ape: torch.Tensor, norm_w: torch.Tensor, eps: float,
              cos_sin: torch.Tensor, comp_block_table: torch.Tensor, ring_pages: Optional[torch.Tensor],
              ring: int, pool: torch.Tensor, workspace: Optional[torch.Tensor] = None) -> None:
    """The HCA cache write of a call: rows, window ring, compressor state
    ring, and every 128-token span the call completes compressed into its
    compressed slot (fp8 pages, or bf16 rows for a bf16 pool)."""
    ops.hca_write(latent, kv_score, slot_mapping, positions, token_seq, qsl, max_query_len, state, state_slot, ape,
                  norm_w, eps, cos_sin, comp_block_table, ring_pages, ring, pool, workspace=workspace)


@torch.library.custom_op(f"{_NS}::hca_write_step",
                         mutates_args=("pool", "state", "out", "lengths", "workspace"))
def hca_write_step(latent: torch.Tensor, kv_score: torch.Tensor, slot_mapping: torch.Tensor, positions: torch.Tensor,
                   token_seq: torch.Tensor, qsl: torch.Tensor, max_query_len: int, state: Optional[torch.Tensor],
                   state_slot: Optional[torch.Tensor], ape: torch.Tensor, norm_w: torch.Tensor, eps: float,
                   cos_sin: torch.Tensor, comp_block_table: torch.Tensor, ring_pages: torch.Tensor, ring: int,
                   pool: torch.Tensor, window: int, out: torch.Tensor, lengths: torch.Tensor,
                   workspace: Optional[torch.Tensor] = None) -> None:
    """``hca_write`` and each query row's decode index row (its compressed
    entries, then its window) into ``out`` / ``lengths``."""
    ops.hca_write_step(latent, kv_score, slot_mapping, positions, token_seq, qsl, max_query_len, state, state_slot,
                       ape, norm_w, eps, cos_sin, comp_block_table, ring_pages, ring, pool, window, out, lengths,
                       workspace=workspace)


@torch.library.custom_op(f"{_NS}::indexer_topk", mutates_args=("topk_out", "workspace"))
def indexer_topk(q_fp8: torch.Tensor, q_digits: torch.Tensor, w: torch.Tensor, kcache: torch.Tensor,
                 block_table: torch.Tensor, req_ids: torch.Tensor, lengths: torch.Tensor, max_len: int,
                 topk_out: torch.Tensor, workspace: torch.Tensor) -> None:
    """Exact top-k of the lightning-indexer scores over s < lengths[t], in
    ascending token order, lowest index first on ties, -1 padded."""
    ops.indexer_topk(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, max_len, topk_out, workspace)


@torch.library.custom_op(f"{_NS}::indexer_topk_merged", mutates_args=("topk_out", "workspace", "merged"))
def indexer_topk_merged(q_fp8: torch.Tensor, q_digits: torch.Tensor, w: torch.Tensor, kcache: torch.Tensor,
                        block_table: torch.Tensor, req_ids: torch.Tensor, lengths: torch.Tensor, max_len: int,
                        topk_out: torch.Tensor, workspace: torch.Tensor, merged: torch.Tensor,
                        positions: torch.Tensor, window: int, merged_slots: bool = False) -> None:
    """``indexer_topk`` and ``merge_swa_topk`` of its result in one call."""
    ops.indexer_topk_merged(q_fp8, q_digits, w, kcache, block_table, req_ids, lengths, max_len, topk_out, workspace,
                            merged=merged, positions=positions, window=window, merged_slots=merged_slots)


@torch.library.custom_op(f"{_NS}::merge_swa_topk", mutates_args=("out",))
def merge_swa_topk(topk_indices: torch.Tensor, out: torch.Tensor, positions: torch.Tensor, window: int) -> None:
    """[topk[:n] | seq - window .. seq - 1 | -1 ...] per row (attention.py:606-641)."""
    ops.merge_swa_topk(topk_indices, out, positions, window)


@torch.library.custom_op(f"{_NS}::sparse_mla_decode", mutates_args=("out", "lse", "workspace"))
def sparse_mla_decode(q: torch.Tensor, cache: torch.Tensor, indices: torch.Tensor, scale: float, out: torch.Tensor,
                      lse: Optional[torch.Tensor] = None, sinks: Optional[torch.Tensor] = None,
                      lengths: Optional[torch.Tensor] = None, block_table: Optional[torch.Tensor] = None,
                      req_ids: Optional[torch.Tensor] = None, cache_bf16: bool = False,
                      workspace: Optional[torch.Tensor] = None) -> None:
    """Sparse MLA decode with the attention sink in the denominator:
    q [T, H, D] bf16 over the gathered rows of ``indices`` -> out [T, H, 512]
    bf16 and the natural-log lse [T, H]."""
    ops.sparse_mla_decode(q, cache, indices, scale, out, lse, sinks=sinks, lengths=lengths, block_table=block_table,
                          req_ids=req_ids, cache_bf16=cache_bf16, workspace=workspace)


OPS = ("kv_append_quant", "indexer_k_insert", "hca_write", "hca_write_step", "indexer_topk", "indexer_topk_merged",
       "merge_swa_topk", "sparse_mla_decode")


# Fake (meta) implementations: every operator only writes tensors the caller
# passed, so under tracing (torch.compile, FakeTensorMode) it produces
# nothing and launches nothing.
def _no_output(*args, **kwargs) -> None:
    return None


for _name in OPS:
    globals()[_name].register_fake(_no_output)
