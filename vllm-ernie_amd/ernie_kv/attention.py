"""Drop-in mirror of the reference plugin's KV-cache-path interface.

Mirrors names, argument meaning and error behaviour of
``src/vllm_ernie/models/ernie5_5/nvidia/attention.py`` for the attention
KV-cache hot path; every array op is a HIP kernel of ``libernie_kv.so``
(through ``ernie_kv.ops``).  vLLM itself is not a dependency: the few vLLM
types the reference subclasses (``MultipleOf``, ``KVCacheLayout``, the KV
cache spec, the indexer / FlashMLA metadata) are given minimal stand-ins here
with the fields the path reads.
"""

from __future__ import annotations

import dataclasses
import enum
import math
from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Any

import torch

from . import ops

DSA_BLOCK_SIZE = 64  # attention.py:97-98
INDEXER_QUANT_BLOCK = 128  # attention.py:99


# --------------------------------------------------------------------------- vLLM stand-ins
@dataclass(frozen=True)
class MultipleOf:
    """Kernel block-size constraint (vllm.v1.attention.backend.MultipleOf)."""

    base: int


class KVCacheLayout(enum.Enum):
    NHD = "NHD"
    HND = "HND"
    BLNHC = "BLNHC"
    BLHNC = "BLHNC"


@dataclass
class KVCacheSpec:
    """Fields of vLLM's KV cache spec this path reads and rewrites."""

    block_size: int
    num_kv_heads: int = 1
    head_size: int = 576
    dtype: Any = torch.uint8
    block_stride_alignment: int = 1


# --------------------------------------------------------------------------- helpers
def hadamard_rows(x: torch.Tensor) -> torch.Tensor:
    """Hadamard transform per 128-wide row (attention.py:102-108)."""
    return ops.hadamard_rows(x)


def merge_swa_topk(
    topk_indices: torch.Tensor, out: torch.Tensor, positions: torch.Tensor, window: int
) -> None:
    """Write each top-k row followed by the sliding window into ``out``
    (attention.py:606-641): ``[topk[:n] | seq-w .. seq-1 | -1 ...]``."""
    ops.merge_swa_topk(topk_indices, out, positions, window)


def packed_block_stride_alignment(vllm_config) -> int:
    """Byte alignment of the shared block stride (attention.py:561-571)."""
    hf_config = vllm_config.model_config.hf_config
    hca_row = hf_config.head_dim * 2
    dsa_row = (hf_config.mla_kv_lora_rank + hf_config.mla_qk_rope_head_dim) * 2
    return math.lcm(512, hca_row, dsa_row)


def _dsa_page_spec(spec: KVCacheSpec, vllm_config) -> KVCacheSpec:
    return dataclasses.replace(
        spec, block_size=DSA_BLOCK_SIZE, block_stride_alignment=packed_block_stride_alignment(vllm_config)
    )


def _dsa_kernel_block_sizes(kv_cache_spec=None) -> list[int | MultipleOf]:
    return [MultipleOf(DSA_BLOCK_SIZE)]


def _check_attn_tp(config, tp_size: int = 1) -> None:
    """TP must divide the head groups (attention.py:111-118)."""
    for name in ("o_groups", "num_attention_heads", "hybrid_mla_num_attention_heads"):
        if getattr(config, name) % tp_size:
            raise ValueError(
                f"ERNIE 5.5 attention TP size {tp_size} must divide {name}={getattr(config, name)}."
            )


# --------------------------------------------------------------------------- sparse MLA
class FlashMLASparseImplBase:
    """Minimal base: the fields the sink impl reads."""

    def __init__(self, num_heads: int, head_size: int, scale: float, kv_cache_dtype: str = "fp8",
                 fp8_decode_padded_heads: int | None = None, prefill_padding: int = 16, **_: Any):
        self.num_heads = num_heads
        self.head_size = head_size
        self.softmax_scale = scale
        self.kv_cache_dtype = kv_cache_dtype
        self.fp8_decode_padded_heads = fp8_decode_padded_heads or num_heads
        self.prefill_padding = prefill_padding
        self._workspace: torch.Tensor | None = None


class Ernie5_5FlashMLASparseImpl(FlashMLASparseImplBase):
    """Sparse MLA impl passing the per-head sink to the kernel (attention.py:701-790).

    The sink enters the softmax denominator; padded heads get a -inf sink (a
    no-op).  ``lse`` is the natural-log sum of exp of the real scores.
    """

    def __init__(self, *args, **kwargs) -> None:
        self.sinks: torch.Tensor = kwargs.pop("sinks")
        super().__init__(*args, **kwargs)

    def _padded_sinks(self, kernel_heads: int) -> torch.Tensor:
        num_heads = self.sinks.shape[0]
        if kernel_heads == num_heads:
            return self.sinks
        padded = self.sinks.new_full((kernel_heads,), float("-inf"))
        padded[:num_heads] = self.sinks
        return padded

    def _ws(self, nbytes: int, device) -> torch.Tensor:
        if self._workspace is None or self._workspace.numel() < nbytes:
            self._workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        return self._workspace

    def _fp8_flash_mla_kernel(
        self, q: torch.Tensor, kv_c_and_k_pe_cache: torch.Tensor, topk_indices: torch.Tensor,
        kernel_metadata: Any = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """q [batch, seq_len, heads, 576]; cache uint8 pages; global indices
        [batch, seq_len, width] (the reference passes a dummy block table)."""
        b, s, h, d = q.shape
        flat_q = q.reshape(b * s, h, d)
        idx = topk_indices.reshape(b * s, -1).to(torch.int32)
        out = torch.empty((b * s, h, 512), dtype=q.dtype, device=q.device)
        lse = torch.empty((b * s, h), dtype=torch.float32, device=q.device)
        cache = kv_c_and_k_pe_cache.view(torch.uint8)
        cache = cache.reshape(cache.shape[0], -1)
        ws = self._ws(ops._lib.load().ekv_sparse_mla_decode_workspace_size(b * s, h, idx.shape[1]), q.device)
        ops.sparse_mla_decode(flat_q, cache, idx, self.softmax_scale, out, lse,
                              sinks=self._padded_sinks(h), workspace=ws)
        return out.view(b, s, h, 512), lse.view(b, s, h)

    def _bf16_flash_mla_kernel(
        self, q: torch.Tensor, kv_c_and_k_pe_cache: torch.Tensor, topk_indices: torch.Tensor,
        topk_length: torch.Tensor | None = None, actual_num_heads: int | None = None,
        out: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        num_tokens = q.shape[0]
        cache = kv_c_and_k_pe_cache.view(-1, 1, kv_c_and_k_pe_cache.shape[-1])
        if actual_num_heads is None:
            actual_num_heads = q.shape[1]
        padded = ((actual_num_heads + 15) // 16) * 16
        if q.shape[1] < padded:
            q_padded = q.new_zeros((num_tokens, padded, q.shape[2]))
            q_padded[:, :actual_num_heads] = q
            q = q_padded
        heads = q.shape[1]
        res = out if out is not None else torch.empty((num_tokens, heads, 512), dtype=q.dtype, device=q.device)
        lse = torch.empty((num_tokens, heads), dtype=torch.float32, device=q.device)
        idx = topk_indices.view(num_tokens, -1).to(torch.int32)
        ws = self._ws(ops._lib.load().ekv_sparse_mla_decode_workspace_size(num_tokens, heads, idx.shape[1]), q.device)
        ops.sparse_mla_decode(q, cache.view(-1, cache.shape[-1]), idx, self.softmax_scale, res, lse,
                              sinks=self._padded_sinks(heads), lengths=topk_length, cache_bf16=True,
                              workspace=ws)
        return res[:, :actual_num_heads], lse[:, :actual_num_heads]


class Ernie5_5FlashMLASparseBackend:
    """Keeps the parent's name (attention.py:792-805)."""

    get_supported_kernel_block_sizes = staticmethod(_dsa_kernel_block_sizes)

    @staticmethod
    def get_name() -> str:
        return "FLASHMLA_SPARSE"

    @staticmethod
    def get_impl_cls() -> type[Ernie5_5FlashMLASparseImpl]:
        return Ernie5_5FlashMLASparseImpl

    @classmethod
    def supports_sink(cls) -> bool:
        return True


# --------------------------------------------------------------------------- indexer metadata
@dataclass
class IndexerPrefillChunk:
    cu_seqlen_ks: torch.Tensor
    cu_seqlen_ke: torch.Tensor


@dataclass
class IndexerPrefill:
    chunks: list = field(default_factory=list)


@dataclass
class IndexerDecode:
    seq_lens: torch.Tensor
    block_table: torch.Tensor | None = None
    schedule_metadata: Any = None
    indices: Any = None


@dataclass
class IndexerMetadata:
    prefill: IndexerPrefill | None = None
    decode: IndexerDecode | None = None


class Ernie5_5IndexerMetadataBuilder:
    """Excludes the trailing sliding window from the indexer KV range
    (attention.py:644-691).  ``base_build`` stands in for the vLLM parent's
    ``build`` and must return an ``IndexerMetadata``."""

    def __init__(self, window: int, max_num_reqs: int, device, base_build=None) -> None:
        self.window = window
        self.base_build = base_build
        self.decode_seq_lens_buffer = torch.zeros(max_num_reqs, dtype=torch.int32, device=device)
        self.windowed_seq_lens_buffer = torch.zeros_like(self.decode_seq_lens_buffer)
        self._positions = torch.zeros(max_num_reqs, dtype=torch.int64, device=device)

    def build(self, common_prefix_len: int, common_attn_metadata, fast_build: bool = False) -> IndexerMetadata:
        metadata = self.base_build(common_prefix_len, common_attn_metadata, fast_build)
        if metadata.prefill is not None:
            metadata.prefill.chunks = [
                dataclasses.replace(
                    chunk, cu_seqlen_ke=torch.maximum(chunk.cu_seqlen_ke - self.window, chunk.cu_seqlen_ks)
                )
                for chunk in metadata.prefill.chunks
            ]
        if metadata.decode is not None:
            seq_lens = metadata.decode.seq_lens
            n = seq_lens.numel()
            windowed = self.windowed_seq_lens_buffer[:n].view(seq_lens.shape)
            # max(seq_len - window, 0) == max((seq_len - 1) + 1 - window, 0)
            pos = self._positions[:n]
            pos.copy_(seq_lens.reshape(-1).to(torch.int64) - 1)
            ops.indexer_windowed_lengths(pos, self.window, windowed.reshape(-1))
            metadata.decode = dataclasses.replace(metadata.decode, seq_lens=windowed)
        return metadata


class Ernie5_5IndexerBackend:
    """Keeps the parent's name (attention.py:807-820)."""

    get_supported_kernel_block_sizes = staticmethod(_dsa_kernel_block_sizes)

    @staticmethod
    def get_name() -> str:
        return "DEEPSEEK_V32_INDEXER"

    @classmethod
    def supported_kv_cache_layouts(cls) -> tuple[KVCacheLayout, ...]:
        return (KVCacheLayout.BLNHC, KVCacheLayout.BLHNC)

    @staticmethod
    def get_builder_cls() -> type[Ernie5_5IndexerMetadataBuilder]:
        return Ernie5_5IndexerMetadataBuilder


class Ernie5_5IndexerCache:
    """Indexer K cache: 132-byte fp8 rows in 64-token pages (attention.py:823-828, 929-941)."""

    def __init__(self, head_dim: int, dtype, prefix: str, cache_config=None) -> None:
        self.head_dim = head_dim
        self.dtype = dtype
        self.prefix = prefix
        self.kv_cache: torch.Tensor | None = None

    def get_kv_cache_spec(self, vllm_config) -> KVCacheSpec:
        base = KVCacheSpec(block_size=vllm_config.cache_config.block_size, head_size=self.head_dim, dtype=self.dtype)
        return _dsa_page_spec(base, vllm_config)

    def get_attn_backend(self) -> type[Ernie5_5IndexerBackend]:
        return Ernie5_5IndexerBackend


class Ernie5_5MLAAttention:
    """Sparse MLA layer whose KV cache uses the DSA page size (attention.py:1028-1032)."""

    def __init__(self, head_size: int = 576, cache_block_size: int = 64) -> None:
        self.head_size = head_size
        self.cache_block_size = cache_block_size

    def get_kv_cache_spec(self, vllm_config) -> KVCacheSpec:
        base = KVCacheSpec(block_size=vllm_config.cache_config.block_size, head_size=self.head_size)
        return _dsa_page_spec(base, vllm_config)


def _check_sink_backend(head_size: int, kv_cache_dtype: str) -> None:
    """Validates the sink-capable sparse backend (attention.py:1035-1057)."""
    reasons = []
    if head_size not in (512, 576):
        reasons.append(f"head_size {head_size} not supported")
    if not (kv_cache_dtype.startswith("fp8") or kv_cache_dtype in ("auto", "bfloat16")):
        reasons.append(f"kv_cache_dtype {kv_cache_dtype} not supported")
    if reasons:
        raise RuntimeError("ERNIE 5.5 DSA needs the sink-capable FLASHMLA_SPARSE backend: " + ", ".join(reasons))


# --------------------------------------------------------------------------- HCA layer class choice
class Ernie5_5HCAFlashInferAttention:
    """HCA layer on a bf16 KV row (attention.py:542-545)."""

    kv_cache_dtype = "bfloat16"


class Ernie5_5HCAFlashMLAAttention:
    """HCA layer on an fp8 KV row (attention.py:548-551)."""

    kv_cache_dtype = "fp8"


def select_ernie5_5_hca_cls(kv_cache_dtype: str):
    """fp8 caches -> the FlashMLA class, else FlashInfer (attention.py:554-558)."""
    if kv_cache_dtype.startswith("fp8"):
        return Ernie5_5HCAFlashMLAAttention
    return Ernie5_5HCAFlashInferAttention


def simple_vllm_config(head_dim=512, mla_kv_lora_rank=512, mla_qk_rope_head_dim=64, block_size=64):
    """A SimpleNamespace config with the fields the KV-spec helpers read."""
    hf = SimpleNamespace(head_dim=head_dim, mla_kv_lora_rank=mla_kv_lora_rank,
                         mla_qk_rope_head_dim=mla_qk_rope_head_dim)
    return SimpleNamespace(model_config=SimpleNamespace(hf_config=hf),
                           cache_config=SimpleNamespace(block_size=block_size))
