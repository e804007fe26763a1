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

import contextlib
import copy
import dataclasses
import enum
import math
from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Any

import torch

from . import ops
from . import torch_ops  # noqa: F401  (registers the path's operators as torch.ops.ernie_kv.*)

DSA_BLOCK_SIZE = 64  # attention.py:97-98
INDEXER_QUANT_BLOCK = 128  # attention.py:99
MXFP4_BLOCK_SIZE = 32  # values per UE8M0 scale of the MXFP4 indexer cache (attention.py:47, 932)


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
        """q [batch, seq_len, heads, 576]; cache uint8 pages; indices
        [batch, seq_len, width].  As in the reference (dummy block table),
        the indices are global cache slots; a ``kernel_metadata`` carrying
        ``block_table`` and ``req_ids`` instead marks them request-local, and
        the kernel converts them through the block table.  Heads are padded
        with zero q rows and -inf sinks to ``fp8_decode_padded_heads``.

        The cache must hold this library's rows (d fp8 codes per row, then
        the page's fp32 scales).  Upstream's ``fp8_ds_mla`` pages (656-byte
        rows) have the same 46,080-byte page stride, so the format is taken
        from ``kv_cache_dtype`` and an ``fp8_ds_mla`` cache is refused rather
        than misread: ``ops.import_fp8_ds_mla_pages`` converts its pages."""
        if self.kv_cache_dtype == "fp8_ds_mla":
            raise ValueError("_fp8_flash_mla_kernel reads 580-byte fp8 rows with per-token fp32 scales; this cache "
                             "holds fp8_ds_mla pages (656-byte rows): convert them with "
                             "ops.import_fp8_ds_mla_pages")
        b, s, h, d = q.shape
        padded = max(self.fp8_decode_padded_heads, h)
        padded = (padded + 15) // 16 * 16
        flat_q = q.reshape(b * s, h, d)
        if padded > h:
            qp = q.new_zeros((b * s, padded, d))
            qp[:, :h] = flat_q
            flat_q = qp
        idx = topk_indices.reshape(b * s, -1)
        if idx.dtype != torch.int32:
            idx = idx.to(torch.int32)
        out = torch.empty((b * s, padded, 512), dtype=q.dtype, device=q.device)
        lse = torch.empty((b * s, padded), dtype=torch.float32, device=q.device)
        cache = kv_c_and_k_pe_cache.view(torch.uint8)
        cache = cache.reshape(cache.shape[0], -1)
        ws = self._ws(ops._lib.load().ekv_sparse_mla_decode_workspace_size(b * s, padded, idx.shape[1]), q.device)
        bt = getattr(kernel_metadata, "block_table", None)
        req = getattr(kernel_metadata, "req_ids", None)
        ops.sparse_mla_decode(flat_q, cache, idx, self.softmax_scale, out, lse, sinks=self._padded_sinks(padded),
                              block_table=bt, req_ids=req, workspace=ws)
        return out[:, :h].reshape(b, s, h, 512), lse[:, :h].reshape(b, s, h)

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
    ``build`` and must return an ``IndexerMetadata``.  The decode seq_lens
    buffers hold ``max_num_reqs * max_query_len`` entries: decode seq_lens
    are ``[num_reqs]``, or ``[num_reqs, next_n]`` with draft tokens."""

    def __init__(self, window: int, max_num_reqs: int, device, base_build=None, max_query_len: int = 1) -> None:
        self.window = window
        self.base_build = base_build
        n = max_num_reqs * max(1, max_query_len)
        self.decode_seq_lens_buffer = torch.zeros(n, dtype=torch.int32, device=device)
        self.windowed_seq_lens_buffer = torch.zeros_like(self.decode_seq_lens_buffer)
        self._positions = torch.zeros(n, dtype=torch.int64, device=device)

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
            if n > self.windowed_seq_lens_buffer.numel():
                raise ValueError(f"decode seq_lens has {n} entries; the builder holds "
                                 f"{self.windowed_seq_lens_buffer.numel()} (max_num_reqs * max_query_len)")
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


def _check_sink_backend(head_size: int, kv_cache_dtype: str) -> None:
    """Validates the sink-capable sparse backend (attention.py:1035-1057)."""
    reasons = []
    if head_size not in (512, 576):
        reasons.append(f"head_size {head_size} not supported")
    if not (kv_cache_dtype.startswith("fp8") or kv_cache_dtype in ("auto", "bfloat16")):
        reasons.append(f"kv_cache_dtype {kv_cache_dtype} not supported")
    if reasons:
        raise RuntimeError("ERNIE 5.5 DSA needs the sink-capable FLASHMLA_SPARSE backend: " + ", ".join(reasons))


# --------------------------------------------------------------------------- forward context
@dataclass
class ForwardContext:
    """Stand-in for vLLM's forward context: the per-layer attention
    metadata of the step, keyed by layer (cache) prefix."""

    attn_metadata: dict = field(default_factory=dict)


_forward_context: ForwardContext | None = None


@contextlib.contextmanager
def set_forward_context(attn_metadata: dict):
    """Makes ``attn_metadata`` the step's metadata for the layers' forwards."""
    global _forward_context
    prev = _forward_context
    _forward_context = ForwardContext(attn_metadata)
    try:
        yield _forward_context
    finally:
        _forward_context = prev


def get_forward_context() -> ForwardContext:
    if _forward_context is None:
        raise RuntimeError("no forward context: run the layer inside set_forward_context(...)")
    return _forward_context


@dataclass
class DSAStepMetadata:
    """What a DSA layer reads from the step's metadata: both of its caches
    (indexer K and latent) use 64-token pages named by one block table."""

    slot_mapping: torch.Tensor  # [T] int64, negative = skip
    block_table: torch.Tensor   # [B, P] int32
    req_ids: torch.Tensor       # [T] int32, query row -> request (row of block_table)
    max_seq_len: int            # tokens of the longest request
    max_query_len: int = 0      # most query rows of one request in the step (0: not given)


@dataclass
class HCAStepMetadata:
    """What an HCA layer reads from the step's metadata: the latent rows'
    slots, each request's query rows, and the compressed / window-ring /
    compressor-state placement of each request."""

    slot_mapping: torch.Tensor      # [T] int64
    query_start_loc: torch.Tensor   # [B + 1] int32
    token_seq: torch.Tensor         # [T] int32, query row -> request
    max_query_len: int
    comp_block_table: torch.Tensor  # [B, CP] int32 pages of the compressed entries
    ring_pages: torch.Tensor        # [B, R / 64] int32 pages of the window ring
    state_slot: torch.Tensor        # [B] int32 row of the compressor state ring
    max_seq_len: int


_rope_tables: dict = {}


def rope_cos_sin_table(rot_dim: int, theta: float, max_position: int, device) -> torch.Tensor:
    """fp32 ``[max_position, rot_dim]`` cos | sin table (plain RoPE,
    ``inv_freq_i = theta ** (-2i / rot_dim)``), shared per (theta, size,
    device) across layers."""
    key = (rot_dim, float(theta), int(max_position), str(device))
    t = _rope_tables.get(key)
    if t is None:
        inv = theta ** (-torch.arange(rot_dim // 2, dtype=torch.float64) * 2.0 / rot_dim)
        ang = torch.arange(max_position, dtype=torch.float64)[:, None] * inv[None, :]
        t = torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).to(torch.float32).to(device).contiguous()
        _rope_tables[key] = t
    return t


_topk_workspaces: dict = {}


def _indexer_workspace(rows: int, max_len: int, device) -> torch.Tensor:
    """A zero-filled indexer top-k workspace per device, grown on demand
    (calls leave its counters zero, so layers share it on one stream)."""
    key = str(device)
    need = ops._lib.load().ekv_indexer_topk_workspace_size(int(rows), int(max_len))
    ws = _topk_workspaces.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
        _topk_workspaces[key] = ws
    return ws


# --------------------------------------------------------------------------- layer building blocks
class Linear(torch.nn.Module):
    """A bias-free linear layer (stand-in for vLLM's parallel linear layers
    at TP = 1): ``weight [out, in]``; returns ``(y, None)`` when
    ``return_bias`` (the vLLM convention the reference's call sites index
    with ``[0]``), else ``y``.  A plain library GEMM outside the KV path."""

    def __init__(self, in_features: int, out_features: int, return_bias: bool = False, device=None,
                 dtype=torch.bfloat16) -> None:
        super().__init__()
        self.input_size, self.output_size = in_features, out_features
        self.return_bias = return_bias
        self.weight = torch.nn.Parameter(torch.empty(out_features, in_features, device=device, dtype=dtype),
                                          requires_grad=False)

    def forward(self, x: torch.Tensor):
        y = x @ self.weight.t()
        return (y, None) if self.return_bias else y


class RMSNorm(torch.nn.Module):
    """``x / sqrt(mean(x^2) + eps) * weight``, computed in fp32 and returned
    in the input dtype (vLLM's RMSNorm)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, device=None, dtype=torch.bfloat16) -> None:
        super().__init__()
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype), requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class InterleavedRotaryEmbedding:
    """RoPE on interleaved pairs (2i, 2i + 1) (``is_neox_style=False``),
    plain frequencies ``theta ** (-2i / rot_dim)``; ``cos_sin_cache`` is the
    ``[max_position, rot_dim]`` cos | sin table (the layout the post-attention
    inverse-RoPE kernel reads).  ``__call__(positions, q, k)`` returns the
    rotated copies, computed in fp32 (torch ops around the KV path)."""

    def __init__(self, rot_dim: int, max_position: int, rope_parameters: dict, device) -> None:
        rope_type = rope_parameters.get("rope_type", "default")
        if rope_type != "default":
            raise NotImplementedError(f"rope_type {rope_type!r}: pass the layer a cos | sin table instead")
        self.rot_dim = rot_dim
        self.cos_sin_cache = rope_cos_sin_table(rot_dim, rope_parameters["rope_theta"], max_position, device)

    @classmethod
    def from_table(cls, cos_sin_cache: torch.Tensor) -> "InterleavedRotaryEmbedding":
        """From a given ``[max_position, rot_dim]`` cos | sin table."""
        self = cls.__new__(cls)
        self.rot_dim = cos_sin_cache.shape[1]
        self.cos_sin_cache = cos_sin_cache.contiguous()
        return self

    def rotate(self, positions: torch.Tensor, x: torch.Tensor, inverse: bool = False) -> torch.Tensor:
        half = self.rot_dim // 2
        cs = self.cos_sin_cache[positions]
        shape = (cs.shape[0],) + (1,) * (x.dim() - 2) + (half,)
        c, s = cs[:, :half].reshape(shape), cs[:, half:].reshape(shape)
        if inverse:
            s = -s
        xf = x.float()
        e, o = xf[..., 0::2], xf[..., 1::2]
        out = torch.stack([e * c - o * s, e * s + o * c], dim=-1).flatten(-2)
        return out.to(x.dtype)

    def __call__(self, positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor):
        return self.rotate(positions, q), self.rotate(positions, k)


_fp8_luts: dict = {}


def _fp8_values(codes: torch.Tensor) -> torch.Tensor:
    """fp32 values of e4m3fn codes (a 256-entry table per device)."""
    key = str(codes.device)
    lut = _fp8_luts.get(key)
    if lut is None:
        lut = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).to(codes.device)
        _fp8_luts[key] = lut
    return lut[codes.view(torch.uint8).long()]


def _ue8m0_bytes(packed: torch.Tensor) -> torch.Tensor:
    """int32 words of four biased exponents -> their 4 bytes (last dim x4)."""
    w = packed.to(torch.int64) & 0xFFFFFFFF
    return torch.stack([(w >> (8 * c)) & 0xFF for c in range(4)], dim=-1).flatten(-2)


def dequant_sigmoid_mul(data: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Values of ``sigmoid_mul_quant_fp8``'s output: 1 x 128 groups scaled
    by ``2 ** (byte - 127)`` (the exponents packed four per int32)."""
    N, hidden = data.shape
    exps = _ue8m0_bytes(scale)[:, : hidden // 128].float() - 127.0
    return _fp8_values(data) * torch.exp2(exps).repeat_interleave(128, dim=1)


def dequant_vha(data: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Values of ``vha_inv_rope_fp8_quant``'s output ``[T, G, hpg * 512]``:
    each head's four 128-wide chunks scaled by their exponent bytes."""
    T, G, width = data.shape
    exps = _ue8m0_bytes(scale).reshape(T, G, -1).float() - 127.0  # [T, G, hpg * 4]
    return _fp8_values(data) * torch.exp2(exps).repeat_interleave(128, dim=2)


def dsa_indexer_uses_fp4(vllm_config) -> bool:
    """Stand-in for vLLM's MXFP4 indexer-cache selector: the
    ``use_fp4_indexer_cache`` flag of ``vllm_config.attention_config``."""
    return bool(getattr(getattr(vllm_config, "attention_config", None), "use_fp4_indexer_cache", False))


def _device_of(vllm_config):
    dc = getattr(vllm_config, "device_config", None)
    return getattr(dc, "device", None) or ("cuda" if torch.cuda.is_available() else "cpu")


def _load(module: torch.nn.Module, weights) -> set:
    """vLLM-style ``load_weights``: copy each ``(name, tensor)`` into the
    parameter or buffer of that name; returns the names loaded."""
    params = dict(module.named_parameters())
    params.update(dict(module.named_buffers()))
    loaded = set()
    for name, w in weights:
        if name not in params:
            raise KeyError(f"{type(module).__name__} has no weight {name!r}")
        params[name].data.copy_(w.to(params[name].dtype))
        loaded.add(name)
    return loaded


# Query rows scored per indexer call: one call's workspace holds
# rows x max_len x 20 bytes, so long prefill chunks run in pieces.
_INDEXER_WORKSPACE_BYTES = 1 << 30


# --------------------------------------------------------------------------- layers
class Ernie5_5Indexer(torch.nn.Module):
    """Lightning indexer scoring the tokens older than the sliding window
    (attention.py:863-984), constructed as the reference's
    ``(vllm_config, config, quant_config, cache_config, topk_indices_buffer,
    swa_topk_buffer, prefix)``.

    ``forward(hidden_states, qr, positions)`` runs the reference's order:
    the two projections (``wq_b`` on ``qr``, ``wk_weights_proj`` on
    ``hidden_states``; plain library GEMMs), then on the HIP library
    ``k_norm`` LayerNorm, NeoX RoPE of dims 0..63, Hadamard, the fp8
    UE8M0 q quant with the weight fold, the K-cache insert and the exact
    top-k of each query row over its first ``position + 1 - window``
    tokens, written to ``indexer_op.topk_indices_buffer[:T]``.
    ``topk_indices_buffer`` (the layer attribute) is the swa buffer the
    sparse MLA reads: the merged rows.  K cache rows are 132 bytes (fp8
    values + fp32 scale) or, with the MXFP4 cache (``dsa_indexer_uses_fp4``),
    68 bytes (MXFP4 values + four E8M0 scales; ``_quantize_fp4``,
    attention.py:986-1025), which the reference allows only without context
    parallelism (:881-892)."""

    def __init__(self, vllm_config, config, quant_config, cache_config, topk_indices_buffer: torch.Tensor | None,
                 swa_topk_buffer: torch.Tensor | None, prefix: str = "") -> None:
        super().__init__()
        self.n_head = config.index_n_heads
        self.head_dim = config.index_head_dim
        self.rope_dim = config.mla_qk_rope_head_dim
        self.use_fp4_kv = dsa_indexer_uses_fp4(vllm_config)
        if self.use_fp4_kv:
            parallel_config = vllm_config.parallel_config
            pcp_size = parallel_config.prefill_context_parallel_size
            dcp_size = parallel_config.decode_context_parallel_size
            if pcp_size != 1 or dcp_size != 1:
                raise NotImplementedError(
                    "ERNIE 5.5 MXFP4 indexer currently requires PCP=DCP=1 "
                    "(prefill_context_parallel_size=1 and decode_context_parallel_size=1). "
                    f"Got PCP={pcp_size}, DCP={dcp_size}.")
        if (self.n_head, self.head_dim, self.rope_dim) != (64, 128, 64):
            raise NotImplementedError("the indexer kernels take 64 heads x 128 dims with a 64-dim rope")
        dev = _device_of(vllm_config)
        self.wq_b = Linear(config.mla_q_lora_rank, self.n_head * self.head_dim, return_bias=True, device=dev)
        self.wk_weights_proj = Linear(config.hidden_size, self.head_dim + self.n_head, return_bias=True, device=dev)
        self.k_norm = torch.nn.LayerNorm(self.head_dim, eps=1e-6, device=dev, dtype=torch.float32)
        self.topk = config.index_topk
        self.window = config.sliding_window
        self.rope_theta = config.mla_rope_parameters["rope_theta"]
        self.max_position = config.max_position_embeddings
        self.weights_scale = self.head_dim ** -0.5 * self.n_head ** -0.5
        self.topk_indices_buffer = swa_topk_buffer
        if self.use_fp4_kv:  # 64 packed values + 4 UE8M0 scales = 68 bytes
            k_cache_head_dim = self.head_dim // 2 + self.head_dim // MXFP4_BLOCK_SIZE
        else:  # 128 fp8 + 4-byte fp32 scale = 132 bytes
            k_cache_head_dim = self.head_dim + self.head_dim // INDEXER_QUANT_BLOCK * 4
        self.k_cache = Ernie5_5IndexerCache(head_dim=k_cache_head_dim, dtype=torch.uint8, prefix=f"{prefix}.k_cache",
                                            cache_config=cache_config)
        self.indexer_op = SimpleNamespace(topk_indices_buffer=topk_indices_buffer, topk_tokens=self.topk)
        self._lengths: torch.Tensor | None = None

    @property
    def k_norm_weight(self) -> torch.Tensor:
        return self.k_norm.weight.detach()

    @property
    def k_norm_bias(self) -> torch.Tensor:
        return self.k_norm.bias.detach()

    def _project(self, hidden_states: torch.Tensor, qr: torch.Tensor):
        q, _ = self.wq_b(qr)
        q = q.view(-1, self.n_head, self.head_dim)
        kw, _ = self.wk_weights_proj(hidden_states)
        k, weights = kw.split([self.head_dim, self.n_head], dim=-1)
        return q, k.contiguous(), weights.contiguous()

    def _prep_args(self, device):
        return (self.k_norm_weight.contiguous(), self.k_norm_bias.contiguous(), self.k_norm.eps,
                rope_cos_sin_table(self.rope_dim, self.rope_theta, self.max_position, device))

    def _lengths_buf(self, T: int, device) -> torch.Tensor:
        if self._lengths is None or self._lengths.numel() < T:
            self._lengths = torch.empty(max(T, 1), dtype=torch.int32, device=device)
        return self._lengths[:T]

    def _topk(self, qa, qb, wf, md: DSAStepMetadata, lengths, positions, merged=None) -> None:
        """Exact top-k of every query row (filter + select, one launch when the
        filter fits one), in row pieces whose workspace fits
        _INDEXER_WORKSPACE_BYTES; with ``merged`` the select also writes
        merge_swa_topk's rows.  ``(qa, qb)`` are the fp8 codes and digit
        planes, or the MXFP4 values and scale words."""
        T = qa.shape[0]
        kcache = self.k_cache.kv_cache
        out = self.indexer_op.topk_indices_buffer
        L = max(int(md.max_seq_len), 1)
        step = max(1, min(T, _INDEXER_WORKSPACE_BYTES // (20 * L)))
        for r0 in range(0, T, step):
            r1 = min(T, r0 + step)
            ws = _indexer_workspace(r1 - r0, L, qa.device)
            args = (kcache, md.block_table, md.req_ids[r0:r1], lengths[r0:r1], L)
            sel = dict(merged=None if merged is None else merged[r0:r1], positions=positions[r0:r1],
                       window=self.window)
            if self.use_fp4_kv:
                ops.indexer_topk_merged_fp4(qa[r0:r1], qb[r0:r1], wf[r0:r1], *args, out[r0:r1, : self.topk], ws,
                                            **sel)
            else:
                ops.indexer_topk_merged(qa[r0:r1], qb[r0:r1], wf[r0:r1], *args, out[r0:r1, : self.topk], ws, **sel)

    def _quantize_fp4(self, q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor, slot_mapping: torch.Tensor):
        """MXFP4 q (values [T, 64, 64], scale words [T, 64]) and the K insert
        of k at ``slot_mapping`` (attention.py:986-1025), plus the fp32 weights
        ``weights * weights_scale`` (:973)."""
        T = q.shape[0]
        num_tokens = min(k.shape[0], slot_mapping.numel())
        if num_tokens:
            ops.indexer_k_insert_fp4(k[:num_tokens], slot_mapping[:num_tokens], self.k_cache.kv_cache)
        return ops.indexer_q_quant_fp4(q.view(T, self.n_head, self.head_dim), weights)

    def forward(self, hidden_states: torch.Tensor, qr: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        md: DSAStepMetadata = get_forward_context().attn_metadata[self.k_cache.prefix]
        T = hidden_states.shape[0]
        q, k, weights = self._project(hidden_states, qr)
        qp, kp = ops.indexer_prep(q, k, *self._prep_args(q.device), positions)
        if self.use_fp4_kv:
            qa, qb, wf = self._quantize_fp4(qp, kp, weights, md.slot_mapping)
        else:
            ops.indexer_k_insert(kp, md.slot_mapping, self.k_cache.kv_cache)
            qa, wf, qb = ops.indexer_q_quant(qp, weights)
        lengths = self._lengths_buf(T, q.device)
        ops.indexer_windowed_lengths(positions, self.window, lengths)
        self._topk(qa, qb, wf, md, lengths, positions)
        return self.indexer_op.topk_indices_buffer[:T]

    def load_weights(self, weights) -> set:
        return _load(self, weights)


class Ernie5_5MLAAttention:
    """Sparse MLA over the DSA latent cache (attention.py:1028-1032 for the
    KV spec; the layer vLLM's MLAAttention provides around the impl).

    Holds the impl (sink-capable sparse decode), the bound latent cache
    (``kv_cache``, fp8 pages of 576-byte rows + fp32 scales) and the
    absorbed-MLA projections split from ``kv_b_proj`` by
    ``process_weights_after_loading``: W_UK maps the nope part of q into the
    512-d latent space, W_UV maps the decode's latent output to the v heads
    (plain batched GEMMs)."""

    def __init__(self, num_heads: int = 64, scale: float = 256 ** -0.5, qk_nope_head_dim: int = 192,
                 qk_rope_head_dim: int = 64, v_head_dim: int = 256, q_lora_rank: int | None = None,
                 kv_lora_rank: int = 512, kv_b_proj: Linear | None = None, cache_config=None, quant_config=None,
                 prefix: str = "", attn_backend=None, use_sparse: bool = True, indexer=None,
                 topk_indices_buffer=None, sinks: torch.Tensor | None = None, head_size: int = 576,
                 cache_block_size: int = 64) -> None:
        self.num_heads = num_heads
        self.head_size = head_size
        self.cache_block_size = cache_block_size
        self.qk_nope_head_dim = qk_nope_head_dim
        self.qk_rope_head_dim = qk_rope_head_dim
        self.v_head_dim = v_head_dim
        self.kv_lora_rank = kv_lora_rank
        self.prefix = prefix
        self.indexer = indexer
        self.topk_indices_buffer = topk_indices_buffer
        self.kv_b_proj = kv_b_proj
        self.kv_cache: torch.Tensor | None = None
        self.W_UK: torch.Tensor | None = None
        self.W_UV_T: torch.Tensor | None = None
        cache_dtype = getattr(cache_config, "cache_dtype", "fp8")
        self.impl = None
        if sinks is not None:
            self.impl = Ernie5_5FlashMLASparseImpl(num_heads, head_size, scale, kv_cache_dtype=cache_dtype,
                                                   sinks=sinks)

    def get_kv_cache_spec(self, vllm_config) -> KVCacheSpec:
        base = KVCacheSpec(block_size=vllm_config.cache_config.block_size, head_size=self.head_size)
        return _dsa_page_spec(base, vllm_config)

    def process_weights_after_loading(self) -> None:
        """W_UK [H, 192, 512] and W_UV^T [H, 512, 256] from kv_b_proj."""
        w = self.kv_b_proj.weight.detach().view(self.num_heads, self.qk_nope_head_dim + self.v_head_dim,
                                                self.kv_lora_rank)
        self.W_UK = w[:, : self.qk_nope_head_dim].contiguous()
        self.W_UV_T = w[:, self.qk_nope_head_dim:].transpose(1, 2).contiguous()

    def absorb_q(self, q: torch.Tensor) -> torch.Tensor:
        """q [T, H, 192 + 64] -> [T, H, 512 + 64]: the nope part through W_UK."""
        if self.W_UK is None:
            self.process_weights_after_loading()
        T = q.shape[0]
        q_nope = q[..., : self.qk_nope_head_dim].transpose(0, 1).contiguous()  # [H, T, 192]
        q_lat = torch.bmm(q_nope, self.W_UK)                                    # [H, T, 512]
        return torch.cat([q_lat.transpose(0, 1), q[..., self.qk_nope_head_dim:]], dim=-1).contiguous().view(
            T, self.num_heads, self.kv_lora_rank + self.qk_rope_head_dim)

    def up_proj(self, o_latent: torch.Tensor) -> torch.Tensor:
        """[T, H, 512] -> [T, H * 256] through W_UV."""
        if self.W_UV_T is None:
            self.process_weights_after_loading()
        T = o_latent.shape[0]
        o = torch.bmm(o_latent.transpose(0, 1).contiguous(), self.W_UV_T)  # [H, T, 256]
        return o.transpose(0, 1).reshape(T, self.num_heads * self.v_head_dim)


class Ernie5_5DSAAttention(torch.nn.Module):
    """MLA layer with a DSA indexer, attention sink, VHA and an output gate
    (attention.py:1059-1226), constructed as the reference's
    ``(vllm_config, prefix, topk_indices_buffer, swa_topk_buffer)``.

    ``forward(positions, hidden_states, llama_4_scaling=None)`` follows the
    reference: fused_qkv_a_proj, q_a_layernorm, o_gate, q_b_proj,
    kv_a_layernorm and the interleaved RoPE of the q / k rope parts (torch
    ops around the path), then ``_indexer_and_attn`` on the HIP library,
    then VHA and the gated ``wo_b``.  ``_indexer_and_attn(hidden_states,
    q_c, positions, q, kv_c_normed, k_pe, out)`` keeps the reference's
    signature and order -- indexer (K insert, scores, top-k), window merge,
    latent append, sparse MLA decode with the sink -- with the decode step's
    launches fused: one prologue (indexer prep, K insert, latent append, q
    quant, lengths), the top-k (filter, exact scoring, select, merged rows
    in one launch), the decode (block-table conversion in-kernel).  The
    absorbed-MLA W_UK / W_UV products run as batched GEMMs.  With
    ``fp8_o_proj`` the gated ``wo_b`` input is quantized by
    ``sigmoid_mul_quant_fp8`` (the reference's fused DeepGEMM input) and
    dequantized for the bf16 GEMM."""

    def __init__(self, vllm_config, prefix: str, topk_indices_buffer: torch.Tensor | None = None,
                 swa_topk_buffer: torch.Tensor | None = None, **kwargs) -> None:
        super().__init__()
        config = vllm_config.model_config.hf_config
        _check_attn_tp(config)
        cache_config = copy.copy(vllm_config.cache_config)
        dev = _device_of(vllm_config)
        self.prefix = prefix
        self.num_heads = config.mla_num_heads
        self.num_local_heads = self.num_heads
        self.q_lora_rank = config.mla_q_lora_rank
        self.kv_lora_rank = config.mla_kv_lora_rank
        self.qk_nope_head_dim = config.mla_qk_nope_head_dim
        self.qk_rope_head_dim = config.mla_qk_rope_head_dim
        self.qk_head_dim = self.qk_nope_head_dim + self.qk_rope_head_dim
        self.v_head_dim = config.mla_v_head_dim
        self.window = config.sliding_window
        self.fp8_o_proj = bool(kwargs.get("fp8_o_proj", False))
        self.fused_qkv_a_proj = Linear(config.hidden_size, self.q_lora_rank + self.kv_lora_rank + self.qk_rope_head_dim,
                                       return_bias=True, device=dev)
        self.q_a_layernorm = RMSNorm(self.q_lora_rank, eps=config.rms_norm_eps, device=dev)
        self.q_b_proj = Linear(self.q_lora_rank, self.num_heads * self.qk_head_dim, return_bias=True, device=dev)
        self.kv_a_layernorm = RMSNorm(self.kv_lora_rank, eps=config.rms_norm_eps, device=dev)
        self.kv_b_proj = Linear(self.kv_lora_rank, self.num_heads * (self.qk_nope_head_dim + self.v_head_dim),
                                return_bias=True, device=dev)
        self.wo_b = Linear(self.num_heads * self.v_head_dim, config.hidden_size, device=dev)
        self.o_gate = Linear(self.q_lora_rank, self.num_heads * self.v_head_dim, device=dev)
        self.vha = VHAPostMix(self.num_heads, device=dev)
        self.rotary_emb = InterleavedRotaryEmbedding(self.qk_rope_head_dim, config.max_position_embeddings,
                                                     config.mla_rope_parameters, dev)
        self.attn_sink = torch.nn.Parameter(torch.zeros(self.num_local_heads, dtype=torch.float32, device=dev),
                                            requires_grad=False)
        _check_sink_backend(self.kv_lora_rank + self.qk_rope_head_dim, cache_config.cache_dtype)
        if not cache_config.cache_dtype.startswith("fp8"):
            raise NotImplementedError("the DSA latent append writes fp8 page rows; use an fp8 KV cache")
        self.indexer = Ernie5_5Indexer(vllm_config, config, None, cache_config, topk_indices_buffer, swa_topk_buffer,
                                       prefix=f"{prefix}.indexer")
        self.mla_attn = Ernie5_5MLAAttention(
            num_heads=self.num_local_heads, scale=self.qk_head_dim ** -0.5, qk_nope_head_dim=self.qk_nope_head_dim,
            qk_rope_head_dim=self.qk_rope_head_dim, v_head_dim=self.v_head_dim, q_lora_rank=self.q_lora_rank,
            kv_lora_rank=self.kv_lora_rank, kv_b_proj=self.kv_b_proj, cache_config=cache_config,
            prefix=f"{prefix}.attn", attn_backend=Ernie5_5FlashMLASparseBackend, use_sparse=True,
            indexer=self.indexer, topk_indices_buffer=swa_topk_buffer, sinks=self.attn_sink)

    def load_weights(self, weights) -> set:
        loaded = _load(self, weights)
        self.mla_attn.process_weights_after_loading()
        self.vha.fold()
        return loaded

    def forward(self, positions: torch.Tensor, hidden_states: torch.Tensor,
                llama_4_scaling: torch.Tensor | None = None) -> torch.Tensor:
        num_tokens = hidden_states.shape[0]
        q_c, kv_lora = self.fused_qkv_a_proj(hidden_states)[0].split(
            [self.q_lora_rank, self.kv_lora_rank + self.qk_rope_head_dim], dim=-1)
        q_c = self.q_a_layernorm(q_c)
        gate = self.o_gate(q_c)
        q = self.q_b_proj(q_c)[0].view(-1, self.num_local_heads, self.qk_head_dim)
        kv_c, k_pe = kv_lora.split([self.kv_lora_rank, self.qk_rope_head_dim], -1)
        kv_c_normed = self.kv_a_layernorm(kv_c)
        q[..., self.qk_nope_head_dim:], k_pe = self.rotary_emb(positions, q[..., self.qk_nope_head_dim:],
                                                               k_pe.unsqueeze(1))
        attn_out = torch.empty((num_tokens, self.num_local_heads * self.v_head_dim), dtype=hidden_states.dtype,
                               device=hidden_states.device)
        self._indexer_and_attn(hidden_states, q_c, positions, q, kv_c_normed, k_pe, attn_out)
        o = self.vha(attn_out.view(num_tokens, self.num_local_heads, self.v_head_dim))
        if self.fp8_o_proj:
            data, scale = sigmoid_mul_quant_fp8(o.flatten(1).contiguous(), gate.contiguous())
            return self.wo_b(dequant_sigmoid_mul(data, scale).to(hidden_states.dtype))
        return self.wo_b(o.flatten(1) * torch.sigmoid(gate))

    def _indexer_and_attn(self, hidden_states: torch.Tensor, q_c: torch.Tensor, positions: torch.Tensor,
                          q: torch.Tensor, kv_c_normed: torch.Tensor, k_pe: torch.Tensor, out: torch.Tensor) -> None:
        """Indexer, window merge and sparse MLA in one eager segment
        (attention.py:1205-1226): ``out [T, H * v_head_dim]`` in place."""
        num_tokens = hidden_states.shape[0]
        md: DSAStepMetadata = get_forward_context().attn_metadata[self.mla_attn.prefix]
        ix = self.indexer
        iq, ik, iw = ix._project(hidden_states, q_c)
        latent = torch.cat([kv_c_normed, k_pe.reshape(num_tokens, -1)], dim=-1).contiguous()
        lengths = ix._lengths_buf(num_tokens, q.device)
        if ix.use_fp4_kv:  # prep, MXFP4 K insert and q, latent append, lengths: one launch
            qa, qb, wf = ops.dsa_decode_prologue_fp4(
                ik, ix.k_cache.kv_cache, latent, self.mla_attn.kv_cache, md.slot_mapping, iq, iw, positions,
                self.window, lengths, prep=ix._prep_args(q.device))
        merged = ix.topk_indices_buffer[:num_tokens]
        L = max(int(md.max_seq_len), 1)
        if ix.use_fp4_kv:
            ix._topk(qa, qb, wf, md, lengths, positions, merged=merged)
        elif md.max_query_len >= 1 and num_tokens * 20 * L <= _INDEXER_WORKSPACE_BYTES:
            # the prologue and the top-k in one call (in one launch when the
            # step's rows are decode rows and the top-k is one launch)
            ops.dsa_decode_prologue_topk_merged(
                ik, ix.k_cache.kv_cache, latent, self.mla_attn.kv_cache, md.slot_mapping, iq, iw, positions,
                self.window, lengths, md.block_table, md.req_ids, L,
                ix.indexer_op.topk_indices_buffer[:num_tokens, : ix.topk], _indexer_workspace(num_tokens, L, q.device),
                merged, prep=ix._prep_args(q.device), max_new_rows=md.max_query_len)
        else:  # one prologue launch, then the top-k
            qa, wf, qb = ops.dsa_decode_prologue(
                ik, ix.k_cache.kv_cache, latent, self.mla_attn.kv_cache, md.slot_mapping, iq, iw, positions,
                self.window, lengths, prep=ix._prep_args(q.device))
            ix._topk(qa, qb, wf, md, lengths, positions, merged=merged)
        q_abs = self.mla_attn.absorb_q(q)
        o_latent, _ = self.mla_attn.impl._fp8_flash_mla_kernel(
            q_abs[:, None], self.mla_attn.kv_cache, merged[:, None],
            SimpleNamespace(block_table=md.block_table, req_ids=md.req_ids))
        out.copy_(self.mla_attn.up_proj(o_latent[:, 0]))


class _Compressor(torch.nn.Module):
    """The HCA layer's compressor parameters (``compressor.*``): the fused
    ``fused_wkv_wgate`` projection of the hidden states to kv || score
    (model.py:684-685), the position embedding ``ape [128, D]`` added to the
    score, and the RMSNorm weight of the compressed row."""

    def __init__(self, hidden_size: int, dim: int, eps: float, device) -> None:
        super().__init__()
        self.fused_wkv_wgate = Linear(hidden_size, 2 * dim, device=device)
        self.ape = torch.nn.Parameter(torch.zeros(128, dim, dtype=torch.float32, device=device), requires_grad=False)
        self.norm = RMSNorm(dim, eps=eps, device=device, dtype=torch.float32)


class Ernie5_5HCAAttentionMixin(torch.nn.Module):
    """The HCA attention layer (attention.py:410-539), constructed as the
    reference's ``(vllm_config, prefix, **kwargs)``.

    The reference subclasses upstream ``DeepseekV4Attention`` (absent: vLLM
    is not in this tree); this class restates the parts its forward calls,
    with the config's shapes: ``_run_parallel_input_projections`` (the fused
    ``fused_wqa_wkv`` projection of the hidden states to the q low-rank
    input and the latent row, and ``compressor.fused_wkv_wgate`` to the
    compressor input), ``_split_qkv_and_norm`` (RMSNorms of both), and
    ``_prepare_and_attn_fn(hidden_states, qr, kv, qr_scale, kv_score,
    indexer_kv_score, indexer_weights, positions, o_padded)`` -- upstream's
    nine-argument call (:495-505): ``wq_b``, the interleaved RoPE of the q
    and latent rope parts at the token positions, then on the HIP library
    the cache write (latent rows, window ring, compressor state ring, every
    completed 128-token span compressed), each query row's index row (its
    compressed entries, then its window) and the sparse decode with the
    sink into ``o_padded[:, :heads]`` (``_cache_and_attn``).  ``forward
    (positions, hidden_states, llama_4_scaling=None)`` is the reference's:
    projections, the KV path, the ``o_gate`` gate, VHA, and the output
    projection (inverse RoPE of the output's rope part, the grouped
    ``wo_a``, the gated ``wo_b``; with ``fp8_o_proj`` VHA + inverse RoPE +
    fp8 quant run as ``vha_inv_rope_fp8_quant`` and the gated ``wo_b`` input
    as ``sigmoid_mul_quant_fp8``, dequantized for the bf16 GEMMs).  The KV
    cache is fp8 pages of per-token-scaled rows (``Ernie5_5HCAFlashMLAAttention``)
    or bf16 rows (``Ernie5_5HCAFlashInferAttention``)."""

    kv_cache_dtype = "fp8"

    def __init__(self, vllm_config, prefix: str, **kwargs) -> None:
        config = vllm_config.model_config.hf_config
        _check_attn_tp(config)
        super().__init__()
        dev = _device_of(vllm_config)
        self.prefix = prefix
        self.n_heads = config.num_attention_heads
        self.n_local_heads = self.n_heads
        self.padded_heads = max(int(kwargs.get("padded_heads", 64)), self.n_local_heads)
        self.head_dim = config.head_dim
        self.nope_head_dim = config.qk_nope_head_dim
        self.rope_head_dim = config.qk_rope_head_dim
        self.q_lora_rank = config.q_lora_rank
        self.n_groups = config.o_groups
        self.n_local_groups = self.n_groups
        self.o_lora_rank = config.o_lora_rank
        self.window = config.sliding_window
        self.ring = int(kwargs.get("ring", 192))
        if self.ring % DSA_BLOCK_SIZE or self.ring < self.window:
            raise ValueError("the window ring must be whole 64-row pages holding at least the window")
        self.softmax_scale = kwargs.get("scale") or self.head_dim ** -0.5
        self.norm_eps = config.rms_norm_eps
        self.fp8_o_proj = bool(kwargs.get("fp8_o_proj", False))
        self.fused_wqa_wkv = Linear(config.hidden_size, self.q_lora_rank + self.head_dim, device=dev)
        self.q_norm = RMSNorm(self.q_lora_rank, eps=config.rms_norm_eps, device=dev)
        self.kv_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps, device=dev)
        self.wq_b = Linear(self.q_lora_rank, self.n_heads * self.head_dim, device=dev)
        self.compressor = _Compressor(config.hidden_size, self.head_dim, config.rms_norm_eps, dev)
        hpg = self.n_heads // self.n_groups
        self.wo_a = torch.nn.Parameter(torch.empty(self.n_groups, self.o_lora_rank, hpg * self.head_dim,
                                                   dtype=torch.bfloat16, device=dev), requires_grad=False)
        self.wo_b = Linear(self.n_groups * self.o_lora_rank, config.hidden_size, device=dev)
        self.o_gate = Linear(self.q_lora_rank, self.n_groups * self.o_lora_rank, device=dev)
        self.vha = VHAPostMix(self.n_heads, device=dev)
        self.attn_sink = torch.nn.Parameter(torch.zeros(self.n_heads, dtype=torch.float32, device=dev),
                                            requires_grad=False)
        self.indexer = None
        if kwargs.get("rope_cos_sin") is not None:  # a given cos | sin table (e.g. YaRN) for q / kv
            self.rotary_emb = InterleavedRotaryEmbedding.from_table(kwargs["rope_cos_sin"])
        else:
            self.rotary_emb = InterleavedRotaryEmbedding(self.rope_head_dim, config.max_position_embeddings,
                                                         config.rope_parameters, dev)
        cs = kwargs.get("compress_cos_sin")
        if cs is None:  # the compressed entry j rotated at position 128 j, compress_rope_theta
            spans = config.max_position_embeddings // 128 + 1
            cs = rope_cos_sin_table(self.rope_head_dim, config.compress_rope_theta, spans * 128, dev)[::128]
        self.compress_cos_sin = cs.contiguous()
        self.kv_cache: torch.Tensor | None = None     # fp8 pages [num_pages, 64 * (D + 4)] or bf16 rows [N, D]
        self.state_cache: torch.Tensor | None = None  # bf16 [num_state, 256, 2 D]
        self._idx: torch.Tensor | None = None
        self._ws: torch.Tensor | None = None
        self._write_ws: torch.Tensor | None = None
        self._write_spans = 0

    # --- views of the compressor parameters the write kernels read
    @property
    def ape(self) -> torch.Tensor:
        return self.compressor.ape.detach()

    @property
    def norm_w(self) -> torch.Tensor:
        return self.compressor.norm.weight.detach()

    def load_weights(self, weights) -> set:
        loaded = _load(self, weights)
        self.vha.fold()
        return loaded

    # --- the projections around the KV path
    def _run_parallel_input_projections(self, hidden_states: torch.Tensor):
        qr_kv = self.fused_wqa_wkv(hidden_states)
        kv_score = self.compressor.fused_wkv_wgate(hidden_states)
        return qr_kv, kv_score, None, None

    def _split_qkv_and_norm(self, qr_kv: torch.Tensor):
        qr, kv = qr_kv.split([self.q_lora_rank, self.head_dim], dim=-1)
        return self.q_norm(qr), None, self.kv_norm(kv)

    def _gate(self, qr: torch.Tensor) -> torch.Tensor:
        return self.o_gate(qr) if self.fp8_o_proj else torch.sigmoid(self.o_gate(qr))

    def forward(self, positions: torch.Tensor, hidden_states: torch.Tensor,
                llama_4_scaling: torch.Tensor | None = None) -> torch.Tensor:
        num_tokens = hidden_states.shape[0]
        o_padded = torch.empty((num_tokens, self.padded_heads, self.head_dim), dtype=hidden_states.dtype,
                               device=hidden_states.device)
        qr_kv, kv_score, indexer_kv_score, indexer_weights = self._run_parallel_input_projections(hidden_states)
        qr, qr_scale, kv = self._split_qkv_and_norm(qr_kv)
        self._prepare_and_attn_fn(hidden_states, qr, kv, qr_scale, kv_score, indexer_kv_score, indexer_weights,
                                  positions, o_padded)
        gate = self._gate(qr)
        o = o_padded[:, : self.n_local_heads, :]
        return self._o_proj(o, positions, gate)

    def _o_proj(self, o: torch.Tensor, positions: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        """VHA, inverse RoPE of the rope part, grouped wo_a, gated wo_b."""
        T = o.shape[0]
        G = self.n_local_groups
        if self.fp8_o_proj:
            data, scale = ops.vha_inv_rope_fp8_quant(o, self.vha.m, positions, self.rotary_emb.cos_sin_cache, G,
                                                     self.nope_head_dim, self.rope_head_dim)
            og = dequant_vha(data, scale).to(o.dtype)  # [T, G, hpg * D]
        else:
            o = self.vha(o)
            o = torch.cat([o[..., : self.nope_head_dim],
                           self.rotary_emb.rotate(positions, o[..., self.nope_head_dim:], inverse=True)], dim=-1)
            og = o.reshape(T, G, -1)
        z = torch.bmm(og.transpose(0, 1).contiguous(), self.wo_a.transpose(1, 2).contiguous())  # [G, T, r]
        z = z.transpose(0, 1).reshape(T, G * self.o_lora_rank)
        if self.fp8_o_proj:
            data, scale = ops.sigmoid_mul_quant_fp8(z.contiguous(), gate.contiguous())
            return self.wo_b(dequant_sigmoid_mul(data, scale).to(o.dtype))
        return self.wo_b(z * gate)

    # --- the KV path
    def _write_workspace(self, num_seqs: int, max_query_len: int, D: int, device) -> torch.Tensor:
        """The cache write's workspace, grown to the most span slots a call
        has had (one per sequence and 128 rows of its longest query, plus
        one): decode-sized calls compress a span with D / 64 workgroups, longer
        ones with D / 64."""
        spans = num_seqs * (max_query_len // 128 + 1)
        if self._write_ws is None or self._write_spans < spans:
            self._write_spans = max(spans, 2 * self._write_spans)
            self._write_ws = ops.hca_write_workspace(self._write_spans, D, device)
        return self._write_ws

    def _decode_buffers(self, T: int, width: int, device):
        if self._idx is None or self._idx.shape[0] < T or self._idx.shape[1] < width:
            self._idx = torch.empty((T, width), dtype=torch.int32, device=device)
            self._lens = torch.empty(T, dtype=torch.int32, device=device)
            self._lse = torch.empty((T, self.padded_heads), dtype=torch.float32, device=device)
            self._ws = ops.decode_workspace(T, self.padded_heads, width, device)
        return self._idx[:T, :width], self._lens[:T], self._lse[:T], self._ws

    def _prepare_and_attn_fn(self, hidden_states: torch.Tensor, qr: torch.Tensor, kv: torch.Tensor,
                             qr_scale: torch.Tensor | None, kv_score: torch.Tensor,
                             indexer_kv_score: torch.Tensor | None, indexer_weights: torch.Tensor | None,
                             positions: torch.Tensor, o_padded: torch.Tensor) -> None:
        """Upstream's call (attention.py:495-505): q from ``wq_b(qr)``, the
        interleaved RoPE of q's and kv's rope parts at ``positions``, then
        ``_cache_and_attn``.  HCA layers have no indexer, so
        ``indexer_kv_score`` / ``indexer_weights`` are None; ``qr_scale``
        (a quantized-qr scale) is None for bf16 qr."""
        T = qr.shape[0]
        q = self.wq_b(qr).view(T, self.n_local_heads, self.head_dim)
        nope = self.nope_head_dim
        q = torch.cat([q[..., :nope], self.rotary_emb.rotate(positions, q[..., nope:])], dim=-1)
        kv = torch.cat([kv[..., :nope], self.rotary_emb.rotate(positions, kv[..., nope:])], dim=-1)
        self._cache_and_attn(q, kv.contiguous(), kv_score.contiguous(), positions, o_padded)

    def _cache_and_attn(self, q: torch.Tensor, kv: torch.Tensor, kv_score: torch.Tensor, positions: torch.Tensor,
                        o_padded: torch.Tensor) -> None:
        """The HIP part of the layer: q ``[T, heads, D]``, the latent rows kv
        ``[T, D]`` and the compressor input kv_score ``[T, 2D]``; appends kv
        (pool rows, window ring, compressor state ring), compresses every
        128-token span that completes, builds each query row's index row
        and runs the sparse decode with the sink into ``o_padded[:, :heads]``."""
        md: HCAStepMetadata = get_forward_context().attn_metadata[self.prefix]
        T, H, D = q.shape
        bf16_cache = self.kv_cache.dtype == torch.bfloat16
        # A request with more than ring - window rows in the call would
        # overwrite ring rows that its own first rows' windows still read:
        # such calls update the ring after the decode.
        late_ring = md.max_query_len > self.ring - self.window
        width = md.max_seq_len // 128 + self.window
        idx, lens, lse, ws = self._decode_buffers(T, width, q.device)
        write_ws = self._write_workspace(md.query_start_loc.numel() - 1, md.max_query_len, D, q.device)
        if late_ring:
            ops.hca_write(kv, kv_score, md.slot_mapping, positions, md.token_seq, md.query_start_loc,
                          md.max_query_len, self.state_cache, md.state_slot, self.ape, self.norm_w, self.norm_eps,
                          self.compress_cos_sin, md.comp_block_table, None, self.ring, self.kv_cache,
                          workspace=write_ws)
            ops.hca_decode_indices(positions, md.token_seq, md.comp_block_table, md.ring_pages, self.ring, idx, lens,
                                   self.window, query_start_loc=md.query_start_loc, slot_mapping=md.slot_mapping)
        else:  # the write and the index rows (one launch for decode-sized calls)
            ops.hca_write_step(kv, kv_score, md.slot_mapping, positions, md.token_seq, md.query_start_loc,
                               md.max_query_len, self.state_cache, md.state_slot, self.ape, self.norm_w,
                               self.norm_eps, self.compress_cos_sin, md.comp_block_table, md.ring_pages, self.ring,
                               self.kv_cache, self.window, idx, lens, workspace=write_ws)
        if H < self.padded_heads:
            qp = q.new_zeros((T, self.padded_heads, D))
            qp[:, :H] = q
            q = qp
        sinks = self.attn_sink.detach().float()
        if sinks.numel() < self.padded_heads:
            sinks = torch.cat([sinks, sinks.new_full((self.padded_heads - sinks.numel(),), float("-inf"))])
        ops.sparse_mla_decode(q, self.kv_cache, idx, self.softmax_scale, o_padded, lse, sinks=sinks.contiguous(),
                              lengths=lens, cache_bf16=bf16_cache, workspace=ws)
        if late_ring:  # the window ring rows only (pool rows skipped, state ring already written)
            skip = torch.full((T,), -1, dtype=torch.int64, device=q.device)
            ops.hca_append(kv, None, skip, positions, md.token_seq, md.query_start_loc, self.kv_cache, md.ring_pages,
                           self.ring, None, None)


# --------------------------------------------------------------------------- post-attention quant
VHA_RANK = 16


@dataclass
class QuantizedActivation:
    """Stand-in for vLLM's QuantizedActivation: the fields the fp8 o-proj reads."""

    data: torch.Tensor
    scale: torch.Tensor
    orig_dtype: Any
    orig_shape: tuple
    quant_key: str = "fp8_dynamic_128_sym"


class VHAPostMix(torch.nn.Module):
    """Head mixing ``o[h] <- sum_g m[h, g] o[g]`` with ``m = I + V U^T``
    (attention.py:120-157, TP = 1): a plain batched product outside this
    path; ``m`` is what vha_inv_rope_fp8_quant fuses."""

    def __init__(self, num_heads: int, rank: int = VHA_RANK, device=None, dtype=torch.bfloat16) -> None:
        super().__init__()
        self.tp_size = 1
        self.U = torch.nn.Parameter(torch.zeros(num_heads, rank, dtype=dtype, device=device), requires_grad=False)
        self.V = torch.nn.Parameter(torch.zeros(num_heads, rank, dtype=dtype, device=device), requires_grad=False)
        self.register_buffer("m", torch.eye(num_heads, dtype=dtype, device=device), persistent=False)

    def fold(self) -> None:
        eye = torch.eye(self.U.shape[0], dtype=self.U.dtype, device=self.U.device)
        self.m.copy_(torch.addmm(eye, self.V, self.U.t()))

    def forward(self, o: torch.Tensor) -> torch.Tensor:
        return torch.matmul(self.m, o)


def vha_inv_rope_fp8_quant(o: torch.Tensor, mix: torch.Tensor, positions: torch.Tensor, cos_sin_cache: torch.Tensor,
                           n_groups: int, nope_dim: int, rope_dim: int) -> QuantizedActivation:
    """VHA head mixing + inverse RoPE + fp8 quant in one kernel
    (attention.py:232-285): data [T, n_groups, hpg * 512] fp8, scale
    [T, n_groups, hpg] int32 (byte c = biased exponent of channel chunk c)."""
    data, scale = ops.vha_inv_rope_fp8_quant(o, mix, positions, cos_sin_cache, n_groups, nope_dim, rope_dim)
    return QuantizedActivation(data=data, scale=scale, orig_dtype=o.dtype, orig_shape=tuple(data.shape))


def sigmoid_mul_quant_fp8(x: torch.Tensor, gate: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``x * sigmoid(gate)`` as 1x128 UE8M0 fp8 with DeepGEMM-packed scales
    (attention.py:340-361)."""
    return ops.sigmoid_mul_quant_fp8(x, gate)


# --------------------------------------------------------------------------- HCA layer class choice
class Ernie5_5HCAFlashInferAttention(Ernie5_5HCAAttentionMixin):
    """HCA layer on a bf16 KV row (attention.py:542-545): the cache is bf16
    rows (64 a page); the write stores the latent rows as given and the
    compressed rows rounded to bf16, the decode reads bf16 rows."""

    kv_cache_dtype = "bfloat16"


class Ernie5_5HCAFlashMLAAttention(Ernie5_5HCAAttentionMixin):
    """HCA layer on an fp8 KV row (attention.py:548-551): fp8 pages of
    per-token-scaled rows (580 bytes at D = 576, 516 at D = 512)."""

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


def ernie5_5_config(**overrides) -> SimpleNamespace:
    """The Ernie5_5Config fields this path reads, at their defaults
    (src/vllm_ernie/models/ernie5_5/config.py:13-62, 154-189)."""
    cfg = dict(hidden_size=4096, num_attention_heads=64, head_dim=512, q_lora_rank=1024, kv_lora_rank=512,
               qk_nope_head_dim=448, qk_rope_head_dim=64, o_groups=8, o_lora_rank=1024, sliding_window=128,
               hybrid_mla_num_attention_heads=64, hybrid_mla_q_lora_rank=1024, hybrid_mla_kv_lora_rank=512,
               hybrid_mla_qk_nope_head_dim=192, hybrid_mla_qk_rope_head_dim=64, hybrid_mla_v_head_dim=256,
               index_n_heads=64, index_head_dim=128, index_topk=2048, max_position_embeddings=200192,
               rope_theta=2500000.0, compress_rope_theta=160000.0, rms_norm_eps=1e-6, rope_parameters=None)
    cfg.update(overrides)
    ns = SimpleNamespace(**cfg)
    if ns.rope_parameters is None:
        ns.rope_parameters = {"rope_type": "default", "rope_theta": ns.rope_theta}
    ns.mla_num_heads = ns.hybrid_mla_num_attention_heads
    ns.mla_q_lora_rank = ns.hybrid_mla_q_lora_rank
    ns.mla_kv_lora_rank = ns.hybrid_mla_kv_lora_rank
    ns.mla_qk_nope_head_dim = ns.hybrid_mla_qk_nope_head_dim
    ns.mla_qk_rope_head_dim = ns.hybrid_mla_qk_rope_head_dim
    ns.mla_v_head_dim = ns.hybrid_mla_v_head_dim
    ns.mla_rope_parameters = {"rope_type": "default", "rope_theta": ns.rope_theta}
    return ns


def ernie5_5_vllm_config(hf_config=None, cache_dtype: str = "fp8", block_size: int = 64,
                         use_fp4_indexer_cache: bool = False, device=None, prefill_context_parallel_size: int = 1,
                         decode_context_parallel_size: int = 1, max_model_len: int | None = None) -> SimpleNamespace:
    """Stand-in for vLLM's VllmConfig with the fields the layers read:
    ``model_config.hf_config`` (``ernie5_5_config()`` by default),
    ``cache_config`` (block size, cache dtype), ``quant_config`` (None: bf16
    weights), ``parallel_config`` (context-parallel sizes; TP = 1),
    ``attention_config`` (the MXFP4 indexer-cache flag) and the device."""
    hf = hf_config if hf_config is not None else ernie5_5_config()
    return SimpleNamespace(
        model_config=SimpleNamespace(hf_config=hf, max_model_len=max_model_len or hf.max_position_embeddings),
        cache_config=SimpleNamespace(block_size=block_size, cache_dtype=cache_dtype),
        quant_config=None,
        parallel_config=SimpleNamespace(prefill_context_parallel_size=prefill_context_parallel_size,
                                        decode_context_parallel_size=decode_context_parallel_size,
                                        tensor_parallel_size=1),
        attention_config=SimpleNamespace(use_fp4_indexer_cache=use_fp4_indexer_cache, sparse_mla_force_mqa=True),
        device_config=SimpleNamespace(device=device),
    )
