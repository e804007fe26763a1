"""Host-side checks (CPU): the C-ABI library loads and exports every symbol
the header declares; the ctypes signatures agree with the header; the
reference-interface mirror behaves like the reference's host logic."""

import re
from pathlib import Path
from types import SimpleNamespace

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ernie_kv.h"


def _header_functions() -> dict[str, int]:
    """name -> number of parameters, parsed from include/ernie_kv.h."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|int32_t|int64_t|const char\*)\s+(ekv_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_library_exports_every_header_symbol():
    import ctypes

    from ernie_kv import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libernie_kv.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _header_functions():
        assert hasattr(lib, name), f"{name} declared in ernie_kv.h but not exported"


def test_ctypes_signatures_match_header():
    from ernie_kv import _lib

    decl = _header_functions()
    assert set(decl) == set(_lib.exported_symbols())
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == decl[name], f"{name}: {len(args)} ctypes args vs {decl[name]} in header"


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from ernie_kv import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.EkvError, match="no CPU fallback"):
        _lib.load()


def test_ops_refuse_cpu_tensors():
    import torch

    from ernie_kv import ops

    with pytest.raises(ValueError, match="device tensors"):
        ops.kv_append_quant(torch.zeros(1, 576, dtype=torch.bfloat16), torch.zeros(1, dtype=torch.int64),
                            torch.zeros(1, 64 * 580, dtype=torch.uint8))


def test_packed_block_stride_alignment():
    """test_dsa_backend.py:40-55."""
    from ernie_kv.attention import packed_block_stride_alignment, simple_vllm_config

    a = packed_block_stride_alignment(simple_vllm_config())
    assert a % 512 == 0 and a % (512 * 2) == 0 and a % ((512 + 64) * 2) == 0


@pytest.mark.parametrize("spec", [None, SimpleNamespace()])
def test_dsa_kernel_block_sizes_accept_kv_cache_spec(spec):
    """test_dsa_backend.py:58-70."""
    from ernie_kv.attention import Ernie5_5FlashMLASparseBackend, Ernie5_5IndexerBackend, MultipleOf

    for backend in (Ernie5_5FlashMLASparseBackend, Ernie5_5IndexerBackend):
        assert backend.get_supported_kernel_block_sizes() == [MultipleOf(64)]
        assert backend.get_supported_kernel_block_sizes(spec) == [MultipleOf(64)]


def test_backend_surface():
    from ernie_kv import attention as A

    assert A.Ernie5_5FlashMLASparseBackend.supports_sink()
    assert A.Ernie5_5FlashMLASparseBackend.get_impl_cls() is A.Ernie5_5FlashMLASparseImpl
    assert A.Ernie5_5FlashMLASparseBackend.get_name() == "FLASHMLA_SPARSE"
    assert A.Ernie5_5IndexerBackend.supported_kv_cache_layouts() == (A.KVCacheLayout.BLNHC, A.KVCacheLayout.BLHNC)
    assert A.Ernie5_5IndexerBackend.get_builder_cls() is A.Ernie5_5IndexerMetadataBuilder
    assert A.select_ernie5_5_hca_cls("fp8_ds_mla") is A.Ernie5_5HCAFlashMLAAttention
    assert A.select_ernie5_5_hca_cls("auto") is A.Ernie5_5HCAFlashInferAttention


def test_kv_cache_specs_use_dsa_pages():
    from ernie_kv import attention as A

    cfg = A.simple_vllm_config(block_size=256)
    spec = A.Ernie5_5MLAAttention().get_kv_cache_spec(cfg)
    assert spec.block_size == 64 and spec.block_stride_alignment == 9216
    ic = A.Ernie5_5IndexerCache(head_dim=132, dtype="uint8", prefix="model.layers.0.indexer.k_cache")
    s2 = ic.get_kv_cache_spec(cfg)
    assert s2.block_size == 64 and s2.head_size == 132 and ic.get_attn_backend() is A.Ernie5_5IndexerBackend


def test_padded_sinks_are_noop_minus_inf():
    import torch

    from ernie_kv.attention import Ernie5_5FlashMLASparseImpl

    impl = Ernie5_5FlashMLASparseImpl(num_heads=16, head_size=576, scale=0.0625, sinks=torch.arange(16.0))
    p = impl._padded_sinks(64)
    assert torch.equal(p[:16], torch.arange(16.0)) and torch.all(torch.isneginf(p[16:]))
    assert impl._padded_sinks(16) is impl.sinks


def test_fp8_kernel_refuses_fp8_ds_mla_pages():
    """Upstream fp8_ds_mla pages share this library's 46,080-byte page
    stride, so the fp8 sparse kernel takes the format from kv_cache_dtype and
    refuses such a cache (before any device work) instead of reading its
    656-byte rows as 580-byte ones."""
    import torch

    from ernie_kv.attention import Ernie5_5FlashMLASparseImpl

    impl = Ernie5_5FlashMLASparseImpl(num_heads=64, head_size=576, scale=0.0625, kv_cache_dtype="fp8_ds_mla",
                                      sinks=torch.zeros(64))
    q = torch.zeros((1, 1, 64, 576), dtype=torch.bfloat16)
    cache = torch.zeros((4, 46080), dtype=torch.uint8)
    with pytest.raises(ValueError, match="fp8_ds_mla"):
        impl._fp8_flash_mla_kernel(q, cache, torch.zeros((1, 1, 2176), dtype=torch.int32))


def test_attn_tp_and_sink_backend_errors():
    from ernie_kv.attention import _check_attn_tp, _check_sink_backend

    cfg = SimpleNamespace(o_groups=8, num_attention_heads=64, hybrid_mla_num_attention_heads=64)
    _check_attn_tp(cfg, 8)
    with pytest.raises(ValueError, match="must divide"):
        _check_attn_tp(cfg, 3)
    with pytest.raises(RuntimeError, match="sink-capable"):
        _check_sink_backend(384, "fp8")


def _indexer(use_fp4_kv, pcp=1, dcp=1):
    from ernie_kv import attention as A

    cfg = A.ernie5_5_config(hidden_size=256, hybrid_mla_q_lora_rank=128)
    vc = A.ernie5_5_vllm_config(cfg, use_fp4_indexer_cache=use_fp4_kv, device="cpu",
                                prefill_context_parallel_size=pcp, decode_context_parallel_size=dcp)
    return A.Ernie5_5Indexer(vc, cfg, vc.quant_config, vc.cache_config, None, None,
                             prefix="model.layers.0.self_attn.indexer")


@pytest.mark.parametrize("pcp,dcp", [(2, 1), (1, 2), (2, 2)])
def test_mxfp4_requires_single_context_parallel(pcp, dcp):
    """test_indexer_fp4.py:59-70 (attention.py:881-892): the MXFP4 indexer
    refuses context parallelism with the reference's message."""
    with pytest.raises(NotImplementedError, match="PCP=DCP=1") as error:
        _indexer(True, pcp, dcp)
    assert f"PCP={pcp}, DCP={dcp}" in str(error.value)
    _indexer(False, pcp, dcp)  # the fp8 cache has no such limit


def test_indexer_k_cache_row_bytes():
    """68-byte MXFP4 rows (64 packed values + 4 UE8M0) vs 132-byte fp8 rows
    (attention.py:929-935)."""
    assert _indexer(True).k_cache.head_dim == 68
    assert _indexer(False).k_cache.head_dim == 132


def test_hca_write_workspace_size_in_span_slots():
    """ekv_hca_write_workspace_size(num_spans, dim) (host arithmetic only):
    monotone in the span count, independent of the width (the layout holds
    576-wide slots so one buffer serves both widths), zero for an invalid
    width, and Python's hca_write_workspace sizes prefill calls by their span
    slots: num_seqs * (max_query_len // 128 + 1)."""
    from ernie_kv import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libernie_kv.so not built (run __graft_entry__.build())")
    lib = _lib.load()
    size = lib.ekv_hca_write_workspace_size
    sizes = [size(n, 576) for n in range(1, 3000, 7)]
    assert all(b > a for a, b in zip(sizes, sizes[1:]))
    for n in (1, 16, 1040, 4096):
        assert size(n, 512) == size(n, 576)
        # counters (u32, padded to 256 B) then 576 + 144 floats per slot
        assert size(n, 576) == (n * 4 + 255) // 256 * 256 + n * (576 + 144) * 4
    assert size(0, 576) == 0 and size(16, 0) == 0 and size(16, 1024) == 0
    # 16 sequences of 8192-row chunks complete at most 16 * 65 spans
    assert size(16 * (8192 // 128 + 1), 576) > size(16, 576)


def test_torch_ops_registered_with_their_writes():
    """torch.ops.ernie_kv.* (ernie_kv.torch_ops): every operator is registered
    without a GPU, returns nothing and names the tensors it writes in its
    schema (Tensor(a!)), so the dispatcher sees the in-place writes."""
    import torch

    import ernie_kv.torch_ops as T

    writes = {"kv_append_quant": {"cache"}, "indexer_k_insert": {"kcache"}, "hca_write": {"pool", "state", "workspace"},
              "hca_write_step": {"pool", "state", "out", "lengths", "workspace"},
              "indexer_topk": {"topk_out", "workspace"}, "indexer_topk_merged": {"topk_out", "workspace", "merged"},
              "merge_swa_topk": {"out"}, "sparse_mla_decode": {"out", "lse", "workspace"}}
    assert set(T.OPS) == set(writes)
    for name, expect in writes.items():
        schema = getattr(torch.ops.ernie_kv, name).default._schema
        assert len(schema.returns) == 0, name
        got = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
        assert got == expect, (name, got)


def test_torch_ops_trace_without_launching():
    """Under FakeTensorMode (what torch.compile traces with) the operators
    run their fake implementations: nothing is launched, no library call is
    made, and the result is None."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    import ernie_kv.torch_ops  # noqa: F401

    with FakeTensorMode():
        rows = torch.empty((4, 576), dtype=torch.bfloat16)
        slots = torch.empty((4,), dtype=torch.int64)
        cache = torch.empty((2, 64 * 580), dtype=torch.uint8)
        assert torch.ops.ernie_kv.kv_append_quant(rows, slots, cache) is None
        topk = torch.empty((4, 2048), dtype=torch.int32)
        merged = torch.empty((4, 2176), dtype=torch.int32)
        assert torch.ops.ernie_kv.merge_swa_topk(topk, merged, slots, 128) is None
