"""GPU parity of the layer-level drop-in surface (ernie_kv/attention.py):
Ernie5_5Indexer.forward, Ernie5_5DSAAttention._indexer_and_attn, the HCA
layer's _prepare_and_attn_fn, the sparse impl's _fp8/_bf16 kernel methods
and Ernie5_5IndexerMetadataBuilder.build, each against the oracle.

The layers' projections are plain torch GEMMs outside the path: the tests
recompute them with the same torch calls on the same inputs (bit-identical
on one device) and start the oracle from their outputs."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, bf16_values, permuted_block_table, randn_bf16, to_dev
from oracle import decode as od
from oracle import hca as oh
from oracle import indexer as oi
from oracle import mxfp4 as om
from oracle import paged
from oracle.fp8 import quantize_rows
from oracle.merge import logical_to_global, merge_swa_topk

pytestmark = pytest.mark.gpu
RTOL, ATOL = 2e-2, 2e-3
TOPK, WINDOW = 2048, 128


def wc_decode(codes, scale):
    from oracle.fp8 import decode_e4m3

    return decode_e4m3(codes).astype(np.float64) * scale.astype(np.float64)[:, None]


def _check_decode(got, ref_o, what):
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref_o)
    bad = err > ATOL + RTOL * np.abs(ref_o)
    assert not bad.any(), f"{what}: max err {err.max()} at {np.argwhere(bad)[0]}"


def _dsa_setup(dev, rng, ctxs, rows_per_req, fp4=False):
    """Caches pre-filled up to each request's context, plus the step's query
    rows (the last rows_per_req positions of each request).  With fp4 the
    indexer K cache holds MXFP4 rows in 9216-byte pages (the packed-block
    stride)."""
    from ernie_kv import attention as A

    cfg = A.ernie5_5_config(hidden_size=256, hybrid_mla_q_lora_rank=128)
    B = len(ctxs)
    P = max((c + 63) // 64 for c in ctxs)
    bt = permuted_block_table(rng, B, P)
    pages = B * P
    kc = np.zeros((pages, 9216), np.uint8) if fp4 else oi.kcache_pages(pages)
    lat = np.zeros((pages, paged.fp8_page_bytes(576)), np.uint8)
    for b, c in enumerate(ctxs):
        s = np.arange(c - rows_per_req[b])  # the step writes the last rows itself
        slots = bt[b, s // 64].astype(np.int64) * 64 + s % 64
        (om.k_insert if fp4 else oi.k_insert)(kc, randn_bf16(rng, (len(s), 128)), slots)
        codes, scale = quantize_rows(randn_bf16(rng, (len(s), 576)))
        paged.write_fp8_rows(lat, slots, codes, scale, 576)
    req = np.concatenate([np.full(r, b, np.int32) for b, r in enumerate(rows_per_req)])
    positions = np.concatenate([np.arange(c - r, c) for c, r in zip(ctxs, rows_per_req)]).astype(np.int64)
    slot_mapping = paged.slots_from_block_table(bt, req, positions)
    T = len(positions)
    params = {
        "indexer.wq_b.weight": bf16_tensor(randn_bf16(rng, (64 * 128, 128), 128 ** -0.5), dev),
        "indexer.wk_weights_proj.weight": bf16_tensor(randn_bf16(rng, (128 + 64, 256), 256 ** -0.5), dev),
        "indexer.k_norm.weight": to_dev((1 + 0.1 * rng.standard_normal(128)).astype(np.float32), dev),
        "indexer.k_norm.bias": to_dev((0.1 * rng.standard_normal(128)).astype(np.float32), dev),
        "kv_b_proj.weight": bf16_tensor(randn_bf16(rng, (64 * (192 + 256), 512), 0.05), dev),
        "attn_sink": to_dev(rng.standard_normal(64).astype(np.float32), dev),
    }
    md = A.DSAStepMetadata(slot_mapping=to_dev(slot_mapping, dev), block_table=to_dev(bt, dev),
                           req_ids=to_dev(req, dev), max_seq_len=int(max(ctxs)), max_query_len=int(max(rows_per_req)))
    inputs = dict(hidden=randn_bf16(rng, (T, 256)), q_c=randn_bf16(rng, (T, 128)), q=randn_bf16(rng, (T, 64, 256)),
                  kv_c=randn_bf16(rng, (T, 512)), k_pe=randn_bf16(rng, (T, 1, 64)))
    return SimpleNamespace(cfg=cfg, bt=bt, kc=kc, lat=lat, req=req, positions=positions, slot_mapping=slot_mapping,
                           T=T, params=params, md=md, inputs=inputs,
                           vllm_config=A.ernie5_5_vllm_config(cfg, use_fp4_indexer_cache=fp4, device=dev))


def _dsa_layer(case, topk_buf, swa_buf):
    """Ernie5_5DSAAttention built as the reference builds it, with the
    case's weights loaded."""
    from ernie_kv import attention as A

    layer = A.Ernie5_5DSAAttention(case.vllm_config, "model.layers.3.attn", topk_buf, swa_buf)
    layer.load_weights(case.params.items())
    return layer


def _oracle_indexer(case, layer, dev):
    """The oracle's indexer from the layer's projection outputs: returns the
    K cache after the insert, the top-k and the windowed lengths."""
    hid = bf16_tensor(case.inputs["hidden"], dev)
    qc = bf16_tensor(case.inputs["q_c"], dev)
    iq, ik, iw = layer._project(hid, qc)
    table = layer._prep_args(dev)[3]
    pos = case.positions
    rq, rk = oi.indexer_prep(bf16_values(iq), bf16_values(ik), layer.k_norm_weight.cpu().numpy(),
                             layer.k_norm_bias.cpu().numpy(), 1e-6, table[to_dev(pos, dev)].cpu().numpy())
    kc = case.kc.copy()
    lens = oi.windowed_lengths(pos, WINDOW)
    if layer.use_fp4_kv:
        qv, qs, wf = om.quantize_q(rq, bf16_values(iw))
        om.k_insert(kc, rk, case.slot_mapping)
        top, _ = om.indexer_topk(qv, qs, wf, kc, case.bt, case.req, lens, TOPK)
    else:
        codes, wf = oi.quantize_q(rq, bf16_values(iw))
        oi.k_insert(kc, rk, case.slot_mapping)
        top, _ = oi.indexer_topk(codes, wf, kc, case.bt, case.req, lens, TOPK)
    return kc, top


@pytest.mark.parametrize("fp4", [False, True], ids=["fp8", "mxfp4"])
def test_indexer_forward_vs_oracle(dev, fp4):
    """Ernie5_5Indexer.forward (attention.py:955-984): projections, prep,
    quant, K insert and the exact top-k into indexer_op.topk_indices_buffer;
    fp8 (132-byte) or MXFP4 (68-byte, _quantize_fp4 :986-1025) K rows."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(61)
    case = _dsa_setup(dev, rng, [3000, 4500], [1, 3], fp4=fp4)
    topk_buf = torch.full((16, TOPK), -7, dtype=torch.int32, device=dev)
    swa_buf = torch.full((16, TOPK + WINDOW), -7, dtype=torch.int32, device=dev)
    vc = case.vllm_config
    ix = A.Ernie5_5Indexer(vc, case.cfg, None, vc.cache_config, topk_buf, swa_buf,
                           prefix="model.layers.3.attn.indexer")
    ix.load_weights((k[len("indexer."):], v) for k, v in case.params.items() if k.startswith("indexer."))
    assert ix.use_fp4_kv == fp4
    assert ix.k_cache.head_dim == (68 if fp4 else 132)
    ix.k_cache.kv_cache = to_dev(case.kc, dev)
    with A.set_forward_context({ix.k_cache.prefix: case.md}):
        got = ix.forward(bf16_tensor(case.inputs["hidden"], dev), bf16_tensor(case.inputs["q_c"], dev),
                         to_dev(case.positions, dev))
    torch.cuda.synchronize()
    kc_ref, top_ref = _oracle_indexer(case, ix, dev)
    assert np.array_equal(ix.k_cache.kv_cache.cpu().numpy(), kc_ref), "indexer K cache bytes differ"
    assert np.array_equal(got.cpu().numpy(), top_ref), "top-k differs"
    assert (swa_buf == -7).all(), "forward alone must not touch the merged (swa) buffer"


@pytest.mark.parametrize("fp4", [False, True], ids=["fp8", "mxfp4"])
def test_dsa_indexer_and_attn_vs_oracle(dev, fp4):
    """Ernie5_5DSAAttention._indexer_and_attn (attention.py:1205-1226): top-k,
    merged rows, both caches' bytes, the sparse decode's latent output and
    the up-projected out (fp8 or MXFP4 indexer K cache)."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(62)
    case = _dsa_setup(dev, rng, [3000, 4500], [1, 3], fp4=fp4)
    T = case.T
    topk_buf = torch.full((16, TOPK), -7, dtype=torch.int32, device=dev)
    swa_buf = torch.full((16, TOPK + WINDOW), -7, dtype=torch.int32, device=dev)
    layer = _dsa_layer(case, topk_buf, swa_buf)
    layer.indexer.k_cache.kv_cache = to_dev(case.kc, dev)
    layer.mla_attn.kv_cache = to_dev(case.lat, dev)
    captured = {}
    orig = layer.mla_attn.impl._fp8_flash_mla_kernel

    def spy(*args, **kwargs):
        captured["out"] = orig(*args, **kwargs)
        return captured["out"]

    layer.mla_attn.impl._fp8_flash_mla_kernel = spy
    inp = case.inputs
    out = torch.zeros((T, 64 * 256), dtype=torch.bfloat16, device=dev)
    meta = {layer.mla_attn.prefix: case.md, layer.indexer.k_cache.prefix: case.md}
    pos_t = to_dev(case.positions, dev)
    with A.set_forward_context(meta):
        layer._indexer_and_attn(bf16_tensor(inp["hidden"], dev), bf16_tensor(inp["q_c"], dev), pos_t,
                                bf16_tensor(inp["q"], dev), bf16_tensor(inp["kv_c"], dev),
                                bf16_tensor(inp["k_pe"], dev), out)
    torch.cuda.synchronize()
    kc_ref, top_ref = _oracle_indexer(case, layer.indexer, dev)
    assert np.array_equal(layer.indexer.k_cache.kv_cache.cpu().numpy(), kc_ref), "indexer K cache bytes differ"
    assert np.array_equal(topk_buf[:T].cpu().numpy(), top_ref), "top-k differs"
    merged_ref = merge_swa_topk(top_ref, case.positions, TOPK + WINDOW, WINDOW)
    assert np.array_equal(swa_buf[:T].cpu().numpy(), merged_ref), "merged rows differ"
    lat = case.lat.copy()
    rows = np.concatenate([inp["kv_c"], inp["k_pe"].reshape(T, 64)], axis=1)
    codes, scale = quantize_rows(rows)
    paged.write_fp8_rows(lat, case.slot_mapping, codes, scale, 576)
    assert np.array_equal(layer.mla_attn.kv_cache.cpu().numpy(), lat), "latent cache bytes differ"
    q_abs = bf16_values(layer.mla_attn.absorb_q(bf16_tensor(inp["q"], dev)))
    glob = logical_to_global(merged_ref, case.req, case.bt)
    ref_o, ref_l = od.sparse_mla_decode(q_abs, lambda s: od.gather_rows_fp8(lat, s, 576), glob, 256 ** -0.5, 512,
                                        case.params["attn_sink"].cpu().numpy())
    o_lat, lse = captured["out"]
    o_lat = bf16_values(o_lat[:, 0])
    _check_decode(o_lat, ref_o, "latent decode output")
    fin = np.isfinite(ref_l)
    assert np.all(np.abs(lse[:, 0].cpu().numpy()[fin] - ref_l[fin]) <= 2e-3 * np.maximum(1, np.abs(ref_l[fin])))
    w_uv = layer.mla_attn.W_UV_T.float().cpu().numpy().astype(np.float64)  # [H, 512, 256]
    ref_out = np.einsum("thc,hcv->thv", o_lat.astype(np.float64), w_uv).reshape(T, -1)
    mag = np.einsum("thc,hcv->thv", np.abs(o_lat.astype(np.float64)), np.abs(w_uv)).reshape(T, -1)
    got = bf16_values(out).astype(np.float64)
    assert np.all(np.abs(got - ref_out) <= 8e-3 * mag + 1e-6), "up-projected out differs"


def test_hca_prepare_and_attn_vs_oracle(dev):
    """The HCA layer's cache write + decode (attention.py:471-539): a
    prefill chunk then a decode step with one and three query rows; pool
    and state bytes exact, o_padded within tolerance."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(63)
    D, H, B, ring = 512, 64, 2, 192
    cfg = A.ernie5_5_config()
    lp, cp, rp = 8, 1, ring // 64
    perm = rng.permutation(B * (lp + cp + rp)).astype(np.int32)
    bt = perm[: B * lp].reshape(B, lp)
    comp_bt = perm[B * lp: B * (lp + cp)].reshape(B, cp)
    ring_pages = perm[B * (lp + cp):].reshape(B, rp)
    pages = len(perm)
    params = {"attn_sink": to_dev(rng.standard_normal(H).astype(np.float32), dev),
              "compressor.ape": to_dev((rng.standard_normal((128, D)) * 0.5).astype(np.float32), dev),
              "compressor.norm.weight": to_dev((1 + 0.1 * rng.standard_normal(D)).astype(np.float32), dev)}
    cos_sin = oi.yarn_cos_sin(np.arange(8) * 128, 64, cfg.compress_rope_theta)
    layer = A.select_ernie5_5_hca_cls("fp8")(A.ernie5_5_vllm_config(cfg, device=dev), "model.layers.0.attn",
                                             ring=ring, compress_cos_sin=to_dev(cos_sin, dev))
    layer.load_weights(params.items())
    layer.kv_cache = torch.zeros((pages, paged.fp8_page_bytes(D)), dtype=torch.uint8, device=dev)
    layer.state_cache = torch.zeros((B, 256, 2 * D), dtype=torch.bfloat16, device=dev)
    st = oh.HcaState(pages, D, B)
    state_slot = np.arange(B, dtype=np.int32)
    sinks = params["attn_sink"].cpu().numpy()
    pos0 = [0, 0]
    hist = {0: [], 1: []}  # latent rows by position, per request
    for counts in ([300, 257], [1, 3], [70, 2]):
        positions = np.concatenate([np.arange(p, p + n) for p, n in zip(pos0, counts)]).astype(np.int64)
        token_seq = np.concatenate([np.full(n, b, np.int32) for b, n in enumerate(counts)])
        qsl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        T = len(positions)
        slots = paged.slots_from_block_table(bt, token_seq, positions)
        kv = randn_bf16(rng, (T, D))
        kv_score = randn_bf16(rng, (T, 2 * D))
        q = randn_bf16(rng, (T, H, D))
        md = A.HCAStepMetadata(slot_mapping=to_dev(slots, dev), query_start_loc=to_dev(qsl, dev),
                               token_seq=to_dev(token_seq, dev), max_query_len=int(max(counts)),
                               comp_block_table=to_dev(comp_bt, dev), ring_pages=to_dev(ring_pages, dev),
                               state_slot=to_dev(state_slot, dev), max_seq_len=int(positions.max()) + 1)
        o_padded = torch.zeros((T, 64, D), dtype=torch.bfloat16, device=dev)
        with A.set_forward_context({layer.prefix: md}):
            layer._cache_and_attn(bf16_tensor(q, dev), bf16_tensor(kv, dev), bf16_tensor(kv_score, dev),
                                  to_dev(positions, dev), o_padded)
        torch.cuda.synchronize()
        oh.hca_write(st, kv, kv_score, positions, token_seq, qsl, slots, ring_pages, ring, comp_bt, state_slot,
                     params["compressor.ape"].cpu().numpy(), params["compressor.norm.weight"].cpu().numpy(),
                     cfg.rms_norm_eps, cos_sin)
        assert np.array_equal(layer.kv_cache.cpu().numpy(), st.pool), f"pool bytes differ after {counts}"
        assert np.array_equal(bf16_values(layer.state_cache).reshape(st.state.shape), st.state)
        for t in range(T):
            hist[int(token_seq[t])].append(kv[t])
        # each row attends its request's compressed entries 0..n_c-1 (as the
        # pool holds them) and the latent rows of its last w positions (by
        # content: the quantized rows written at those positions)
        ref_o = np.zeros((T, H, 512))
        for t in range(T):
            p, b = int(positions[t]), int(token_seq[t])
            n_c, w = (p + 1) // 128, min(p + 1, WINDOW)
            comp = od.gather_rows_fp8(st.pool, np.array([oh.comp_slot(comp_bt, b, j) for j in range(n_c)], np.int64),
                                      D) if n_c else np.zeros((0, D))
            wc, ws_ = quantize_rows(np.stack(hist[b][p - w + 1: p + 1]))
            kv_rows = np.concatenate([comp, wc_decode(wc, ws_)])
            ref_o[t] = od.sparse_mla_decode(q[t:t + 1], lambda s: kv_rows[s], np.arange(len(kv_rows))[None],
                                            D ** -0.5, 512, sinks)[0][0]
        _check_decode(bf16_values(o_padded), ref_o, f"o_padded after {counts}")
        pos0 = [p + n for p, n in zip(pos0, counts)]


@pytest.mark.parametrize("heads,padded", [(64, 64), (16, 64)])
def test_fp8_flash_mla_kernel_method(dev, heads, padded):
    """Ernie5_5FlashMLASparseImpl._fp8_flash_mla_kernel (attention.py:723-749):
    q [batch, seq, heads, 576], global indices, heads padded with -inf sinks."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(64 + heads)
    pages = 30
    rows = randn_bf16(rng, (pages * 64, 576))
    pool = np.zeros((pages, paged.fp8_page_bytes(576)), np.uint8)
    codes, scale = quantize_rows(rows)
    paged.write_fp8_rows(pool, np.arange(pages * 64), codes, scale, 576)
    b, s, W = 3, 1, 2176
    idx = rng.integers(0, pages * 64, (b, s, W)).astype(np.int32)
    idx[1, 0, 1000:] = -1
    q = randn_bf16(rng, (b, s, heads, 576))
    sinks = rng.standard_normal(heads).astype(np.float32)
    impl = A.Ernie5_5FlashMLASparseImpl(heads, 576, 256 ** -0.5, sinks=to_dev(sinks, dev),
                                        fp8_decode_padded_heads=padded)
    out, lse = impl._fp8_flash_mla_kernel(bf16_tensor(q, dev), to_dev(pool, dev), to_dev(idx, dev), None)
    assert out.shape == (b, s, heads, 512) and lse.shape == (b, s, heads)
    ref_o, ref_l = od.sparse_mla_decode(q.reshape(b * s, heads, 576), lambda sl: od.gather_rows_fp8(pool, sl, 576),
                                        idx.reshape(b * s, W), 256 ** -0.5, 512, sinks)
    _check_decode(bf16_values(out).reshape(b * s, heads, 512), ref_o, "fp8 kernel method")
    assert np.all(np.abs(lse.cpu().numpy().reshape(b * s, heads) - ref_l) <= 2e-3 * np.maximum(1, np.abs(ref_l)))


def test_bf16_flash_mla_kernel_method(dev):
    """_bf16_flash_mla_kernel (attention.py:751-789): flat bf16 rows viewed as
    [-1, 1, 576], topk_length, actual_num_heads padded to 16, caller's out."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(65)
    N, T, W, H = 64 * 12, 5, 300, 12
    cache = randn_bf16(rng, (N, 576))
    idx = rng.integers(0, N, (T, W)).astype(np.int32)
    lens = np.array([300, 1, 0, 150, 299], np.int32)
    q = randn_bf16(rng, (T, H, 576))
    sinks = rng.standard_normal(16).astype(np.float32)
    impl = A.Ernie5_5FlashMLASparseImpl(16, 576, 256 ** -0.5, sinks=to_dev(sinks, dev), prefill_padding=16)
    out = torch.zeros((T, 16, 512), dtype=torch.bfloat16, device=dev)
    o, lse = impl._bf16_flash_mla_kernel(bf16_tensor(q, dev), bf16_tensor(cache, dev).view(N, 1, 576),
                                         to_dev(idx, dev), topk_length=to_dev(lens, dev), actual_num_heads=H, out=out)
    assert o.shape == (T, H, 512)
    ref_o, _ = od.sparse_mla_decode(q, lambda sl: od.gather_rows_bf16(cache, sl), idx, 256 ** -0.5, 512, sinks[:H],
                                    lens)
    _check_decode(bf16_values(o), ref_o, "bf16 kernel method")


def test_indexer_metadata_builder_build(dev):
    """Ernie5_5IndexerMetadataBuilder.build (attention.py:652-691) with a stub
    parent build: prefill chunk ends pulled in by the window (never below
    the chunk start), decode seq_lens [num_reqs] and [num_reqs, next_n]
    windowed to max(seq_len - 128, 0), compared with the reference's torch
    expressions; too many decode entries are refused."""
    from ernie_kv import attention as A

    ks = torch.tensor([0, 0, 500, 1000], dtype=torch.int32, device=dev)
    ke = torch.tensor([1, 129, 700, 5000], dtype=torch.int32, device=dev)
    cases = [torch.tensor([0, 1, 127, 128, 129, 5000, 131072], dtype=torch.int32, device=dev),
             torch.tensor([[126, 127], [128, 129], [4000, 4001]], dtype=torch.int32, device=dev)]
    for seq_lens in cases:
        def base_build(prefix_len, common, fast_build, seq_lens=seq_lens):
            return A.IndexerMetadata(prefill=A.IndexerPrefill(chunks=[A.IndexerPrefillChunk(ks.clone(), ke.clone())]),
                                     decode=A.IndexerDecode(seq_lens=seq_lens.clone()))
        builder = A.Ernie5_5IndexerMetadataBuilder(WINDOW, max_num_reqs=8, device=dev, base_build=base_build,
                                                   max_query_len=3)
        md = builder.build(0, None)
        torch.cuda.synchronize()
        ref = torch.sub(seq_lens, WINDOW)
        ref.clamp_min_(0)
        assert md.decode.seq_lens.shape == seq_lens.shape
        assert torch.equal(md.decode.seq_lens, ref)
        assert torch.equal(md.prefill.chunks[0].cu_seqlen_ke, torch.maximum(ke - WINDOW, ks))
    small = A.Ernie5_5IndexerMetadataBuilder(
        WINDOW, max_num_reqs=2, device=dev,
        base_build=lambda *a: A.IndexerMetadata(decode=A.IndexerDecode(seq_lens=cases[0].clone())))
    with pytest.raises(ValueError):
        small.build(0, None)


@pytest.mark.parametrize("fp4", [False, True], ids=["fp8", "mxfp4"])
def test_dsa_prefill_chunk_vs_oracle(dev, fp4):
    """A chunked-prefill step through Ernie5_5DSAAttention._indexer_and_attn:
    1100 prefill rows of one request (positions 2500..3599) beside a decode
    row, so the indexer runs its many-row kernels (more rows than the fused
    filter takes) in workspace pieces.  Every row's top-k equals the exact
    path's (ekv_indexer_score[_fp4] + ekv_topk_select over the cache after
    the step); sampled rows equal the oracle's top-k and decode output; the
    per-row candidate counts equal the prefill chunk form of the metadata
    (cu_seqlen_ke - cu_seqlen_ks after the builder's window rewrite,
    attention.py:659-668); both caches' bytes equal the oracle's."""
    from ernie_kv import attention as A
    from ernie_kv import ops

    rng = np.random.default_rng(66)
    case = _dsa_setup(dev, rng, [3600, 5000], [1100, 1], fp4=fp4)
    T = case.T
    topk_buf = torch.full((T, TOPK), -7, dtype=torch.int32, device=dev)
    swa_buf = torch.full((T, TOPK + WINDOW), -7, dtype=torch.int32, device=dev)
    layer = _dsa_layer(case, topk_buf, swa_buf)
    layer.indexer.k_cache.kv_cache = to_dev(case.kc, dev)
    layer.mla_attn.kv_cache = to_dev(case.lat, dev)
    captured = {}
    orig = layer.mla_attn.impl._fp8_flash_mla_kernel

    def spy(*args, **kwargs):
        captured["out"] = orig(*args, **kwargs)
        return captured["out"]

    layer.mla_attn.impl._fp8_flash_mla_kernel = spy
    inp = case.inputs
    out = torch.zeros((T, 64 * 256), dtype=torch.bfloat16, device=dev)
    meta = {layer.mla_attn.prefix: case.md, layer.indexer.k_cache.prefix: case.md}
    pos_t = to_dev(case.positions, dev)
    with A.set_forward_context(meta):
        layer._indexer_and_attn(bf16_tensor(inp["hidden"], dev), bf16_tensor(inp["q_c"], dev), pos_t,
                                bf16_tensor(inp["q"], dev), bf16_tensor(inp["kv_c"], dev),
                                bf16_tensor(inp["k_pe"], dev), out)
    torch.cuda.synchronize()
    # the prefill chunk's metadata form: cu_seqlen_ks = start of each row's
    # request in the flattened K, cu_seqlen_ke = ks + pos + 1, windowed by the builder
    starts = np.array([0, 3600], np.int64)[case.req]
    ks = torch.tensor(starts, dtype=torch.int32, device=dev)
    ke = torch.tensor(starts + case.positions + 1, dtype=torch.int32, device=dev)
    builder = A.Ernie5_5IndexerMetadataBuilder(
        WINDOW, max_num_reqs=2, device=dev,
        base_build=lambda *a: A.IndexerMetadata(prefill=A.IndexerPrefill(chunks=[A.IndexerPrefillChunk(ks, ke)])))
    chunk = builder.build(0, None).prefill.chunks[0]
    lengths = layer.indexer._lengths_buf(T, dev)
    assert torch.equal((chunk.cu_seqlen_ke - chunk.cu_seqlen_ks).to(torch.int32), lengths)
    # all rows: the exact path over the cache after the step
    hid, qc = bf16_tensor(inp["hidden"], dev), bf16_tensor(inp["q_c"], dev)
    iq, ik, iw = layer.indexer._project(hid, qc)
    qp, kp = ops.indexer_prep(iq, ik, *layer.indexer._prep_args(dev), pos_t)
    L = int(case.md.max_seq_len)
    scores = torch.zeros((T, L), device=dev)
    args = (layer.indexer.k_cache.kv_cache, case.md.block_table, case.md.req_ids, lengths, L)
    if fp4:
        qv, qs, wf = ops.indexer_q_quant_fp4(qp, iw)
        ops.indexer_score_fp4(qv, qs, wf, *args, scores)
    else:
        q8, wf, dig = ops.indexer_q_quant(qp, iw)
        ops.indexer_score(dig, wf, *args, scores)
    ref_top = torch.full((T, TOPK), -9, dtype=torch.int32, device=dev)
    ops.topk_select(scores, lengths, TOPK, ref_top)
    assert torch.equal(topk_buf[:T], ref_top), "top-k differs from the exact path"
    top = topk_buf[:T].cpu().numpy()
    merged_ref = merge_swa_topk(top, case.positions, TOPK + WINDOW, WINDOW)
    assert np.array_equal(swa_buf[:T].cpu().numpy(), merged_ref), "merged rows differ"
    # caches: the oracle's inserts and appends of all T rows
    rq, rk = oi.indexer_prep(bf16_values(iq), bf16_values(ik), layer.indexer.k_norm_weight.cpu().numpy(),
                             layer.indexer.k_norm_bias.cpu().numpy(), 1e-6,
                             layer.indexer._prep_args(dev)[3][pos_t].cpu().numpy())
    kc = case.kc.copy()
    (om.k_insert if fp4 else oi.k_insert)(kc, rk, case.slot_mapping)
    assert np.array_equal(layer.indexer.k_cache.kv_cache.cpu().numpy(), kc), "indexer K cache bytes differ"
    lat = case.lat.copy()
    rows = np.concatenate([inp["kv_c"], inp["k_pe"].reshape(T, 64)], axis=1)
    codes, scale = quantize_rows(rows)
    paged.write_fp8_rows(lat, case.slot_mapping, codes, scale, 576)
    assert np.array_equal(layer.mla_attn.kv_cache.cpu().numpy(), lat), "latent cache bytes differ"
    # sampled rows against the oracle: top-k and the sparse decode
    sample = np.array([0, 1, 129, 700, 1098, 1099, 1100])
    lens = oi.windowed_lengths(case.positions, WINDOW)
    if fp4:
        rv, rs, rw = om.quantize_q(rq[sample], bf16_values(iw)[sample])
        otop, _ = om.indexer_topk(rv, rs, rw, kc, case.bt, case.req[sample], lens[sample], TOPK)
    else:
        codes_q, rw = oi.quantize_q(rq[sample], bf16_values(iw)[sample])
        otop, _ = oi.indexer_topk(codes_q, rw, kc, case.bt, case.req[sample], lens[sample], TOPK)
    assert np.array_equal(top[sample], otop), "sampled top-k rows differ from the oracle"
    q_abs = bf16_values(layer.mla_attn.absorb_q(bf16_tensor(inp["q"], dev)))[sample]
    glob = logical_to_global(merged_ref[sample], case.req[sample], case.bt)
    ref_o, _ = od.sparse_mla_decode(q_abs, lambda s: od.gather_rows_fp8(lat, s, 576), glob, 256 ** -0.5, 512,
                                    case.params["attn_sink"].cpu().numpy())
    o_lat = bf16_values(captured["out"][0][:, 0])[sample]
    _check_decode(o_lat, ref_o, "prefill rows' latent decode output")


def test_dsa_indexer_and_attn_graph_replay(dev):
    """Ernie5_5DSAAttention._indexer_and_attn captured in a HIP graph: the
    layer's launches take fixed workspaces and never synchronize the host, so
    each of three replays, with eager work and synchronizations between
    them, equals the eager call bit for bit (the step rewrites the same
    slots with the same rows, so it is idempotent)."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(67)
    case = _dsa_setup(dev, rng, [3000, 4500], [1, 3])
    T = case.T
    topk_buf = torch.full((16, TOPK), -7, dtype=torch.int32, device=dev)
    swa_buf = torch.full((16, TOPK + WINDOW), -7, dtype=torch.int32, device=dev)
    layer = _dsa_layer(case, topk_buf, swa_buf)
    layer.indexer.k_cache.kv_cache = to_dev(case.kc, dev)
    layer.mla_attn.kv_cache = to_dev(case.lat, dev)
    inp = {k: bf16_tensor(v, dev) for k, v in case.inputs.items()}
    out = torch.zeros((T, 64 * 256), dtype=torch.bfloat16, device=dev)
    meta = {layer.mla_attn.prefix: case.md, layer.indexer.k_cache.prefix: case.md}
    pos_t = to_dev(case.positions, dev)

    def step():
        with A.set_forward_context(meta):
            layer._indexer_and_attn(inp["hidden"], inp["q_c"], pos_t, inp["q"], inp["kv_c"], inp["k_pe"], out)

    def state():
        return [topk_buf[:T].clone(), swa_buf[:T].clone(), out.clone(), layer.indexer.k_cache.kv_cache.clone(),
                layer.mla_attn.kv_cache.clone()]

    step()
    torch.cuda.synchronize()
    ref = state()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for i in range(3):
        topk_buf.fill_(-1)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        got = state()
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"replay {i} differs from the eager call"
        step()  # eager work between replays
        torch.cuda.synchronize()


# ---------------------------------------------------------------- layer forwards
def _rel_err(got, ref):
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def _spy(obj, name, store):
    orig = getattr(obj, name)

    def wrapped(*args, **kwargs):
        out = orig(*args, **kwargs)
        store[name] = (args, kwargs, out)
        return out

    setattr(obj, name, wrapped)


@pytest.mark.parametrize("fp8_o_proj", [False, True], ids=["bf16-o-proj", "fp8-o-proj"])
def test_dsa_forward_vs_oracle(dev, fp8_o_proj):
    """Ernie5_5DSAAttention(vllm_config, prefix, topk_indices_buffer,
    swa_topk_buffer).forward(positions, hidden_states) (attention.py:1062-1203)
    with every weight loaded by name: the KV path's results against the
    oracle from the tensors the layer handed ``_indexer_and_attn`` (indexer K
    and latent cache bytes, top-k and merged rows exact, the latent decode
    within tolerance), and the layer output against an fp64 recomputation of
    the reference's output side (W_UV, VHA head mix, sigmoid gate, wo_b) from
    the oracle's decode.  With fp8_o_proj the wo_b input goes through
    sigmoid_mul_quant_fp8 (1 x 128 fp8 groups), so the output tolerance is
    the fp8 step's."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(71)
    case = _dsa_setup(dev, rng, [3000, 4500], [1, 3])
    T, H = case.T, 64
    hidden, q_lora = 256, 128
    w = dict(case.params)
    w.update({
        "fused_qkv_a_proj.weight": bf16_tensor(randn_bf16(rng, (q_lora + 512 + 64, hidden), hidden ** -0.5), dev),
        "q_a_layernorm.weight": bf16_tensor(1 + 0.1 * randn_bf16(rng, (q_lora,)), dev),
        "q_b_proj.weight": bf16_tensor(randn_bf16(rng, (H * 256, q_lora), q_lora ** -0.5), dev),
        "kv_a_layernorm.weight": bf16_tensor(1 + 0.1 * randn_bf16(rng, (512,)), dev),
        "o_gate.weight": bf16_tensor(randn_bf16(rng, (H * 256, q_lora), q_lora ** -0.5), dev),
        "wo_b.weight": bf16_tensor(randn_bf16(rng, (hidden, H * 256), (H * 256) ** -0.5), dev),
        "vha.U": bf16_tensor(randn_bf16(rng, (H, 16), 0.05), dev),
        "vha.V": bf16_tensor(randn_bf16(rng, (H, 16), 0.05), dev),
    })
    topk_buf = torch.full((16, TOPK), -7, dtype=torch.int32, device=dev)
    swa_buf = torch.full((16, TOPK + WINDOW), -7, dtype=torch.int32, device=dev)
    vc = A.ernie5_5_vllm_config(case.cfg, device=dev)
    layer = A.Ernie5_5DSAAttention(vc, "model.layers.3.attn", topk_buf, swa_buf, fp8_o_proj=fp8_o_proj)
    loaded = layer.load_weights(w.items())
    assert loaded == {n for n, _ in layer.named_parameters()}, "every parameter is loaded by name"
    layer.indexer.k_cache.kv_cache = to_dev(case.kc, dev)
    layer.mla_attn.kv_cache = to_dev(case.lat, dev)
    seen = {}
    _spy(layer, "_indexer_and_attn", seen)
    _spy(layer.mla_attn.impl, "_fp8_flash_mla_kernel", seen)
    hid = bf16_tensor(case.inputs["hidden"], dev)
    pos_t = to_dev(case.positions, dev)
    with A.set_forward_context({layer.mla_attn.prefix: case.md, layer.indexer.k_cache.prefix: case.md}):
        y = layer(pos_t, hid)
    torch.cuda.synchronize()
    assert y.shape == (T, hidden) and y.dtype == torch.bfloat16
    (_, q_c, _, q, kv_c_normed, k_pe, _), _, _ = seen["_indexer_and_attn"]
    # the KV path from the layer's own projected tensors
    case.inputs.update(q_c=bf16_values(q_c), q=bf16_values(q), kv_c=bf16_values(kv_c_normed),
                       k_pe=bf16_values(k_pe).reshape(T, 1, 64))
    kc_ref, top_ref = _oracle_indexer(case, layer.indexer, dev)
    assert np.array_equal(layer.indexer.k_cache.kv_cache.cpu().numpy(), kc_ref), "indexer K cache bytes differ"
    assert np.array_equal(topk_buf[:T].cpu().numpy(), top_ref), "top-k differs"
    merged_ref = merge_swa_topk(top_ref, case.positions, TOPK + WINDOW, WINDOW)
    assert np.array_equal(swa_buf[:T].cpu().numpy(), merged_ref), "merged rows differ"
    lat = case.lat.copy()
    codes, scale = quantize_rows(np.concatenate([case.inputs["kv_c"], case.inputs["k_pe"].reshape(T, 64)], axis=1))
    paged.write_fp8_rows(lat, case.slot_mapping, codes, scale, 576)
    assert np.array_equal(layer.mla_attn.kv_cache.cpu().numpy(), lat), "latent cache bytes differ"
    q_abs = bf16_values(layer.mla_attn.absorb_q(q))
    glob = logical_to_global(merged_ref, case.req, case.bt)
    ref_o, _ = od.sparse_mla_decode(q_abs, lambda s: od.gather_rows_fp8(lat, s, 576), glob, 256 ** -0.5, 512,
                                    case.params["attn_sink"].cpu().numpy())
    # the decode's latent output, as the impl returned it to the layer
    o_lat = seen["_fp8_flash_mla_kernel"][2][0][:, 0]
    _check_decode(bf16_values(o_lat), ref_o, "latent decode output")
    # the output side in fp64 from the oracle's decode
    f64 = lambda t: t.detach().float().cpu().numpy().astype(np.float64)  # noqa: E731
    w_uv = f64(layer.mla_attn.W_UV_T)                                     # [H, 512, 256]
    attn = np.einsum("thc,hcv->thv", ref_o, w_uv)                          # [T, H, 256]
    mix = f64(layer.vha.m)
    o = np.einsum("hg,tgv->thv", mix, attn).reshape(T, -1)
    gate = bf16_values(q_c).astype(np.float64) @ f64(layer.o_gate.weight).T
    ref_y = (o / (1.0 + np.exp(-gate))) @ f64(layer.wo_b.weight).T
    err = _rel_err(bf16_values(y).astype(np.float64), ref_y)
    assert err < (4e-2 if fp8_o_proj else 1.5e-2), f"layer output rel err {err}"


@pytest.mark.parametrize("fp8_o_proj", [False, True], ids=["bf16-o-proj", "fp8-o-proj"])
@pytest.mark.parametrize("cache", ["fp8", "bfloat16"])
def test_hca_forward_vs_oracle(dev, cache, fp8_o_proj):
    """The HCA layer built by select_ernie5_5_hca_cls(kv_cache_dtype)(vllm_config,
    prefix) with every weight loaded by name, forward(positions,
    hidden_states) (attention.py:471-539) over a prefill chunk and two
    decode steps (one and three query rows): the cache (fp8 pages, or bf16
    rows for the FlashInfer class) and state ring bytes against the oracle
    from the tensors the layer handed its KV path, o_padded within the
    decode tolerance, and the layer output against an fp64 recomputation of
    the output side (VHA mix, inverse RoPE of the rope part, grouped wo_a,
    sigmoid gate, wo_b) from the oracle's attention output.  With fp8_o_proj
    VHA + inverse RoPE + quant run in vha_inv_rope_fp8_quant and the wo_b
    input in sigmoid_mul_quant_fp8."""
    from ernie_kv import attention as A

    rng = np.random.default_rng(72)
    D, H, B, ring, hidden, q_lora, r, G = 512, 64, 2, 192, 512, 256, 256, 8
    cfg = A.ernie5_5_config(hidden_size=hidden, q_lora_rank=q_lora, o_lora_rank=r, max_position_embeddings=4096)
    lp, cp, rp = 8, 1, ring // 64
    perm = rng.permutation(B * (lp + cp + rp)).astype(np.int32)
    bt = perm[: B * lp].reshape(B, lp)
    comp_bt = perm[B * lp: B * (lp + cp)].reshape(B, cp)
    ring_pages = perm[B * (lp + cp):].reshape(B, rp)
    pages = len(perm)
    bf = lambda shape, s: bf16_tensor(randn_bf16(rng, shape, s), dev)  # noqa: E731
    w = {"attn_sink": to_dev(rng.standard_normal(H).astype(np.float32), dev),
         "compressor.ape": to_dev((rng.standard_normal((128, D)) * 0.5).astype(np.float32), dev),
         "compressor.norm.weight": to_dev((1 + 0.1 * rng.standard_normal(D)).astype(np.float32), dev),
         "compressor.fused_wkv_wgate.weight": bf((2 * D, hidden), hidden ** -0.5),
         "fused_wqa_wkv.weight": bf((q_lora + D, hidden), hidden ** -0.5),
         "q_norm.weight": bf16_tensor(1 + 0.1 * randn_bf16(rng, (q_lora,)), dev),
         "kv_norm.weight": bf16_tensor(1 + 0.1 * randn_bf16(rng, (D,)), dev),
         "wq_b.weight": bf((H * D, q_lora), q_lora ** -0.5),
         "wo_a": bf((G, r, (H // G) * D), ((H // G) * D) ** -0.5),
         "wo_b.weight": bf((hidden, G * r), (G * r) ** -0.5),
         "o_gate.weight": bf((G * r, q_lora), q_lora ** -0.5),
         "vha.U": bf((H, 16), 0.05), "vha.V": bf((H, 16), 0.05)}
    vc = A.ernie5_5_vllm_config(cfg, cache_dtype=cache, device=dev)
    cls = A.select_ernie5_5_hca_cls(cache)
    assert cls is (A.Ernie5_5HCAFlashMLAAttention if cache == "fp8" else A.Ernie5_5HCAFlashInferAttention)
    layer = cls(vc, "model.layers.0.attn", ring=ring, fp8_o_proj=fp8_o_proj)
    loaded = layer.load_weights(w.items())
    assert loaded == {n for n, _ in layer.named_parameters()}, "every parameter is loaded by name"
    bf16_cache = cache != "fp8"
    if bf16_cache:
        layer.kv_cache = torch.zeros((pages * 64, D), dtype=torch.bfloat16, device=dev)
    else:
        layer.kv_cache = torch.zeros((pages, paged.fp8_page_bytes(D)), dtype=torch.uint8, device=dev)
    layer.state_cache = torch.zeros((B, 256, 2 * D), dtype=torch.bfloat16, device=dev)
    st = oh.HcaState(pages, D, B, bf16=bf16_cache)
    state_slot = np.arange(B, dtype=np.int32)
    sinks = w["attn_sink"].cpu().numpy()
    cos_sin = layer.compress_cos_sin.cpu().numpy()
    rope = layer.rotary_emb.cos_sin_cache.cpu().numpy().astype(np.float64)
    f64 = lambda t: t.detach().float().cpu().numpy().astype(np.float64)  # noqa: E731
    pos0 = [0, 0]
    hist = {0: [], 1: []}
    for counts in ([300, 257], [1, 3], [70, 2]):
        positions = np.concatenate([np.arange(p, p + n) for p, n in zip(pos0, counts)]).astype(np.int64)
        token_seq = np.concatenate([np.full(n, b, np.int32) for b, n in enumerate(counts)])
        qsl = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        T = len(positions)
        slots = paged.slots_from_block_table(bt, token_seq, positions)
        md = A.HCAStepMetadata(slot_mapping=to_dev(slots, dev), query_start_loc=to_dev(qsl, dev),
                               token_seq=to_dev(token_seq, dev), max_query_len=int(max(counts)),
                               comp_block_table=to_dev(comp_bt, dev), ring_pages=to_dev(ring_pages, dev),
                               state_slot=to_dev(state_slot, dev), max_seq_len=int(positions.max()) + 1)
        seen = {}
        _spy(layer, "_prepare_and_attn_fn", seen)
        _spy(layer, "_cache_and_attn", seen)
        with A.set_forward_context({layer.prefix: md}):
            y = layer(to_dev(positions, dev), bf16_tensor(randn_bf16(rng, (T, hidden)), dev))
        torch.cuda.synchronize()
        assert y.shape == (T, hidden)
        (q, kv, kv_score, _, o_padded), _, _ = seen["_cache_and_attn"]
        qr = seen["_prepare_and_attn_fn"][0][1]
        q, kv, kv_score = bf16_values(q), bf16_values(kv), bf16_values(kv_score)
        oh.hca_write(st, kv, kv_score, positions, token_seq, qsl, slots, ring_pages, ring, comp_bt, state_slot,
                     w["compressor.ape"].cpu().numpy(), w["compressor.norm.weight"].cpu().numpy(), cfg.rms_norm_eps,
                     cos_sin)
        got_pool = layer.kv_cache.view(torch.uint8).reshape(pages, -1).cpu().numpy()
        assert np.array_equal(got_pool, st.pool), f"cache bytes differ after {counts}"
        assert np.array_equal(bf16_values(layer.state_cache).reshape(st.state.shape), st.state)
        for t in range(T):
            hist[int(token_seq[t])].append(kv[t])
        ref_o = np.zeros((T, H, D))
        for t in range(T):
            p, b = int(positions[t]), int(token_seq[t])
            n_c, wn = (p + 1) // 128, min(p + 1, WINDOW)
            cs_ = np.array([oh.comp_slot(comp_bt, b, j) for j in range(n_c)], np.int64)
            if bf16_cache:
                vals = bf16_values(layer.kv_cache).reshape(-1, D) if n_c else None
                comp = vals[cs_].astype(np.float64) if n_c else np.zeros((0, D))
                win = np.stack(hist[b][p - wn + 1: p + 1]).astype(np.float64)
            else:
                comp = od.gather_rows_fp8(st.pool, cs_, D) if n_c else np.zeros((0, D))
                wc, ws_ = quantize_rows(np.stack(hist[b][p - wn + 1: p + 1]))
                win = wc_decode(wc, ws_)
            kv_rows = np.concatenate([comp, win])
            ref_o[t] = od.sparse_mla_decode(q[t:t + 1], lambda s: kv_rows[s], np.arange(len(kv_rows))[None],
                                            D ** -0.5, 512, sinks)[0][0]
        _check_decode(bf16_values(o_padded[:, :H]), ref_o, f"o_padded after {counts}")
        # the output side in fp64 from the oracle's attention output
        o = np.einsum("hg,tgd->thd", f64(layer.vha.m), ref_o)
        cs = rope[positions]
        c, s = cs[:, None, :32], cs[:, None, 32:]
        e, od_ = o[..., 448::2].copy(), o[..., 449::2].copy()
        o[..., 448::2], o[..., 449::2] = e * c + od_ * s, od_ * c - e * s
        z = np.einsum("grk,tgk->tgr", f64(layer.wo_a), o.reshape(T, G, -1)).reshape(T, -1)
        gate = bf16_values(qr).astype(np.float64) @ f64(layer.o_gate.weight).T
        ref_y = (z / (1.0 + np.exp(-gate))) @ f64(layer.wo_b.weight).T
        err = _rel_err(bf16_values(y).astype(np.float64), ref_y)
        assert err < (5e-2 if fp8_o_proj else 1.5e-2), f"layer output rel err {err} after {counts}"
        pos0 = [p + n for p, n in zip(pos0, counts)]
