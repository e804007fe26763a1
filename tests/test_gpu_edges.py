"""Empty batches: every op of the path called with zero query rows (or zero
pages) returns without error and leaves the caller's buffers as they were,
as a scheduler step that carries no tokens for a layer would call them."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_empty_batches(dev):
    from ernie_kv import ops

    pages = 4
    cache = torch.full((pages, 64 * 580), 7, dtype=torch.uint8, device=dev)
    kcache = torch.full((pages, 64 * 132), 7, dtype=torch.uint8, device=dev)
    before_c, before_k = cache.clone(), kcache.clone()
    no_slots = torch.empty(0, dtype=torch.int64, device=dev)
    ops.kv_append_quant(torch.empty((0, 576), dtype=torch.bfloat16, device=dev), no_slots, cache)
    ops.indexer_k_insert(torch.empty((0, 128), dtype=torch.bfloat16, device=dev), no_slots, kcache)

    # indexer top-k (with the merged rows) over no query rows
    bt = torch.arange(pages, dtype=torch.int32, device=dev).view(1, pages)
    q8 = torch.empty((0, 64, 128), dtype=torch.uint8, device=dev)
    digits = torch.empty((0, 3, 64, 128), dtype=torch.int8, device=dev)
    w = torch.empty((0, 64), dtype=torch.float32, device=dev)
    i32 = torch.empty(0, dtype=torch.int32, device=dev)
    topk = torch.empty((0, 2048), dtype=torch.int32, device=dev)
    merged = torch.empty((0, 2176), dtype=torch.int32, device=dev)
    ws = ops.indexer_topk_workspace(0, 256, dev)
    ops.indexer_topk(q8, digits, w, kcache, bt, i32, i32, 256, topk, ws)
    ops.indexer_topk_merged(q8, digits, w, kcache, bt, i32, i32, 256, topk, ws, merged=merged,
                            positions=no_slots, window=128)
    ops.merge_swa_topk(topk, merged, no_slots, 128)

    # sparse MLA decode over no query rows
    out = torch.empty((0, 64, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((0, 64), dtype=torch.float32, device=dev)
    q = torch.empty((0, 64, 576), dtype=torch.bfloat16, device=dev)
    ops.sparse_mla_decode(q, cache, torch.empty((0, 2176), dtype=torch.int32, device=dev), 0.0625, out, lse,
                          sinks=torch.zeros(64, device=dev))

    # the HCA write of a step with no sequences and no rows
    D = 576
    pool = torch.full((pages, 64 * (D + 4)), 7, dtype=torch.uint8, device=dev)
    before_p = pool.clone()
    ops.hca_write_step(torch.empty((0, D), dtype=torch.bfloat16, device=dev),
                       torch.empty((0, 2 * D), dtype=torch.bfloat16, device=dev), no_slots, no_slots, i32,
                       torch.zeros(1, dtype=torch.int32, device=dev), 0, None, None,
                       torch.zeros((128, D), device=dev), torch.ones(D, device=dev), 1e-6,
                       torch.zeros((4, 64), device=dev), torch.zeros((1, 1), dtype=torch.int32, device=dev),
                       torch.zeros((1, 2), dtype=torch.int32, device=dev), 128, pool, 128,
                       torch.empty((0, 256), dtype=torch.int32, device=dev), i32)

    # fp8_ds_mla page export / import of no pages
    out_pages = torch.full((pages, ops.ds_mla_page_stride()), 7, dtype=torch.uint8, device=dev)
    ops.export_fp8_ds_mla_pages(cache, i32, out_pages)
    ops.import_fp8_ds_mla_pages(out_pages, i32, cache)

    torch.cuda.synchronize()
    assert torch.equal(cache, before_c) and torch.equal(kcache, before_k) and torch.equal(pool, before_p)
    assert torch.equal(out_pages, torch.full_like(out_pages, 7))
