"""The path's torch operators (torch.ops.ernie_kv.*, ernie_kv.torch_ops):
each writes, in place, exactly what the ernie_kv.ops wrapper it registers
writes on the same inputs (bit for bit: the same kernels behind the
dispatcher), for the six operators the plugin's adapters call and the two
fused forms the layers use."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, permuted_block_table, randn_bf16, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tops(dev):
    import ernie_kv.torch_ops  # noqa: F401  (registers the operators)

    return torch.ops.ernie_kv


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.uint8) if a.dtype != torch.uint8 else a,
                       b.view(torch.uint8) if b.dtype != torch.uint8 else b)


def test_append_and_k_insert_ops(dev, tops):
    from ernie_kv import ops

    rng = np.random.default_rng(81)
    T, pages = 150, 8
    rows = bf16_tensor(randn_bf16(rng, (T, 576)), dev)
    k = bf16_tensor(randn_bf16(rng, (T, 128)), dev)
    slots = to_dev(rng.permutation(pages * 64)[:T].astype(np.int64), dev)
    slots[3] = -1
    c1 = torch.full((pages, 64 * 580), 7, dtype=torch.uint8, device=dev)
    c2 = c1.clone()
    ops.kv_append_quant(rows, slots, c1)
    tops.kv_append_quant(rows, slots, c2)
    k1 = torch.full((pages, 64 * 132), 7, dtype=torch.uint8, device=dev)
    k2 = k1.clone()
    ops.indexer_k_insert(k, slots, k1)
    tops.indexer_k_insert(k, slots, k2)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2) and not torch.equal(c1, torch.full_like(c1, 7))
    assert torch.equal(k1, k2) and not torch.equal(k1, torch.full_like(k1, 7))


def test_indexer_topk_merge_and_decode_ops(dev, tops):
    from ernie_kv import ops

    rng = np.random.default_rng(82)
    B, P, H = 3, 48, 64
    ctx = [3000, 2050, 700]
    bt = to_dev(permuted_block_table(rng, B, P), dev)
    kcache = torch.zeros((B * P, 64 * 132), dtype=torch.uint8, device=dev)
    latent = torch.zeros((B * P, 64 * 580), dtype=torch.uint8, device=dev)
    for b in range(B):
        pos = np.arange(ctx[b])
        sl = to_dev((bt[b].cpu().numpy()[pos // 64].astype(np.int64) * 64 + pos % 64), dev)
        ops.indexer_k_insert(bf16_tensor(randn_bf16(rng, (ctx[b], 128)), dev), sl, kcache)
        ops.kv_append_quant(bf16_tensor(randn_bf16(rng, (ctx[b], 576)), dev), sl, latent)
    q8, wf, digits = ops.indexer_q_quant(bf16_tensor(randn_bf16(rng, (B, H, 128)), dev),
                                         bf16_tensor(randn_bf16(rng, (B, H)), dev))
    req = torch.arange(B, dtype=torch.int32, device=dev)
    positions = torch.tensor([c - 1 for c in ctx], dtype=torch.int64, device=dev)
    lengths = torch.tensor([max(c - 128, 0) for c in ctx], dtype=torch.int32, device=dev)
    L = max(ctx)
    outs = []
    for route in ("ops", "torch"):
        ws = ops.indexer_topk_workspace(B, L, dev)
        topk = torch.full((B, 2048), 5, dtype=torch.int32, device=dev)
        merged = torch.full((B, 2176), 5, dtype=torch.int32, device=dev)
        topk2 = torch.full((B, 2048), 5, dtype=torch.int32, device=dev)
        merged2 = torch.full((B, 2176), 5, dtype=torch.int32, device=dev)
        out = torch.zeros((B, H, 512), dtype=torch.bfloat16, device=dev)
        lse = torch.zeros((B, H), dtype=torch.float32, device=dev)
        q = bf16_tensor(np.random.default_rng(83).standard_normal((B, H, 576)).astype(np.float32), dev)
        sinks = torch.linspace(-1.0, 1.0, H, device=dev)
        dws = ops.decode_workspace(B, H, 2176, dev)
        if route == "ops":
            ops.indexer_topk(q8, digits, wf, kcache, bt, req, lengths, L, topk, ws)
            ops.merge_swa_topk(topk, merged, positions, 128)
            ops.indexer_topk_merged(q8, digits, wf, kcache, bt, req, lengths, L, topk2, ws, merged=merged2,
                                    positions=positions, window=128)
            ops.sparse_mla_decode(q, latent, merged, 256 ** -0.5, out, lse, sinks=sinks, block_table=bt, req_ids=req,
                                  workspace=dws)
        else:
            tops.indexer_topk(q8, digits, wf, kcache, bt, req, lengths, L, topk, ws)
            tops.merge_swa_topk(topk, merged, positions, 128)
            tops.indexer_topk_merged(q8, digits, wf, kcache, bt, req, lengths, L, topk2, ws, merged2, positions, 128)
            tops.sparse_mla_decode(q, latent, merged, 256 ** -0.5, out, lse, sinks=sinks, block_table=bt, req_ids=req,
                                workspace=dws)
        torch.cuda.synchronize()
        outs.append((topk, merged, topk2, merged2, out, lse))
    a, b = outs
    for x, y in zip(a, b):
        assert _same(x, y)
    assert int((a[0] >= 0).sum()) == sum(min(2048, max(c - 128, 0)) for c in ctx)
    assert torch.equal(a[1], a[3]) and torch.equal(a[0], a[2])
    assert torch.isfinite(a[4].float()).all() and float(a[4].float().abs().sum()) > 0


@pytest.mark.parametrize("step", [False, True])
def test_hca_write_ops(dev, tops, step):
    import bench
    from ernie_kv import ops

    st = bench.build_hca_decode(torch, ops, 84, ctxs=[3000, 5000, 256, 129])
    runs = []
    for route in ("ops", "torch"):
        pool, state = st["pool"].clone(), st["state"].clone()
        wws = ops.hca_write_workspace(st["B"], st["D"], dev)
        idx = torch.full_like(st["idx"], 5)
        lens = torch.full_like(st["lens"], 5)
        f = ops if route == "ops" else tops
        common = (st["latent"], st["kv_score"], st["slots"], st["positions"], st["token_seq"], st["qsl"], st["R"],
                  state, st["state_slot"], st["ape"], st["norm_w"], 1e-6, st["cos_sin"], st["comp_bt"],
                  st["ring_pages"], st["ring"], pool)
        if step:
            f.hca_write_step(*common, 128, idx, lens, workspace=wws)
        else:
            f.hca_write(*common, workspace=wws)
        torch.cuda.synchronize()
        runs.append((pool, state, idx, lens))
    (p1, s1, i1, l1), (p2, s2, i2, l2) = runs
    assert torch.equal(p1, p2) and _same(s1, s2)
    assert not torch.equal(p1, st["pool"])  # the rows were written
    if step:
        assert torch.equal(i1, i2) and torch.equal(l1, l2) and int(l1[0]) == 3000 // 128 + 128
