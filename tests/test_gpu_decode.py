"""GPU parity: sparse MLA decode with sink vs the fp64 oracle.

Tolerance (bf16 outputs): |out - ref| <= 2e-3 + 2e-2 * |ref|; lse within 2e-3.
"""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, bf16_values, permuted_block_table, randn_bf16, to_dev
from oracle import decode as od
from oracle import paged
from oracle.fp8 import quantize_rows
from oracle.merge import logical_to_global

pytestmark = pytest.mark.gpu
RTOL, ATOL = 2e-2, 2e-3


def _fp8_pool(rng, pages, dim, scale=1.0):
    rows = randn_bf16(rng, (pages * 64, dim), scale)
    pool = np.zeros((pages, paged.fp8_page_bytes(dim)), np.uint8)
    c, s = quantize_rows(rows)
    paged.write_fp8_rows(pool, np.arange(pages * 64), c, s, dim)
    return pool


def _check(out_t, lse_t, ref_o, ref_l, H, p_bound=0.0):
    got = bf16_values(out_t)[:, :H].astype(np.float64)
    err = np.abs(got - ref_o)
    assert np.all(err <= ATOL + RTOL * np.abs(ref_o) + p_bound), f"max err {err.max()}"
    if lse_t is not None:
        gl = lse_t.cpu().numpy().astype(np.float64)
        fin = np.isfinite(ref_l)
        assert np.array_equal(np.isfinite(gl), fin)
        assert np.all(np.abs(gl[fin] - ref_l[fin]) <= 2e-3 * np.maximum(1.0, np.abs(ref_l[fin])))


@pytest.mark.parametrize("dim,heads,width", [(576, 64, 2176), (576, 16, 160), (512, 64, 200), (576, 64, 33)])
@pytest.mark.parametrize("with_sink", [False, True])
def test_decode_fp8_global_indices(dev, dim, heads, width, with_sink):
    from ernie_kv import ops

    rng = np.random.default_rng(dim + heads + width + int(with_sink))
    T, pages = 4, 48
    pool = _fp8_pool(rng, pages, dim)
    idx = rng.integers(0, pages * 64, (T, width)).astype(np.int32)
    idx[:, -5:] = -1
    idx[1, ::7] = -1
    idx[3, :] = -1  # a row with nothing to attend to
    q = randn_bf16(rng, (T, heads, dim))
    sinks = rng.standard_normal(heads).astype(np.float32) if with_sink else None
    if with_sink:
        sinks[0] = -np.inf
    scale = 256 ** -0.5
    out = torch.zeros((T, heads, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((T, heads), dtype=torch.float32, device=dev)
    ops.sparse_mla_decode(bf16_tensor(q, dev), to_dev(pool, dev), to_dev(idx, dev), scale, out, lse,
                          sinks=None if sinks is None else to_dev(sinks, dev))
    ref_o, ref_l = od.sparse_mla_decode(q, lambda s: od.gather_rows_fp8(pool, s, dim), idx, scale, 512, sinks)
    _check(out, lse, ref_o, ref_l, heads)


def test_decode_logical_indices_block_table(dev):
    """Request-local indices converted through the block table in-kernel."""
    from ernie_kv import ops

    rng = np.random.default_rng(99)
    T, B, P, dim, H, W = 5, 3, 10, 576, 64, 300
    bt = permuted_block_table(rng, B, P)
    pool = _fp8_pool(rng, B * P, dim)
    req = rng.integers(0, B, T).astype(np.int32)
    logical = rng.integers(0, P * 64, (T, W)).astype(np.int32)
    logical[:, 250:] = -1
    lengths = np.array([300, 10, 0, 299, 128], np.int32)
    q = randn_bf16(rng, (T, H, dim))
    sinks = rng.standard_normal(H).astype(np.float32)
    out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
    ops.sparse_mla_decode(bf16_tensor(q, dev), to_dev(pool, dev), to_dev(logical, dev), 256 ** -0.5, out, lse,
                          sinks=to_dev(sinks, dev), lengths=to_dev(lengths, dev), block_table=to_dev(bt, dev),
                          req_ids=to_dev(req, dev))
    glob = logical_to_global(logical, req, bt)
    ref_o, ref_l = od.sparse_mla_decode(q, lambda s: od.gather_rows_fp8(pool, s, dim), glob, 256 ** -0.5, 512,
                                        sinks, lengths)
    _check(out, lse, ref_o, ref_l, H)


def test_decode_bf16_cache(dev):
    """The bf16 path views the cache as flat rows [-1, 1, 576] (attention.py:761-763)."""
    from ernie_kv import ops

    rng = np.random.default_rng(123)
    T, rows, dim, H, W = 3, 64 * 20, 576, 64, 257
    cache = randn_bf16(rng, (rows, dim))
    idx = rng.integers(0, rows, (T, W)).astype(np.int32)
    idx[0, 100:] = -1
    q = randn_bf16(rng, (T, H, dim))
    sinks = rng.standard_normal(H).astype(np.float32)
    out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
    ops.sparse_mla_decode(bf16_tensor(q, dev), bf16_tensor(cache, dev).view(-1, 64, dim), to_dev(idx, dev),
                          256 ** -0.5, out, lse, sinks=to_dev(sinks, dev), cache_bf16=True)
    ref_o, ref_l = od.sparse_mla_decode(q, lambda s: od.gather_rows_bf16(cache, s), idx, 256 ** -0.5, 512, sinks)
    _check(out, lse, ref_o, ref_l, H)


def test_decode_ragged_rows_workspace_reuse(dev):
    """Batches of 32-64 query rows (8, 4 and 2 splits per row) and one of 8
    rows (10 splits) through one workspace, rows ragged from empty to full.
    Rows of a few entries that nearly cancel make the bf16 rounding of the
    softmax weights before P V (which FlashMLA shares) visible against the
    fp64 oracle: the check allows that rounding's bound (oracle ``p_bound``)
    on top of the tolerance."""
    from ernie_kv import ops

    rng = np.random.default_rng(777)
    dim, pages = 576, 64
    pool = to_dev(_fp8_pool(rng, pages, dim), dev)
    pool_np = pool.cpu().numpy()
    ws = ops.decode_workspace(64, 64, 2176, dev)
    for T, H, W in [(32, 64, 2176), (8, 64, 300), (64, 16, 1152), (40, 64, 40)]:
        idx = rng.integers(0, pages * 64, (T, W)).astype(np.int32)
        idx[:, -3:] = -1
        lengths = rng.integers(0, W + 1, T).astype(np.int32)
        lengths[0], lengths[-1] = 0, W
        q = randn_bf16(rng, (T, H, dim))
        sinks = rng.standard_normal(H).astype(np.float32)
        out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
        lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
        ops.sparse_mla_decode(bf16_tensor(q, dev), pool, to_dev(idx, dev), 256 ** -0.5, out, lse,
                              sinks=to_dev(sinks, dev), lengths=to_dev(lengths, dev), workspace=ws)
        ref_o, ref_l, pb = od.sparse_mla_decode(q, lambda s: od.gather_rows_fp8(pool_np, s, dim), idx, 256 ** -0.5,
                                                512, sinks, lengths, p_bound=True)
        _check(out, lse, ref_o, ref_l, H, pb)
