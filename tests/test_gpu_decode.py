"""GPU parity: sparse MLA decode with sink vs the fp64 oracle.

Tolerance (bf16 outputs): |out - ref| <= 2e-3 + 2e-2 * |ref|; lse within 2e-3.
"""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, bf16_values, permuted_block_table, randn_bf16, to_dev
from oracle.fp8 import bf16_round as bf16_round_np
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


def _check(out_t, lse_t, ref_o, ref_l, H):
    got = bf16_values(out_t)[:, :H].astype(np.float64)
    err = np.abs(got - ref_o)
    allow = ATOL + RTOL * np.abs(ref_o)
    print(f"decode worst error: {float((err / allow).max()):.3f} of the allowance, max abs {float(err.max()):.2e}")
    bad = err > allow
    assert not bad.any(), f"max err {err.max()}; first miss at {np.argwhere(bad)[0]}"
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
    """Batches of 32-64 query rows and one of 8 rows through one workspace,
    rows ragged from empty to full.  Rows of a few entries that nearly
    cancel (seed 777: row 30, head 42 of the first batch) expose a softmax
    weight carried in one bf16 before P V; the kernel's hi/lo pair keeps
    them within the plain tolerance."""
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
        ref_o, ref_l = od.sparse_mla_decode(q, lambda s: od.gather_rows_fp8(pool_np, s, dim), idx, 256 ** -0.5,
                                            512, sinks, lengths)
        _check(out, lse, ref_o, ref_l, H)


def test_decode_cancelling_pair(dev):
    """Two entries whose values are exact negatives and whose keys give
    softmax weights differing by ~1e-3: the output is a small difference of
    two large terms.  A weight rounded once to bf16 (relative error up to
    2^-9) moves it by up to ~4x the tolerance; the hi/lo weights do not."""
    from ernie_kv import ops

    rng = np.random.default_rng(5)
    dim, H, T = 576, 64, 16
    v = randn_bf16(rng, (1, dim), 2.0)
    rows = np.concatenate([v, -v, np.zeros((62, dim), np.float32)])
    pool = np.zeros((1, paged.fp8_page_bytes(dim)), np.uint8)
    c, sc = quantize_rows(rows)
    paged.write_fp8_rows(pool, np.arange(64), c, sc, dim)
    k0 = od.gather_rows_fp8(pool, np.array([0]), dim)[0]
    # q . (k0 - k1) = 2 q . k0 sets the weight ratio: choose q along k0 with
    # a per-row small dot product (weights e^{+-x}, x ~ 1e-4 .. 1e-2)
    q = np.zeros((T, H, dim), np.float32)
    for t in range(T):
        target = 10.0 ** rng.uniform(-4, -2) * 16.0 / 2.0
        q[t] = (k0 * target / float(k0 @ k0))[None, :]
    q = bf16_round_np(q)
    idx = np.tile(np.array([[0, 1]], np.int32), (T, 1))
    out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
    ops.sparse_mla_decode(bf16_tensor(q, dev), to_dev(pool, dev), to_dev(idx, dev), 256 ** -0.5, out, lse)
    ref_o, ref_l = od.sparse_mla_decode(q, lambda s: od.gather_rows_fp8(pool, s, dim), idx, 256 ** -0.5, 512)
    assert np.abs(ref_o).max() < 0.05 * np.abs(k0).max()  # the two terms nearly cancel
    _check(out, lse, ref_o, ref_l, H)


def test_decode_one_workspace_serves_smaller_calls(dev):
    """A workspace sized for (64 rows, 64 heads, 2176 entries) serves every
    call with fewer rows, heads or entries (workgroup counts grow with the
    shape); a smaller workspace is refused, not replaced."""
    from ernie_kv import _lib, ops

    rng = np.random.default_rng(4242)
    dim, pages = 576, 40
    pool_np = _fp8_pool(rng, pages, dim)
    pool = to_dev(pool_np, dev)
    ws = ops.decode_workspace(64, 64, 2176, dev)
    lib = _lib.load()
    full = lib.ekv_sparse_mla_decode_workspace_size(64, 64, 2176)
    for T in range(1, 65):
        for W in (1, 33, 1024, 1025, 2176):
            assert lib.ekv_sparse_mla_decode_workspace_size(T, 64, W) <= full
    for T, H, W in [(48, 64, 2176), (1, 64, 2176), (7, 16, 900), (63, 64, 1500), (64, 64, 2176), (33, 32, 64)]:
        idx = rng.integers(0, pages * 64, (T, W)).astype(np.int32)
        lengths = rng.integers(1, W + 1, T).astype(np.int32)
        q = randn_bf16(rng, (T, H, dim))
        sinks = rng.standard_normal(H).astype(np.float32)
        out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
        lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
        ops.sparse_mla_decode(bf16_tensor(q, dev), pool, to_dev(idx, dev), 256 ** -0.5, out, lse,
                              sinks=to_dev(sinks, dev), lengths=to_dev(lengths, dev), workspace=ws)
        ref_o, ref_l = od.sparse_mla_decode(q, lambda s: od.gather_rows_fp8(pool_np, s, dim), idx, 256 ** -0.5,
                                            512, sinks, lengths)
        _check(out, lse, ref_o, ref_l, H)
    small = ops.decode_workspace(8, 64, 300, dev)
    q = torch.zeros((48, 64, dim), dtype=torch.bfloat16, device=dev)
    idx = torch.zeros((48, 2176), dtype=torch.int32, device=dev)
    out = torch.zeros((48, 64, 512), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="workspace too small"):
        ops.sparse_mla_decode(q, pool, idx, 0.1, out, workspace=small)


def _hca_like_rows(rng, ctxs, rows_per_seq, pages, ring=192):
    """Index rows of HCA decode at the given contexts: per query row the
    compressed entries (ctx // 128 of them) then its 128-row window, as
    random slots of an fp8 pool (the decode is order-free)."""
    pos = np.concatenate([np.arange(c - rows_per_seq, c) for c in ctxs])
    n_c = (pos + 1) // 128
    w = np.minimum(pos + 1, 128)
    lens = (n_c + w).astype(np.int32)
    width = int(max(ctxs) // 128 + ring)
    idx = rng.integers(0, pages * 64, (len(pos), width)).astype(np.int32)
    for t, n in enumerate(lens):
        idx[t, n:] = -1
    return idx, lens


@pytest.mark.parametrize("case", ["mtp_1m", "hca_b64"])
def test_decode_hca_shapes_vs_oracle(dev, case):
    """The decode at the widths the HCA layers run: the multi-token workload
    (8 x 262,144 + 1 x 1,048,576 contexts, 3 rows per sequence, index rows
    up to 8,320 of width 8,384) and the 64-sequence step (contexts
    8K-128K, up to 1,152 compressed + 128 window entries)."""
    from ernie_kv import ops

    rng = np.random.default_rng(2026 if case == "mtp_1m" else 2027)
    dim, H, pages = 576, 64, 256
    pool_np = _fp8_pool(rng, pages, dim)
    pool = to_dev(pool_np, dev)
    if case == "mtp_1m":
        idx, lens = _hca_like_rows(rng, [262144] * 8 + [1048576], 3, pages)
    else:
        ctxs = rng.integers(8192, 131072, 64)
        idx, lens = _hca_like_rows(rng, list(ctxs), 1, pages, ring=128)
    T, W = idx.shape
    q = randn_bf16(rng, (T, H, dim))
    sinks = rng.standard_normal(H).astype(np.float32)
    out = torch.zeros((T, H, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((T, H), dtype=torch.float32, device=dev)
    ops.sparse_mla_decode(bf16_tensor(q, dev), pool, to_dev(idx, dev), 256 ** -0.5, out, lse,
                          sinks=to_dev(sinks, dev), lengths=to_dev(lens, dev))
    ref_o, ref_l = od.sparse_mla_decode(q, lambda s: od.gather_rows_fp8(pool_np, s, dim), idx, 256 ** -0.5, 512,
                                        sinks, lens)
    _check(out, lse, ref_o, ref_l, H)
