"""Page-format transcoders on the GPU against the oracle, bit for bit:
export of this library's latent pages to fp8_ds_mla pages (with page maps
and skipped ids), import of fp8_ds_mla pages with arbitrary tile scales, and
the decode over imported pages equal to the decode over the originals."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, randn_bf16, to_dev
from oracle import pages as op
from oracle import paged
from oracle.fp8 import bf16_bits, quantize_rows

pytestmark = pytest.mark.gpu


def _own_pages(rng, n):
    cache = np.zeros((n, paged.fp8_page_bytes(576)), np.uint8)
    rows = (rng.standard_normal((n * 64, 576)) * np.exp(rng.uniform(-6, 6, (n * 64, 1)))).astype(np.float32)
    rows[7] = 0.0
    codes, scale = quantize_rows(rows)
    paged.write_fp8_rows(cache, np.arange(n * 64), codes, scale, 576)
    return cache


def test_export_fp8_ds_mla_pages(dev):
    from ernie_kv import ops

    rng = np.random.default_rng(5)
    cache = _own_pages(rng, 9)
    src = np.array([4, 0, 8, -1, 3, 99, 7], np.int32)    # -1 and 99 skipped
    dst = np.array([0, 5, 2, 1, 4, 3, 6], np.int32)
    stride = ops.ds_mla_page_stride()
    out = torch.full((7, stride), 171, dtype=torch.uint8, device=dev)
    ops.export_fp8_ds_mla_pages(to_dev(cache, dev), to_dev(src, dev), out, to_dev(dst, dev))
    ref = np.full((7, stride), 171, np.uint8)
    op.export_pages(cache, src, ref, dst)
    assert np.array_equal(out.cpu().numpy(), ref)


def test_import_fp8_ds_mla_pages(dev):
    from ernie_kv import ops

    rng = np.random.default_rng(6)
    n = 6
    stride = ops.ds_mla_page_stride()
    ds = np.zeros((n, stride), np.uint8)
    rows = ds[:, : 64 * 656].reshape(n, 64, 656)
    rows[:, :, :512] = rng.integers(0, 126, (n, 64, 512)) | (rng.integers(0, 2, (n, 64, 512)) << 7)
    tiles = (rng.uniform(0.5, 2.0, (n, 64, 4)) * 10.0 ** rng.uniform(-4, 4, (n, 64, 1))).astype(np.float32)
    tiles[0, 3] = 0.0                         # an all-zero row
    rows[:, :, 512:528] = tiles.view(np.uint8).reshape(n, 64, 16)
    rows[:, :, 528:] = bf16_bits((rng.standard_normal((n, 64, 64)) * 3).astype(np.float32)).view(np.uint8).reshape(
        n, 64, 128)
    rows[0, 3, 528:] = 0
    src = np.array([5, 1, 2, 0], np.int32)
    cache = torch.full((4, paged.fp8_page_bytes(576) + 64), 99, dtype=torch.uint8, device=dev)
    ops.import_fp8_ds_mla_pages(to_dev(ds, dev), to_dev(src, dev), cache)
    ref = np.full((4, paged.fp8_page_bytes(576) + 64), 99, np.uint8)
    op.import_pages(ds, src, ref)
    assert np.array_equal(cache.cpu().numpy(), ref)


def test_decode_over_exported_then_imported_pages(dev):
    """A connector round trip (export, then import with page p moved to
    perm[p]) leaves the decode's output unchanged, bit for bit: the values are
    the same, and a row requantized to half the scale with doubled codes
    scales every product by powers of two only."""
    from ernie_kv import ops

    rng = np.random.default_rng(7)
    P = 8
    cache = to_dev(_own_pages(rng, P), dev)
    ds = torch.zeros((P, ops.ds_mla_page_stride()), dtype=torch.uint8, device=dev)
    perm = rng.permutation(P).astype(np.int32)
    ops.export_fp8_ds_mla_pages(cache, to_dev(np.arange(P, dtype=np.int32), dev), ds)
    back = torch.zeros_like(cache)
    ops.import_fp8_ds_mla_pages(ds, to_dev(np.arange(P, dtype=np.int32), dev), back, to_dev(perm, dev))
    T, H, W = 4, 16, 300
    q = bf16_tensor(randn_bf16(rng, (T, H, 576)), dev)
    idx = rng.integers(0, P * 64, (T, W)).astype(np.int32)
    idx_moved = (perm[idx // 64] * 64 + idx % 64).astype(np.int32)
    sinks = torch.zeros(H, device=dev)
    outs = []
    for c, ix in ((cache, idx), (back, idx_moved)):
        o = torch.empty((T, H, 512), dtype=torch.bfloat16, device=dev)
        lse = torch.empty((T, H), dtype=torch.float32, device=dev)
        ops.sparse_mla_decode(q, c, to_dev(ix, dev), 256 ** -0.5, o, lse, sinks=sinks)
        outs.append((o, lse))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
