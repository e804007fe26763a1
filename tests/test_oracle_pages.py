"""Pins of the page-format transcoders (CPU): the fp8_ds_mla row layout
(known-answer row), the page stride's closed form, export losslessness
(dequantized values equal; import after export gives the same values back)
and import as the build's row quantization of the dequantized row."""

import numpy as np

from oracle import pages as op
from oracle import paged
from oracle.fp8 import bf16_bits, decode_e4m3, quantize_rows


def _own_pages(rng, n):
    cache = np.zeros((n, paged.fp8_page_bytes(576)), np.uint8)
    rows = (rng.standard_normal((n * 64, 576)) * np.exp(rng.uniform(-6, 6, (n * 64, 1)))).astype(np.float32)
    rows[5] = 0.0
    codes, scale = quantize_rows(rows)
    paged.write_fp8_rows(cache, np.arange(n * 64), codes, scale, 576)
    return cache


def test_page_stride_closed_form():
    s = op.ds_mla_page_stride()
    assert s == 46080 and s % 9216 == 0 and s >= 64 * 656 and s - 9216 < 64 * 656


def test_export_row_known_answer():
    """Row 3 of a page: codes c, scale 2**-3 -> bytes [0, 512) = c[:512],
    [512, 528) = four fp32 2**-3, [528, 656) = bf16 of decode(c[512:]) / 8."""
    cache = np.zeros((1, paged.fp8_page_bytes(576)), np.uint8)
    c = (np.arange(576) % 126).astype(np.uint8)  # finite codes
    cache[0, 3 * 576: 4 * 576] = c
    cache[0, 64 * 576 + 12: 64 * 576 + 16] = np.array([2.0 ** -3], np.float32).view(np.uint8)
    out = np.full((1, op.ds_mla_page_stride()), 7, np.uint8)
    op.export_pages(cache, [0], out)
    row = out[0, 3 * 656: 4 * 656]
    assert np.array_equal(row[:512], c[:512])
    assert np.array_equal(row[512:528].view(np.float32), np.full(4, 0.125, np.float32))
    assert np.array_equal(row[528:].view(np.uint16), bf16_bits(decode_e4m3(c[512:]) * np.float32(0.125)))
    assert np.all(out[0, 64 * 656:] == 7)  # bytes past the 64 rows untouched


def test_export_is_lossless_and_import_inverts_it():
    rng = np.random.default_rng(0)
    cache = _own_pages(rng, 3)
    ds = np.zeros((3, op.ds_mla_page_stride()), np.uint8)
    op.export_pages(cache, [2, 0, 1], ds)
    for i, p in enumerate([2, 0, 1]):
        codes, scale = op.own_page_rows(cache[p])
        own_vals = decode_e4m3(codes).astype(np.float64) * scale[:, None]
        assert np.array_equal(op.dequant_ds_mla_page(ds[i]).astype(np.float64), own_vals)
    # import(export(page)) holds the same values: the same bytes, except rows
    # whose largest code is 224, which come back with half the scale (the
    # quantization of their dequantized amax) and doubled codes
    back = np.zeros_like(cache)
    op.import_pages(ds, [1, 2, 0], back, dst_pages=[0, 1, 2])
    for p in range(3):
        c0, s0 = op.own_page_rows(cache[p])
        c1, s1 = op.own_page_rows(back[p])
        v0 = decode_e4m3(c0).astype(np.float64) * s0[:, None]
        v1 = decode_e4m3(c1).astype(np.float64) * s1[:, None]
        assert np.array_equal(v0, v1)
        same = np.all(c0 == c1, axis=1) & (s0 == s1)
        top = np.abs(decode_e4m3(c0)).max(1)
        assert np.all(same | (top == 224.0)) and np.all(s1[~same] == s0[~same] / 2)


def test_import_requantizes_arbitrary_tile_scales():
    """Tile scales that are not powers of two (as any writer may choose): the
    imported row is within half an e4m3 step of the source values, and its
    scale is the build's UE8M0 scale of the row's amax."""
    rng = np.random.default_rng(1)
    ds = np.zeros((2, op.ds_mla_page_stride()), np.uint8)
    rows = ds[:, : 64 * 656].reshape(2, 64, 656)
    rows[:, :, :512] = rng.integers(0, 126, (2, 64, 512)) | (rng.integers(0, 2, (2, 64, 512)) << 7)
    tiles = (rng.uniform(0.5, 2.0, (2, 64, 4)) * 10.0 ** rng.uniform(-3, 3, (2, 64, 1))).astype(np.float32)
    rows[:, :, 512:528] = tiles.view(np.uint8).reshape(2, 64, 16)
    rope = (rng.standard_normal((2, 64, 64)) * 3).astype(np.float32)
    rows[:, :, 528:] = bf16_bits(rope).view(np.uint8).reshape(2, 64, 128)
    own = np.zeros((2, paged.fp8_page_bytes(576)), np.uint8)
    op.import_pages(ds, [0, 1], own)
    for p in range(2):
        src = op.dequant_ds_mla_page(ds[p]).astype(np.float64)
        codes, scale = op.own_page_rows(own[p])
        got = decode_e4m3(codes).astype(np.float64) * scale[:, None]
        amax = np.abs(src).max(1)
        assert np.all(scale >= amax / 448.0) and np.all(scale < amax / 224.0)
        # e4m3: 3 mantissa bits -> half a step <= 2**-4 of the value (normal range)
        assert np.all(np.abs(got - src) <= np.maximum(np.abs(src) * 2.0 ** -4, scale[:, None] * 2.0 ** -10))
