"""Pins of the fp8 / UE8M0 oracle (CPU)."""

import math

import numpy as np
import torch

from oracle.fp8 import (
    decode_table, dequantize_rows, encode_e4m3, quantize_rows, ue8m0_byte, ue8m0_exponent, ue8m0_unpack,
)


def test_decode_table_matches_torch_e4m3fn():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(decode_table(), ref, equal_nan=True)


def test_encode_matches_torch_cast_incl_midpoints():
    rng = np.random.default_rng(0)
    tab = decode_table()
    fin = np.unique(tab[np.isfinite(tab)]).astype(np.float64)
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)
    x = np.concatenate([
        rng.uniform(-448, 448, 200_000), rng.standard_normal(100_000) * 1e-2, fin, mids,
        np.nextafter(mids, np.float32(1e9)), np.nextafter(mids, np.float32(-1e9)), [0.0, -0.0, 448, -448],
    ]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(encode_e4m3(x), ref)


def test_all_codes_round_trip():
    tab = decode_table()
    codes = np.array([c for c in range(256) if np.isfinite(tab[c])], np.uint8)
    assert np.array_equal(encode_e4m3(tab[codes]), codes)


def test_ue8m0_closed_form():
    # amax/448 exactly a power of two -> that exponent; just above -> next
    assert ue8m0_exponent(np.float32(448.0)) == 0
    assert ue8m0_exponent(np.float32(224.0)) == -1
    assert ue8m0_exponent(np.float32(np.nextafter(np.float32(448.0), np.float32(1e9)))) == 1
    assert ue8m0_exponent(np.float32(0.0)) == math.ceil(math.log2(np.float32(1e-10) * np.float32(1 / 448)))
    amax = np.abs(np.random.default_rng(1).standard_normal(10000).astype(np.float32)) * 1e3 + 1e-6
    e = ue8m0_exponent(amax)
    r = (amax * np.float32(1.0 / 448.0)).astype(np.float32).astype(np.float64)
    assert np.all(2.0 ** e >= r) and np.all(2.0 ** (e - 1) < r)


def test_ue8m0_byte_unpack():
    """test_vha_quant.py:16-20: the byte b means 2**(b - 127)."""
    e = np.arange(-30, 31)
    s = np.ldexp(np.float32(1.0), e).astype(np.float32)
    assert np.array_equal(ue8m0_byte(s).astype(np.int64) - 127, e)
    assert np.array_equal(ue8m0_unpack(ue8m0_byte(s)), s)


def test_quantize_rows_bounds_and_amax_position():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 576)) * rng.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    codes, scale = quantize_rows(x)
    y = dequantize_rows(codes, scale)
    amax = np.abs(x).max(1)
    # scaled amax lands in (224, 448] and the per-element error is within half an fp8 step
    assert np.all(amax / scale <= 448.0 * (1 + 1e-6)) and np.all(amax / scale > 224.0 * (1 - 1e-6))
    step = np.where(np.abs(x) / scale[:, None] >= 2.0 ** -6, np.abs(x) / 8, 2.0 ** -9 * scale[:, None])
    assert np.all(np.abs(y - x) <= step * 0.5 + 1e-30)
