"""GPU parity: latent append / indexer K insert bytes vs the oracle (bit-exact)."""

import numpy as np
import pytest
import torch

from helpers import bf16_tensor, permuted_block_table, randn_bf16, to_dev
from oracle import paged
from oracle.fp8 import quantize_rows

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim", [128, 512, 576])
@pytest.mark.parametrize("num_tokens", [1, 7, 300])
def test_append_quant_bytes_exact(dev, dim, num_tokens):
    rng = np.random.default_rng(dim * 1000 + num_tokens)
    pages = (num_tokens + 63) // 64 + 3
    stride = paged.fp8_page_bytes(dim) + 64  # larger than one page's bytes
    rows = randn_bf16(rng, (num_tokens, dim), scale=rng.choice([1e-3, 1.0, 300.0]))
    rows[0, :] = 0.0  # all-zero row -> amax floor
    slots = rng.permutation(pages * 64)[:num_tokens].astype(np.int64)
    if num_tokens > 2:
        slots[1] = -1  # padding row: skipped
    cache_ref = np.full((pages, stride), 173, dtype=np.uint8)
    codes, scale = quantize_rows(rows)
    paged.write_fp8_rows(cache_ref, slots, codes, scale, dim)

    cache = torch.full((pages, stride), 173, dtype=torch.uint8, device=dev)
    from ernie_kv import ops

    ops.kv_append_quant(bf16_tensor(rows, dev), to_dev(slots, dev), cache)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    assert np.array_equal(got, cache_ref)


def test_indexer_k_insert_page_layout(dev):
    """Values at page*stride + off*128, scales at page*stride + 64*128 + off*4
    (the values-then-scales page of attention.py:852-860)."""
    rng = np.random.default_rng(5)
    k = randn_bf16(rng, (2, 128))
    kcache = torch.full((1, 64 * 132), 173, dtype=torch.uint8, device=dev)
    from ernie_kv import ops

    ops.indexer_k_insert(bf16_tensor(k, dev), to_dev(np.array([0, 1], np.int64), dev), kcache)
    got = kcache.cpu().numpy()[0]
    codes, scale = quantize_rows(k)
    assert np.array_equal(got[:256].reshape(2, 128), codes)
    assert np.array_equal(got[8192:8200].view(np.float32), scale)
    assert np.all(got[256:8192] == 173) and np.all(got[8200:] == 173)


def test_append_with_block_table_slots(dev):
    rng = np.random.default_rng(11)
    B, P, dim = 3, 4, 576
    bt = permuted_block_table(rng, B, P)
    seq = rng.integers(0, B, 100)
    pos = rng.integers(0, P * 64, 100)
    # unique (seq, pos) pairs so the last-writer question does not arise
    _, keep = np.unique(seq * 100000 + pos, return_index=True)
    seq, pos = seq[keep], pos[keep]
    slots = paged.slots_from_block_table(bt, seq, pos)
    rows = randn_bf16(rng, (len(slots), dim))
    ref = np.zeros((B * P, paged.fp8_page_bytes(dim)), np.uint8)
    c, s = quantize_rows(rows)
    paged.write_fp8_rows(ref, slots, c, s, dim)
    cache = torch.zeros_like(to_dev(ref, dev))
    from ernie_kv import ops

    ops.kv_append_quant(bf16_tensor(rows, dev), to_dev(slots, dev), cache)
    assert np.array_equal(cache.cpu().numpy(), ref)


@pytest.mark.parametrize("dim", [576, 512])
def test_dsa_decode_prologue_matches_separate_calls(dev, dim):
    """ekv_dsa_decode_prologue == K insert + latent append + q quant + windowed
    lengths issued one by one (each checked against the oracle elsewhere)."""
    from ernie_kv import ops

    rng = np.random.default_rng(dim)
    T, H, pages = 21, 64, 40
    slots = rng.choice(pages * 64, T, replace=False).astype(np.int64)
    slots[3] = -1  # skipped row
    slots_t = to_dev(slots, dev)
    positions = to_dev(rng.integers(0, 5000, T).astype(np.int64), dev)
    k = bf16_tensor(randn_bf16(rng, (T, 128)), dev)
    lat = bf16_tensor(randn_bf16(rng, (T, dim)), dev)
    q = bf16_tensor(randn_bf16(rng, (T, H, 128), 2.0), dev)
    w = bf16_tensor(randn_bf16(rng, (T, H)), dev)
    kc = [torch.zeros((pages, 64 * 132), dtype=torch.uint8, device=dev) for _ in range(2)]
    lc = [torch.zeros((pages, 64 * (dim + 4)), dtype=torch.uint8, device=dev) for _ in range(2)]
    lens = [torch.full((T,), -5, dtype=torch.int32, device=dev) for _ in range(2)]
    ops.indexer_k_insert(k, slots_t, kc[0])
    ops.kv_append_quant(lat, slots_t, lc[0])
    ref_q = ops.indexer_q_quant(q, w)
    ops.indexer_windowed_lengths(positions, 128, lens[0])
    got_q = ops.dsa_decode_prologue(k, kc[1], lat, lc[1], slots_t, q, w, positions, 128, lens[1])
    assert torch.equal(kc[0], kc[1]) and torch.equal(lc[0], lc[1]) and torch.equal(lens[0], lens[1])
    for a, b in zip(ref_q, got_q):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dim", [576, 512])
def test_dsa_decode_prologue_with_indexer_prep(dev, dim):
    """With the prep arguments the prologue takes the raw indexer projections:
    it equals ekv_indexer_prep followed by the prologue without them."""
    from ernie_kv import ops
    from oracle import indexer as oi

    rng = np.random.default_rng(dim + 7)
    T, H, pages = 19, 64, 40
    slots = rng.choice(pages * 64, T, replace=False).astype(np.int64)
    slots[5] = -1
    slots_t = to_dev(slots, dev)
    pos_np = rng.integers(0, 9000, T).astype(np.int64)
    pos_np[0] = 0
    positions = to_dev(pos_np, dev)
    k = bf16_tensor((rng.standard_normal((T, 128)) * 3 + 1).astype(np.float32), dev)
    lat = bf16_tensor(randn_bf16(rng, (T, dim)), dev)
    q = bf16_tensor(randn_bf16(rng, (T, H, 128), 2.0), dev)
    w = bf16_tensor(randn_bf16(rng, (T, H)), dev)
    ln_w = to_dev((1 + 0.2 * rng.standard_normal(128)).astype(np.float32), dev)
    ln_b = to_dev((0.1 * rng.standard_normal(128)).astype(np.float32), dev)
    cs = to_dev(oi.rope_cos_sin(np.arange(10000), 64, 8e6), dev)
    kc = [torch.zeros((pages, 64 * 132), dtype=torch.uint8, device=dev) for _ in range(2)]
    lc = [torch.zeros((pages, 64 * (dim + 4)), dtype=torch.uint8, device=dev) for _ in range(2)]
    lens = [torch.full((T,), -5, dtype=torch.int32, device=dev) for _ in range(2)]
    qh, kh = ops.indexer_prep(q, k, ln_w, ln_b, 1e-6, cs, positions)
    ref_q = ops.dsa_decode_prologue(kh, kc[0], lat, lc[0], slots_t, qh, w, positions, 128, lens[0])
    got_q = ops.dsa_decode_prologue(k, kc[1], lat, lc[1], slots_t, q, w, positions, 128, lens[1],
                                    prep=(ln_w, ln_b, 1e-6, cs))
    assert torch.equal(kc[0], kc[1]) and torch.equal(lc[0], lc[1]) and torch.equal(lens[0], lens[1])
    for a, b in zip(ref_q, got_q):
        assert torch.equal(a, b)
