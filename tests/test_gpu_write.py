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
