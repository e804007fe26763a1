"""ekv_dsa_decode_prologue_fp4 (one launch) against the calls it stands for:
ekv_indexer_prep of q and k (with the prep), ekv_indexer_k_insert_fp4,
ekv_indexer_q_quant_fp4, ekv_kv_append_quant of the latent rows and
ekv_indexer_windowed_lengths.  Every byte must agree: the MXFP4 K cache, the
fp8 latent cache, q values, scale words, folded weights and the lengths;
with and without the prep, bf16 and fp32 weights, a skipped slot, positions
past the RoPE table and a row count that is not a multiple of 16."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("prep_on", [True, False])
@pytest.mark.parametrize("fp32_w", [False, True])
def test_fp4_prologue_matches_separate_calls(dev, prep_on, fp32_w):
    from ernie_kv import ops

    g = torch.Generator(device=dev).manual_seed(11 + 2 * prep_on + fp32_w)
    T, H, D, pages = 37, 64, 576, 8
    rnd = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)  # noqa: E731
    k, q, latent = rnd(T, 128), rnd(T, H, 128), rnd(T, D)
    w = rnd(T, H)
    if fp32_w:
        w = w.float().contiguous()
    positions = torch.randint(0, 600, (T,), device=dev, generator=g, dtype=torch.int64)
    positions[3] = 5000  # past the RoPE table: left unrotated
    slots = torch.randperm(pages * 64, device=dev, generator=g)[:T].to(torch.int64)
    slots[5] = -1  # skipped
    ln_w = (1.0 + 0.1 * torch.randn(128, device=dev, generator=g)).contiguous()
    ln_b = (0.1 * torch.randn(128, device=dev, generator=g)).contiguous()
    ang = torch.arange(1024, device=dev, dtype=torch.float64)[:, None] * (
        1e4 ** (-torch.arange(32, device=dev, dtype=torch.float64) * 2.0 / 64))[None, :]
    cos_sin = torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).float().contiguous()
    prep = (ln_w, ln_b, 1e-6, cos_sin) if prep_on else None

    kc0 = torch.full((pages, ops.fp4_page_bytes()), 7, dtype=torch.uint8, device=dev)
    lc0 = torch.full((pages, 64 * (D + 4)), 7, dtype=torch.uint8, device=dev)
    kc1, lc1 = kc0.clone(), lc0.clone()
    len0 = torch.full((T,), -3, dtype=torch.int32, device=dev)
    len1 = len0.clone()

    qp, kp = ops.indexer_prep(q, k, *prep, positions) if prep_on else (q, k)
    ops.indexer_k_insert_fp4(kp, slots, kc0)
    v0, s0, w0 = ops.indexer_q_quant_fp4(qp, w)
    ops.kv_append_quant(latent, slots, lc0)
    ops.indexer_windowed_lengths(positions, 128, len0)

    v1, s1, w1 = ops.dsa_decode_prologue_fp4(k, kc1, latent, lc1, slots, q, w, positions, 128, len1, prep=prep)
    torch.cuda.synchronize()
    assert torch.equal(kc0, kc1), "MXFP4 K cache"
    assert torch.equal(lc0, lc1), "latent cache"
    assert torch.equal(v0, v1) and torch.equal(s0, s1), "q values / scale words"
    assert torch.equal(w0.view(torch.int32), w1.view(torch.int32)), "folded weights"
    assert torch.equal(len0, len1), "lengths"
