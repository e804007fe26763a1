"""Committed golden vectors (tests/golden/ekv_golden.npz): the oracle must
reproduce them (CPU), and so must the HIP kernels (GPU)."""

from pathlib import Path

import numpy as np
import pytest

from oracle import decode as od
from oracle import hca as oh
from oracle import indexer as oi
from oracle.fp8 import bf16_from_bits, quantize_rows
from oracle.merge import merge_swa_topk

G = np.load(Path(__file__).resolve().parent / "golden" / "ekv_golden.npz")


def test_oracle_reproduces_golden():
    rows = bf16_from_bits(G["quant_rows_bits"])
    c, s = quantize_rows(rows)
    assert np.array_equal(c, G["quant_codes"]) and np.array_equal(s, G["quant_scale"])
    q, w, k = (bf16_from_bits(G[n]) for n in ("idx_q_bits", "idx_w_bits", "idx_k_bits"))
    qc, wf = oi.quantize_q(q, w)
    kc, ks = quantize_rows(k)
    assert np.array_equal(qc, G["idx_q_codes"]) and np.array_equal(wf, G["idx_w_folded"])
    sc = oi.exact_scores(qc[0], wf[0], kc, ks)
    assert np.array_equal(sc.view(np.uint32), G["idx_scores"].view(np.uint32))
    assert np.array_equal(oi.topk_ascending(sc, 64), G["idx_top64"])
    assert np.array_equal(merge_swa_topk(G["merge_topk"], G["merge_positions"], 2176, 128), G["merge_out"])
    kvs = bf16_from_bits(G["comp_kv_score_bits"])
    D = 512
    y = oh.compress_span(kvs[:, :D], kvs[:, D:], G["comp_ape"], G["comp_norm_w"], 1e-6, G["comp_cos_sin"][1])
    cc, cs = quantize_rows(y[None])
    assert np.array_equal(cc[0], G["comp_codes"]) and np.array_equal(cs, G["comp_scale"])
    o, l = od.sparse_mla_decode(bf16_from_bits(G["dec_q_bits"]),
                                lambda sl: od.gather_rows_fp8(G["dec_page"], sl, 576), G["dec_indices"],
                                256 ** -0.5, 512, G["dec_sinks"])
    np.testing.assert_allclose(o, G["dec_out"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(l, G["dec_lse"], rtol=1e-6)


@pytest.mark.gpu
def test_kernels_reproduce_golden(dev):
    import torch

    from ernie_kv import ops
    from helpers import bf16_values

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    bf = lambda bits: t(bits.view(np.int16)).view(torch.bfloat16)  # noqa: E731
    # quant
    cache = torch.zeros((1, 64 * 580), dtype=torch.uint8, device=dev)
    ops.kv_append_quant(bf(G["quant_rows_bits"]), t(np.arange(8, dtype=np.int64)), cache)
    got = cache.cpu().numpy()[0]
    assert np.array_equal(got[: 8 * 576].reshape(8, 576), G["quant_codes"])
    assert np.array_equal(got[64 * 576 : 64 * 576 + 32].view(np.float32), G["quant_scale"])
    # indexer
    q8, wf, dig = ops.indexer_q_quant(bf(G["idx_q_bits"]), bf(G["idx_w_bits"]))
    assert np.array_equal(q8.cpu().numpy(), G["idx_q_codes"])
    assert np.array_equal(wf.cpu().numpy(), G["idx_w_folded"])
    kc = torch.zeros((5, 64 * 132), dtype=torch.uint8, device=dev)
    ops.indexer_k_insert(bf(G["idx_k_bits"]), t(np.arange(300, dtype=np.int64)), kc)
    scores = torch.zeros((1, 300), dtype=torch.float32, device=dev)
    bt = t(np.arange(5, dtype=np.int32)[None])
    one = t(np.array([0], np.int32))
    lens = t(np.array([300], np.int32))
    ops.indexer_score(dig, wf, kc, bt, one, lens, 300, scores)
    assert np.array_equal(scores.cpu().numpy()[0].view(np.uint32), G["idx_scores"].view(np.uint32))
    top = torch.zeros((1, 64), dtype=torch.int32, device=dev)
    ops.topk_select(scores, lens, 64, top)
    assert np.array_equal(top.cpu().numpy()[0], G["idx_top64"])
    # merge
    out = torch.zeros((8, 2176), dtype=torch.int32, device=dev)
    ops.merge_swa_topk(t(G["merge_topk"]), out, t(G["merge_positions"]), 128)
    assert np.array_equal(out.cpu().numpy(), G["merge_out"])
    # compressor (one sequence whose span 1 completes in this call)
    D = 512
    pool = torch.zeros((2, 64 * (D + 4)), dtype=torch.uint8, device=dev)
    ops.hca_compress(bf(G["comp_kv_score_bits"]), t(np.arange(128, 256, dtype=np.int64)), t(np.array([0, 128], np.int32)),
                     128, None, None, t(G["comp_ape"]), t(G["comp_norm_w"]), 1e-6, t(G["comp_cos_sin"]),
                     t(np.array([[1]], np.int32)), pool)
    got = pool.cpu().numpy()[1]
    assert np.array_equal(got[D : 2 * D], G["comp_codes"])
    assert np.array_equal(got[64 * D + 4 : 64 * D + 8].view(np.float32), G["comp_scale"])
    # decode
    o = torch.zeros((2, 16, 512), dtype=torch.bfloat16, device=dev)
    lse = torch.zeros((2, 16), dtype=torch.float32, device=dev)
    ops.sparse_mla_decode(bf(G["dec_q_bits"]), t(G["dec_page"]), t(G["dec_indices"]), 256 ** -0.5, o, lse,
                          sinks=t(G["dec_sinks"]))
    err = np.abs(bf16_values(o) - G["dec_out"])
    assert np.all(err <= 2e-3 + 2e-2 * np.abs(G["dec_out"]))
    assert np.allclose(lse.cpu().numpy(), G["dec_lse"], atol=2e-3)
