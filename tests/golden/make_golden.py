"""Writes tests/golden/ekv_golden.npz: seeded inputs and the oracle's outputs.

The reference cannot run here (vLLM 0.32.0 and CUDA are absent), so these
vectors come from the oracle; they pin the oracle against drift and the HIP
kernels against the same bytes.  The merge case transcribes the reference's
own known-answer positions (test_dsa_backend.py:18-37).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import decode as od  # noqa: E402
from oracle import hca as oh  # noqa: E402
from oracle import indexer as oi  # noqa: E402
from oracle import paged  # noqa: E402
from oracle.fp8 import bf16_bits, bf16_round, quantize_rows  # noqa: E402
from oracle.merge import merge_swa_topk  # noqa: E402

OUT = Path(__file__).resolve().parent / "ekv_golden.npz"


def make() -> dict:
    rng = np.random.default_rng(20261201)
    g = {}
    # fp8 per-token quant of latent rows (varied magnitudes, a zero row)
    rows = bf16_round((rng.standard_normal((8, 576)) * np.exp2(rng.integers(-12, 12, (8, 1)))).astype(np.float32))
    rows[3] = 0.0
    g["quant_rows_bits"] = bf16_bits(rows)
    g["quant_codes"], g["quant_scale"] = quantize_rows(rows)
    # indexer: q quant, K quant, exact scores and top-64 with ties
    q = bf16_round(rng.standard_normal((1, 64, 128)).astype(np.float32))
    w = bf16_round(rng.standard_normal((1, 64)).astype(np.float32))
    k = bf16_round(rng.standard_normal((300, 128)).astype(np.float32))
    k[::7] = k[0]  # identical rows -> exact score ties
    qc, wf = oi.quantize_q(q, w)
    kc, ks = quantize_rows(k)
    sc = oi.exact_scores(qc[0], wf[0], kc, ks)
    g.update(idx_q_bits=bf16_bits(q), idx_w_bits=bf16_bits(w), idx_k_bits=bf16_bits(k), idx_q_codes=qc,
             idx_w_folded=wf, idx_k_codes=kc, idx_k_scale=ks, idx_scores=sc, idx_top64=oi.topk_ascending(sc, 64))
    # merge_swa_topk on the reference's positions
    pos = np.array([0, 5, 127, 128, 200, 2175, 2176, 5000], np.int64)
    top = rng.integers(0, 1 << 20, (8, 2048)).astype(np.int32)
    g.update(merge_positions=pos, merge_topk=top, merge_out=merge_swa_topk(top, pos, 2176, 128))
    # compressor: one 128-token span at D = 512
    D = 512
    kvs = bf16_round(rng.standard_normal((128, 2 * D)).astype(np.float32))
    ape = (rng.standard_normal((128, D)) * 0.5).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    cs = oi.rope_cos_sin(np.array([0, 128]), 64, 1.6e5)
    y = oh.compress_span(kvs[:, :D], kvs[:, D:], ape, nw, 1e-6, cs[1])
    cc, cscale = quantize_rows(y[None])
    g.update(comp_kv_score_bits=bf16_bits(kvs), comp_ape=ape, comp_norm_w=nw, comp_cos_sin=cs,
             comp_codes=cc[0], comp_scale=cscale)
    # sparse decode with sink over an fp8 page
    lat = bf16_round(rng.standard_normal((64, 576)).astype(np.float32))
    page = np.zeros((1, paged.fp8_page_bytes(576)), np.uint8)
    c, s = quantize_rows(lat)
    paged.write_fp8_rows(page, np.arange(64), c, s, 576)
    qd = bf16_round(rng.standard_normal((2, 16, 576)).astype(np.float32))
    ind = rng.integers(0, 64, (2, 40)).astype(np.int32)
    ind[1, 30:] = -1
    sinks = rng.standard_normal(16).astype(np.float32)
    o, l = od.sparse_mla_decode(qd, lambda sl: od.gather_rows_fp8(page, sl, 576), ind, 256 ** -0.5, 512, sinks)
    g.update(dec_page=page, dec_q_bits=bf16_bits(qd), dec_indices=ind, dec_sinks=sinks,
             dec_out=o.astype(np.float32), dec_lse=l.astype(np.float32))
    return g


if __name__ == "__main__":
    g = make()
    np.savez_compressed(OUT, **g)
    print(OUT, OUT.stat().st_size, "bytes")
