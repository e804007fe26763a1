#!/usr/bin/env python3
"""Benchmark of the MI355X ERNIE 5.5 attention KV-cache path.

Default workload (the headline): one decode step of a DSA layer at batch 32 x
131,072-token context -- append the new token's latent (fp8) and indexer key,
quantize the indexer queries, score every non-window token exactly, select the
top-2048 (lowest index on ties), append the 128-token window, gather the 2176
rows and run 64-head sparse MLA decode with a sink.  Inputs are synthetic
(seeded) and resident in HBM before the timed region.  The step is issued
eagerly on one stream.

Prints ONE JSON line.  ``value`` = algorithmic HBM bytes of the DSA step /
step time (GB/s), the metric's unit.  Algorithmic bytes per step: indexer K
rows 132 B x sum of windowed lengths, gathered latent rows 580 B x 2176 per
row, plus q / out tensors.  ``tok_per_s`` = decode tokens per second of the
model's whole attention KV path at this shape: 6 DSA layer steps + 37 HCA
layer steps (the HCA decode measured at the same 32 x 131,072 contexts);
``tok_per_s_dsa_layer`` is one DSA layer alone.

The line also carries the other workloads, each measured on its own:
``hca_write`` (chunked-prefill cache write, 16 x 8192 tokens), ``hca_decode``
(HCA decode step, 64 sequences at 8K-128K contexts) and ``mtp`` (DSA and HCA
layer decode steps at 8 x 256K + 1 x 1M contexts with 3 query rows per
sequence, drafts accepted with p = 0.7 and rejected ones re-appended at the
next step, and the model step composed from them).  ``--only`` runs one of
them alone.  ``roofline.traffic`` (and each leg's ``traffic``) is the HBM
traffic per launch of the leg's dominant kernel from the committed rocprofv3
counter summary profiles/hbm_traffic.json, or null when that file holds no
reading for the workload.  ``cpu_baseline`` (and each leg's) is the numpy
oracle on a process pool over the host's cores, timed before the GPU is
touched.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "vllm-ernie_amd"))

METRIC = "KV gather+decode HBM GB/s (% of 8 TB/s); decode tok/s/GPU at 128K ctx"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
MODEL_LAYERS = {"dsa": 6, "hca": 37}  # ERNIE 5.5: 37 HCA : 6 DSA attention layers
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.json"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--ctx", type=int, default=131072)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-hca", action="store_true",
                   help="skip the HCA measurements (chunked-prefill write, decode step)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-mtp", action="store_true", help="skip the multi-token-prediction (1M-context) measurement")
    p.add_argument("--no-fp4", action="store_true", help="skip the MXFP4 indexer measurement")
    p.add_argument("--no-prefill", action="store_true", help="skip the DSA prefill-chunk measurement")
    p.add_argument("--no-pages", action="store_true", help="skip the page-format transcoder measurement")
    p.add_argument("--only", choices=["hca_small", "hca_write", "hca_decode", "hca_layer", "mtp", "dsa",
                                      "dsa_random_row", "model", "indexer_fp4", "dsa_prefill", "pages"],
                   default=None,
                   help="run only this measurement and print its JSON object (for profiling one workload)")
    p.add_argument("--copy-mb", type=int, default=0,
                   help="also run one plain device copy of this many MiB (a known-size kernel that calibrates "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    return p.parse_args()


def csrc_sha16() -> str:
    """Hash of the library's kernel sources (names and bytes, sorted): the
    key a committed counter reading must carry to describe this build."""
    import hashlib

    h = hashlib.sha256()
    for p in sorted((ROOT / "vllm-ernie_amd" / "csrc").iterdir()):
        if p.is_file():
            h.update(p.name.encode() + b"\0" + p.read_bytes())
    return h.hexdigest()[:16]


def _counter_record(workload: str, kernel: str):
    """The committed counter record of `kernel` on `workload`, or None when
    the file holds none or was measured on other kernel sources (its
    csrc_sha16 differs from this tree's)."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    if data.get("csrc_sha16") != csrc_sha16():
        return None
    return data.get("workloads", {}).get(workload, {}).get(kernel)


# The headline step's dominant kernel: the one-launch top-k with the step's
# prologue folded in (profile kernel names drop trailing false flags).
HEADLINE_KERNEL = "filter_verify_kernel<12, false, true>"


def traffic_of(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    counter summary (rocprofv3 FETCH_SIZE / WRITE_SIZE), or None."""
    rec = _counter_record(workload, kernel)
    return None if rec is None else rec.get("bytes")


def mfma_report(workload: str, kernel: str, ms):
    """MFMA utilisation of `kernel` from the committed counters: the busy
    fraction of its matrix cores and, with the kernel's measured time `ms`,
    the rate of the ops it issued against the dense peak of their type."""
    m = mfma_of(workload, kernel)
    if m is None:
        return None
    out = {"busy_frac": m.get("busy_frac"), "ops_per_launch": m.get("ops"),
           "source": f"{TRAFFIC_FILE.relative_to(ROOT)} (rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE, "
                     "SQ_INSTS_VALU_MFMA_MOPS_*)"}
    peaks = {"F8": FP8_PEAK_TFLOPS, "I8": 5000.0, "BF16": BF16_PEAK_TFLOPS}
    if ms:
        out["rates"] = {k: {"tops": round(v / (ms * 1e-3) / 1e12, 1),
                            "frac": round(v / (ms * 1e-3) / 1e12 / peaks[k], 4)}
                        for k, v in (m.get("ops") or {}).items() if k in peaks and v}
    return out


def mfma_of(workload: str, kernel: str):
    """The committed MFMA counters of `kernel` on `workload`: the fraction of
    the dispatch's active cycles the SIMDs' matrix cores were busy
    (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs)) and the MFMA ops
    per dispatch by type (SQ_INSTS_VALU_MFMA_MOPS_* x 512), or None."""
    rec = _counter_record(workload, kernel)
    return None if rec is None else rec.get("mfma")


# --------------------------------------------------------------------------- DSA step
SPIKE_SIGMA = 4.0


def build_dsa_decode(torch, ops, ctxs: list, seed: int, rows_per_seq: int = 1, spike_frac: float = 0.05,
                     extra_tokens: int = 0, spikes: str = "sigma4"):
    """Synthetic DSA-layer decode state: sequence s holds ctxs[s] tokens, the
    last rows_per_seq of them new this step (one query row each: the token
    and its draft tokens), in permuted pages (extra_tokens more positions
    are mapped for steps that grow the sequences).

    Indexer keys (``spike_frac`` of the scored positions are spikes):

    * ``spikes="sigma4"`` (the DSA decode workload at 5% spikes): every key is
      an N(0,1) bf16 row written by the library's K insert (fp8 codes + UE8M0
      scale); each sequence then gets its own spike key row whose exact score
      for the sequence's query row is the smallest reachable at or above
      mean + 4 sigma of the row's ordinary scores, written at a seeded
      ``spike_frac`` of its scored positions.  The spikes score identically,
      so a row's top-2048 is the few ordinary tokens above +4 sigma and then
      the lowest-index spikes: every row's threshold is a tie.
    * ``spikes="random_row"``: uniformly random fp8 codes (scale 2^-8) and
      one random code row copied into ``spike_frac`` of all positions; its
      score is random, so it ties the threshold of only some rows.
    """
    if spike_frac <= 0:
        spikes = "none"
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    S, R = len(ctxs), rows_per_seq
    ctx = max(ctxs) + extra_tokens
    B = S * R  # query rows
    pps = [(c + extra_tokens + 63) // 64 for c in ctxs]
    num_pages = sum(pps)
    perm = torch.randperm(num_pages, device=dev, generator=g).to(torch.int32)
    block_table = torch.full((S, max(pps)), -1, dtype=torch.int32, device=dev)
    o = 0
    for s, n in enumerate(pps):
        block_table[s, :n] = perm[o:o + n]
        o += n

    def random_fp8_pages(dim: int, scale_exp: int):
        pages = torch.randint(0, 256, (num_pages, 64 * dim), device=dev, dtype=torch.uint8, generator=g)
        pages -= ((pages & 0x7F) == 0x7F).to(torch.uint8)  # no NaN codes (0x7f/0xff -> 0x7e/0xfe)
        scales = torch.full((num_pages, 64), 2.0 ** scale_exp, device=dev, dtype=torch.float32)
        return torch.cat([pages, scales.view(torch.uint8)], dim=1).contiguous()

    if spikes == "sigma4":
        kcache = torch.zeros((num_pages, 64 * 132), dtype=torch.uint8, device=dev)
        rows = num_pages * 64
        for r0 in range(0, rows, 1 << 20):
            n = min(1 << 20, rows - r0)
            k = torch.randn(n, 128, device=dev, generator=g).to(torch.bfloat16)
            ops.indexer_k_insert(k, torch.arange(r0, r0 + n, device=dev, dtype=torch.int64), kcache)
        del k
    else:
        kcache = random_fp8_pages(128, -8)
    if spikes == "random_row":
        # a fraction of tokens hold one identical "spike" key row: exact score ties
        spike = kcache[0, :128].clone()
        mask = torch.rand(num_pages, 64, device=dev, generator=g) < spike_frac
        vals = kcache[:, : 64 * 128].unflatten(1, (64, 128))
        vals[mask] = spike
    latent = random_fp8_pages(576, -8)
    ctx_t = torch.tensor(ctxs, dtype=torch.int64, device=dev)
    req_ids = torch.arange(S, dtype=torch.int32, device=dev).repeat_interleave(R)
    positions = (ctx_t.repeat_interleave(R) - R + torch.arange(R, device=dev).repeat(S)).contiguous()
    pos = positions
    slots = (block_table[req_ids.long(), (pos // 64)].to(torch.int64) * 64 + pos % 64).contiguous()
    rnd = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)  # noqa: E731
    st = dict(
        B=B, S=S, R=R, ctxs=list(ctxs), ctx=ctx, block_table=block_table, kcache=kcache, latent=latent,
        positions=positions,
        req_ids=req_ids, slots=slots, k_new=rnd(B, 128), latent_new=rnd(B, 576), q_idx=rnd(B, 64, 128),
        w_idx=rnd(B, 64), q=rnd(B, 64, 576), sinks=torch.randn(64, device=dev, generator=g),
        lengths=torch.empty(B, dtype=torch.int32, device=dev),
        topk=torch.empty((B, 2048), dtype=torch.int32, device=dev),
        merged=torch.empty((B, 2176), dtype=torch.int32, device=dev),
        out=torch.empty((B, 64, 512), dtype=torch.bfloat16, device=dev),
        lse=torch.empty((B, 64), dtype=torch.float32, device=dev),
    )
    # indexer prep: k_norm LayerNorm parameters and the rope table (theta
    # 2.5e6, rope_theta of the config) for every position of the context
    st["ln_w"] = (1.0 + 0.1 * torch.randn(128, device=dev, generator=g)).contiguous()
    st["ln_b"] = (0.1 * torch.randn(128, device=dev, generator=g)).contiguous()
    inv = 2.5e6 ** (-torch.arange(32, device=dev, dtype=torch.float64) * 2.0 / 64)
    ang = torch.arange(ctx, device=dev, dtype=torch.float64)[:, None] * inv[None, :]
    st["rope"] = torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).to(torch.float32).contiguous()
    st["dec_ws"] = ops.decode_workspace(B, 64, 2176, dev)
    st["idx_ws"] = ops.indexer_topk_workspace(B, ctx, dev)
    if spikes == "sigma4":
        _place_sigma_spikes(torch, ops, st, g, spike_frac)
    return st


def _place_sigma_spikes(torch, ops, st, g, spike_frac: float, sigma: float = SPIKE_SIGMA) -> None:
    """Per sequence, a spike key row scoring mean + `sigma` standard
    deviations of its query row's ordinary exact scores (the smallest such
    score the row's fp8 quantization reaches), written by the K insert at a
    seeded `spike_frac` of the sequence's scored positions."""
    dev = st["kcache"].device
    S, R = st["S"], st["R"]
    dsa_pre(ops, st)  # q codes and folded weights of the step's query rows
    scores = torch.empty((st["B"], st["ctx"]), dtype=torch.float32, device=dev)
    ops.indexer_score(st["digits"], st["wf"], st["kcache"], st["block_table"], st["req_ids"], st["lengths"],
                      st["ctx"], scores)
    lut = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float64).to(dev)
    lengths = st["lengths"].cpu()
    # candidate spike rows beta * v / rms(v), beta = 2^-8 .. 2^8 in steps of 2^(1/256)
    betas = torch.exp2(torch.arange(-2048, 2048, device=dev, dtype=torch.float64) / 256.0)
    J = betas.numel()
    scratch = torch.zeros((J // 64, 64 * 132), dtype=torch.uint8, device=dev)
    spike_rows, spike_slots, achieved = [], [], []
    for s in range(S):
        t = s * R  # the sequence's first query row
        n = int(lengths[t])
        ordinary = scores[t, :n].double()
        mu, sd = float(ordinary.mean()), float(ordinary.std())
        target = mu + sigma * sd
        qd = lut[st["q8"][t].long()]  # [64, 128]
        w = st["wf"][t].double()
        v = (w.clamp(min=0)[:, None] * qd).sum(0)
        v = v / v.pow(2).mean().sqrt()
        cand = (betas[:, None] * v[None, :]).to(torch.bfloat16)
        ops.indexer_k_insert(cand, torch.arange(J, device=dev, dtype=torch.int64), scratch)
        codes = scratch[:, : 64 * 128].reshape(J, 128)
        scale = scratch[:, 64 * 128:].contiguous().view(torch.float32).reshape(J).double()
        est = ((lut[codes.long()] @ qd.T).clamp(min=0) * w[None, :]).sum(1) * scale
        ok = torch.nonzero(est >= target).flatten()
        if ok.numel() == 0:
            raise RuntimeError(f"no spike row reaches +{sigma} sigma for sequence {s}")
        j = int(ok[0])
        achieved.append((float(est[j]) - mu) / sd)
        mask = torch.rand(n, device=dev, generator=g) < spike_frac
        pos = torch.nonzero(mask).flatten()
        bt = st["block_table"][s]
        spike_slots.append(bt[pos // 64].to(torch.int64) * 64 + pos % 64)
        spike_rows.append(cand[j:j + 1].expand(pos.numel(), 128))
    ops.indexer_k_insert(torch.cat(spike_rows).contiguous(), torch.cat(spike_slots).contiguous(), st["kcache"])
    torch.cuda.synchronize()
    st["spikes"] = {"sigma": [round(a, 3) for a in achieved],
                    "per_row": [int(x.numel()) for x in spike_slots]}


def dsa_step(ops, st, ev=None):
    """One DSA decode step, eager; ``ev`` = (start, end, start, end) events
    around the indexer call and around the sparse MLA decode."""
    if ev is not None:
        ev[0].record()
    dsa_indexer(ops, st)
    if ev is not None:
        ev[1].record()
    dsa_post(ops, st, ev)


def dsa_indexer(ops, st):
    """The prologue (k_norm, rope and Hadamard of q and k from the raw
    indexer projections, the new token's K and latent appends, the q
    quantization, the windowed lengths) and the indexer (filter, exact
    scoring of the candidates, exact top-2048 and its merge with the window
    as cache slots) in one call: one launch when the top-k is one launch and
    every sequence's new rows lie in its window, else the two calls
    (``dsa_pre`` then ``dsa_filter``)."""
    st["q8"], st["wf"], st["digits"] = ops.dsa_decode_prologue_topk_merged(
        st["k_new"], st["kcache"], st["latent_new"], st["latent"], st["slots"], st["q_idx"], st["w_idx"],
        st["positions"], 128, st["lengths"], st["block_table"], st["req_ids"], st["ctx"], st["topk"], st["idx_ws"],
        st["merged"], merged_slots=True, prep=(st["ln_w"], st["ln_b"], 1e-6, st["rope"]), max_new_rows=st["R"])


def dsa_pre(ops, st):
    """From the raw indexer projections: k_norm, rope and Hadamard of q and k,
    cache appends of the new token, the indexer's q quantization and the
    windowed lengths, in one launch."""
    st["q8"], st["wf"], st["digits"] = ops.dsa_decode_prologue(
        st["k_new"], st["kcache"], st["latent_new"], st["latent"], st["slots"], st["q_idx"], st["w_idx"],
        st["positions"], 128, st["lengths"], prep=(st["ln_w"], st["ln_b"], 1e-6, st["rope"]))


def dsa_filter(ops, st):
    """The indexer: filter, exact scoring of the candidates, exact top-2048
    and its merge with the window as cache slots (one launch when the
    filter fits one)."""
    common = (st["kcache"], st["block_table"], st["req_ids"], st["lengths"], st["ctx"])
    ops.indexer_topk_merged(st["q8"], st["digits"], st["wf"], *common, st["topk"], st["idx_ws"],
                            merged=st["merged"], positions=st["positions"], window=128, merged_slots=True)


def dsa_post(ops, st, ev=None):
    """The sparse MLA decode over the merged rows, which hold cache slots (the
    indexer and the latent cache share the block table)."""
    if ev is not None:
        ev[2].record()
    ops.sparse_mla_decode(st["q"], st["latent"], st["merged"], 256 ** -0.5, st["out"], st["lse"], sinks=st["sinks"],
                          workspace=st["dec_ws"])
    if ev is not None:
        ev[3].record()


def dsa_bytes(B: int, ctx: int) -> dict:
    n = max(ctx - 128, 0)
    k_read = B * n * 132
    gather = B * (min(n, 2048) + min(ctx, 128)) * 580
    qo = B * 64 * 576 * 2 + B * 64 * 512 * 2 + B * 64 * 128 * 2 + B * 64 * 2 + B * 64 * 4
    return {"indexer_k": k_read, "gather": gather, "q_out": qo, "total": k_read + gather + qo}


# --------------------------------------------------------------------------- DSA prefill chunk
def measure_dsa_prefill(torch, ops, seed: int, chunk: int = 4096, ctx: int = 32768, reps: int = 5) -> dict:
    """A DSA layer's chunked-prefill step: `chunk` new tokens of one request
    ending at `ctx`, each a query row -- prologue (indexer prep, K insert,
    latent append, q quant, lengths), indexer top-k of every row (the
    many-row filter / bound / verify kernels and the select, with merged rows), and
    the sparse MLA over the rows' 2176 entries.  The indexer's work is
    quadratic in the chunk: row t scores pos_t + 1 - 128 keys."""
    st = build_dsa_decode(torch, ops, [ctx], seed, rows_per_seq=chunk, spike_frac=0.0)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for _ in range(2):
        dsa_step(ops, st)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    filt = dec = 0.0
    t0.record()
    for _ in range(reps):
        dsa_step(ops, st, ev)
        torch.cuda.synchronize()
        filt += ev[0].elapsed_time(ev[1])
        dec += ev[2].elapsed_time(ev[3])
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    n = [max(p + 1 - 128, 0) for p in range(ctx - chunk, ctx)]
    keys = sum(n)
    flops = keys * 64 * 128 * 2
    filt_ms = filt / reps
    return {
        "workload": f"dsa_prefill_chunk{chunk}_ctx{ctx}",
        "ms": round(ms, 3), "tok_per_s": round(chunk / (ms * 1e-3), 1),
        "indexer_topk_ms": round(filt_ms, 3), "decode_ms": round(dec / reps, 3),
        "indexer_keys_scored": keys, "indexer_key_bytes": keys * 132,
        "indexer_fp8_tflops": round(flops / (filt_ms * 1e-3) / 1e12, 1),
        "indexer_mfma_frac": round(flops / (filt_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
        "what": "one request's prefill chunk as query rows through the DSA step (prologue, indexer top-k with "
                "merged rows, sparse MLA); indexer_topk_ms = the prologue and indexer top-k call (a chunk's "
                "later rows score the keys it appends, so the prologue launch, then the filter, bound, verify and "
                "select launches, merged rows as cache slots) timed by events around it; indexer_mfma_frac = the "
                "fp8 filter flops over that time",
    }


# --------------------------------------------------------------------------- upstream page format
def measure_pages(torch, ops, seed: int, num_pages: int = 4096, reps: int = 20) -> dict:
    """Export of `num_pages` latent pages (576-wide, 64 rows) to fp8_ds_mla
    pages and import back: bytes read + written per call over its time."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed + 5)
    own = torch.randint(0, 126, (num_pages, 64 * 580), device=dev, dtype=torch.uint8, generator=g)
    own[:, 64 * 576:] = torch.full((num_pages, 64), 2.0 ** -6, device=dev).view(torch.uint8)
    ds = torch.zeros((num_pages, ops.ds_mla_page_stride()), dtype=torch.uint8, device=dev)
    ids = torch.arange(num_pages, dtype=torch.int32, device=dev)
    res = {}
    for name, fn in (("export", lambda: ops.export_fp8_ds_mla_pages(own, ids, ds)),
                     ("import", lambda: ops.import_fp8_ds_mla_pages(ds, ids, own))):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        nbytes = num_pages * 64 * (580 + 656)
        res[name] = {"ms": round(ms, 4), "bytes": nbytes, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    res["workload"] = f"fp8_ds_mla_pages_{num_pages}"
    res["what"] = "this library's 580-byte latent rows <-> fp8_ds_mla 656-byte rows, 64 rows per page"
    return res


# --------------------------------------------------------------------------- MXFP4 indexer (use_fp4_kv)
def measure_indexer_fp4(torch, ops, seed: int, B: int = 32, ctx: int = 131072, reps: int = 20,
                        spike_frac: float = 0.05) -> dict:
    """The indexer top-k with 68-byte MXFP4 key rows at the headline shape:
    filter (scaled fp4 MFMA over every key row) + exact select with the
    merged rows, from q already quantized; key bytes random e2m1 with scale
    bytes 2^-8..2^-1 and 5% identical spike rows (exact ties)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed + 4)
    pps = (ctx + 63) // 64
    num_pages = B * pps
    block_table = torch.randperm(num_pages, device=dev, generator=g).to(torch.int32).view(B, pps)
    vals = torch.randint(0, 256, (num_pages, 64 * 64), device=dev, dtype=torch.uint8, generator=g)
    scl = torch.randint(119, 127, (num_pages, 64 * 4), device=dev, dtype=torch.uint8, generator=g)
    if spike_frac > 0:
        mask = torch.rand(num_pages, 64, device=dev, generator=g) < spike_frac
        v3 = vals.view(num_pages, 64, 64)
        v3[mask] = v3[0, 0].clone()
        s3 = scl.view(num_pages, 64, 4)
        s3[mask] = s3[0, 0].clone()
    kcache = torch.cat([vals, scl], dim=1).contiguous()
    del vals, scl
    q = torch.randn(B, 64, 128, device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn(B, 64, device=dev, generator=g).to(torch.bfloat16)
    qv, qs, wf = ops.indexer_q_quant_fp4(q, w)
    req = torch.arange(B, dtype=torch.int32, device=dev)
    positions = torch.full((B,), ctx - 1, dtype=torch.int64, device=dev)
    lengths = torch.full((B,), max(ctx - 128, 0), dtype=torch.int32, device=dev)
    ws = ops.indexer_topk_workspace(B, ctx, dev)
    topk = torch.empty((B, 2048), dtype=torch.int32, device=dev)
    merged = torch.empty((B, 2176), dtype=torch.int32, device=dev)
    common = (kcache, block_table, req, lengths, ctx)

    def step():
        ops.indexer_topk_merged_fp4(qv, qs, wf, *common, topk, ws, merged=merged, positions=positions, window=128)

    ms = time_ms(torch, step, reps)
    n = max(ctx - 128, 0)
    k_bytes = B * n * 68
    timeouts = int(ws[:16].view(torch.int32).sum())

    # the indexer half of an MXFP4 DSA decode step from the raw projections:
    # the one-launch prologue (prep, MXFP4 K insert and q quant, latent
    # append, lengths), then the top-k; and the same with the prologue as
    # the separate calls it replaces
    k_new = torch.randn(B, 128, device=dev, generator=g).to(torch.bfloat16)
    lat_new = torch.randn(B, 576, device=dev, generator=g).to(torch.bfloat16)
    latent = torch.empty((num_pages, 64 * 580), dtype=torch.uint8, device=dev)  # only the appended rows are written
    slots = (block_table[:, (ctx - 1) // 64].to(torch.int64) * 64 + (ctx - 1) % 64).contiguous()
    ang = torch.arange(ctx, device=dev, dtype=torch.float64)[:, None] * (
        1e4 ** (-torch.arange(32, device=dev, dtype=torch.float64) * 2.0 / 64))[None, :]
    prep = ((1.0 + 0.1 * torch.randn(128, device=dev, generator=g)).contiguous(),
            (0.1 * torch.randn(128, device=dev, generator=g)).contiguous(), 1e-6,
            torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).float().contiguous())
    lens = torch.empty(B, dtype=torch.int32, device=dev)

    def indexer_step():
        a, b, c = ops.dsa_decode_prologue_fp4(k_new, kcache, lat_new, latent, slots, q, w, positions, 128, lens,
                                              prep=prep)
        ops.indexer_topk_merged_fp4(a, b, c, kcache, block_table, req, lens, ctx, topk, ws, merged=merged,
                                    positions=positions, window=128)

    def indexer_step_separate():
        qp, kp = ops.indexer_prep(q, k_new, *prep, positions)
        ops.indexer_k_insert_fp4(kp, slots, kcache)
        a, b, c = ops.indexer_q_quant_fp4(qp, w)
        ops.kv_append_quant(lat_new, slots, latent)
        ops.indexer_windowed_lengths(positions, 128, lens)
        ops.indexer_topk_merged_fp4(a, b, c, kcache, block_table, req, lens, ctx, topk, ws, merged=merged,
                                    positions=positions, window=128)

    step_ms = time_ms(torch, indexer_step, reps)
    step_sep_ms = time_ms(torch, indexer_step_separate, reps)
    del kcache, latent
    return {
        "workload": f"indexer_fp4_b{B}_ctx{ctx}",
        "ms": round(ms, 4), "key_bytes": k_bytes, "GB/s_keys": round(k_bytes / (ms * 1e-3) / 1e9, 1),
        "frac_keys": round(k_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "wait_timeouts": timeouts,
        "indexer_step_ms": round(step_ms, 4), "indexer_step_separate_ms": round(step_sep_ms, 4),
        "what": "ekv_indexer_topk_merged_fp4 (filter, exact scoring of the candidates, exact top-2048 and the "
                "merged rows in one launch) over 68-byte MXFP4 key rows, q pre-quantized; frac_keys = key bytes "
                "/ call time / 8 TB/s; indexer_step_ms = the indexer half of an MXFP4 DSA decode step from the raw "
                "projections (ekv_dsa_decode_prologue_fp4, one launch, then the top-k), "
                "indexer_step_separate_ms = the same with the prologue as its five separate calls",
    }


# --------------------------------------------------------------------------- HCA write (config 4)
def build_hca_write(torch, ops, seed: int, B: int = 16, chunk: int = 8192, max_off: int = 65536, D: int = 576):
    """Chunked-prefill cache write: B sequences each appending a `chunk`-token
    chunk at a random offset in [0, max_off), scattered by a random slot
    mapping into a 1M-slot fp8 pool; every completed 128-token span is
    compressed and the 128-token window ring is updated.  Synthetic inputs."""
    dev = torch.device("cuda:0")
    gc = torch.Generator().manual_seed(seed + 1)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    pages = 16384  # 1,048,576 slots
    spans = (max_off + chunk) // 128 + 1
    comp_pages, ring_pages_per = (spans + 63) // 64, 2
    perm = torch.randperm(pages, generator=gc)
    comp_bt = perm[: B * comp_pages].view(B, comp_pages).to(torch.int32).to(dev)
    ring_pages = perm[B * comp_pages: B * (comp_pages + ring_pages_per)].view(B, ring_pages_per).to(torch.int32)
    rest = perm[B * (comp_pages + ring_pages_per):]
    T = B * chunk
    free_slots = (rest[:, None] * 64 + torch.arange(64)[None, :]).flatten()
    slots = free_slots[torch.randperm(free_slots.numel(), generator=gc)[:T]].to(torch.int64).to(dev)
    offs = torch.randint(0, max_off, (B,), generator=gc)
    positions = (offs[:, None] + torch.arange(chunk)[None, :]).flatten().to(torch.int64).to(dev)
    token_seq = torch.arange(B, dtype=torch.int32).repeat_interleave(chunk).to(dev)
    qsl = (torch.arange(B + 1, dtype=torch.int32) * chunk).to(dev)
    ang = (torch.arange(spans, dtype=torch.float64)[:, None] * 128.0) * (
        1.6e5 ** (-torch.arange(32, dtype=torch.float64) * 2.0 / 64))[None, :]
    cos_sin = torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).to(torch.float32).to(dev)
    st = dict(
        B=B, T=T, chunk=chunk, D=D, spans_done=int(((offs + chunk) // 128 - offs // 128).sum()),
        pool=torch.zeros((pages, 64 * (D + 4)), dtype=torch.uint8, device=dev),
        latent=torch.randn(T, D, device=dev, generator=gd).to(torch.bfloat16),
        kv_score=torch.randn(T, 2 * D, device=dev, generator=gd).to(torch.bfloat16),
        state=torch.randn(B + 2, 256, 2 * D, device=dev, generator=gd).to(torch.bfloat16),
        state_slot=torch.randperm(B + 2, generator=gc)[:B].to(torch.int32).to(dev),
        ape=(torch.randn(128, D, device=dev, generator=gd) * 0.5).contiguous(),
        norm_w=(1.0 + 0.1 * torch.randn(D, device=dev, generator=gd)).contiguous(),
        cos_sin=cos_sin, comp_bt=comp_bt, ring_pages=ring_pages.to(dev), slots=slots, positions=positions,
        token_seq=token_seq, qsl=qsl,
        # a workspace slot per (sequence, span slot): each span compressed by D / 64 one-wave workgroups
        ws=ops.hca_write_workspace(B, D, dev, max_query_len=chunk),
    )
    return st


def hca_write_step(ops, st):
    """One HCA write call: compress the completed spans, then append (fp8
    rows, window ring, state ring)."""
    ops.hca_write(st["latent"], st["kv_score"], st["slots"], st["positions"], st["token_seq"], st["qsl"], st["chunk"],
                  st["state"], st["state_slot"], st["ape"], st["norm_w"], 1e-6, st["cos_sin"], st["comp_bt"],
                  st["ring_pages"], 128, st["pool"], workspace=st["ws"])


def hca_write_bytes(T: int, D: int, B: int, spans_done: int) -> dict:
    # the survey's algorithmic bytes: latent rows read (bf16) and written
    # (fp8 + scale), compressed entries and window-ring rows written
    surveyed = T * D * 2 + T * (D + 4) + spans_done * (D + 4) + B * 128 * (D + 4)
    # plus the compressor's kv || score rows (bf16, 2D per token) read once and
    # the state-ring rows (last 256 positions per sequence) copied
    full = surveyed + T * 2 * D * 2 + 2 * B * 256 * 2 * D * 2
    return {"latent_rows": surveyed, "with_kv_score": full}


def measure_hca_write(torch, ops, seed: int, reps: int = 10) -> dict:
    st = build_hca_write(torch, ops, seed)
    ms = time_ms(torch, lambda: hca_write_step(ops, st), reps, warmup=2)
    by = hca_write_bytes(st["T"], st["D"], st["B"], st["spans_done"])
    workload = f"hca_chunked_prefill_b{st['B']}_chunk{st['chunk']}"
    return {
        "workload": workload,
        "kernels": "hca_compress_slab_kernel<576> (9 one-wave workgroups per span) + hca_append_kernel<576> "
                   "(rows, window ring, state ring)",
        "ms": round(ms, 4),
        "bytes_latent_rows": by["latent_rows"],
        "GB/s_latent_rows": round(by["latent_rows"] / (ms * 1e-3) / 1e9, 1),
        "frac_latent_rows": round(by["latent_rows"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_with_kv_score": by["with_kv_score"],
        "GB/s_with_kv_score": round(by["with_kv_score"] / (ms * 1e-3) / 1e9, 1),
        "frac_with_kv_score": round(by["with_kv_score"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "traffic": {"kernel": "hca_compress_slab_kernel<576>",
                    "bytes": traffic_of(workload, "hca_compress_slab_kernel<576>")},
    }


# --------------------------------------------------------------------------- HCA layer in bf16 (config 1)
def build_hca_small(torch, ops, seed: int, B: int = 4, ctx: int = 4096, D: int = 576, heads: int = 16,
                    hidden: int = 4096):
    """The small HCA layer workload: B sequences of ctx tokens written into a
    bf16 paged cache (block size 64, permuted block table) in one prefill
    call -- every row appended, every 128-token span compressed (compressor
    input = hidden N(0,1) x fused_wkv_wgate N(0, 0.02), ape N(0, 0.02),
    RMSNorm weight 1, RoPE at compress_rope_theta 1.6e5), the 128-row window
    ring written -- then one decode query per sequence (its last token, 16
    heads, q N(0,1)) over its ctx/128 compressed entries and 128 window rows.
    Latents N(0,1).  Synthetic inputs, seeded."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed + 6)
    gc = torch.Generator().manual_seed(seed + 6)
    lat_pp, spans, ring = ctx // 64, ctx // 128, 128
    comp_pp, ring_pp = (spans + 1 + 63) // 64, ring // 64
    pages = B * (lat_pp + comp_pp + ring_pp)
    perm = torch.randperm(pages, generator=gc).to(torch.int32)
    bt = perm[: B * lat_pp].view(B, lat_pp)
    comp_bt = perm[B * lat_pp: B * (lat_pp + comp_pp)].view(B, comp_pp).to(dev)
    ring_pages = perm[B * (lat_pp + comp_pp):].view(B, ring_pp).to(dev)
    T = B * ctx
    positions = torch.arange(ctx, dtype=torch.int64).repeat(B)
    token_seq = torch.arange(B, dtype=torch.int32).repeat_interleave(ctx)
    slots = bt[token_seq.long(), positions // 64].to(torch.int64) * 64 + positions % 64
    h = torch.randn(T, hidden, device=dev, generator=g)
    w = torch.randn(hidden, 2 * D, device=dev, generator=g) * 0.02
    kv_score = (h @ w).to(torch.bfloat16)
    del h, w
    ang = (torch.arange(spans + 1, dtype=torch.float64)[:, None] * 128.0) * (
        1.6e5 ** (-torch.arange(32, dtype=torch.float64) * 2.0 / 64))[None, :]
    width = spans + ring
    st = dict(
        B=B, T=T, ctx=ctx, D=D, heads=heads, ring=ring, width=width, scale=D ** -0.5,
        latent=torch.randn(T, D, device=dev, generator=g).to(torch.bfloat16), kv_score=kv_score,
        slots=slots.to(dev), positions=positions.to(dev), token_seq=token_seq.to(dev),
        qsl=(torch.arange(B + 1, dtype=torch.int32) * ctx).to(dev),
        state=torch.zeros((B, 256, 2 * D), dtype=torch.bfloat16, device=dev),
        state_slot=torch.arange(B, dtype=torch.int32, device=dev),
        ape=(0.02 * torch.randn(128, D, device=dev, generator=g)).contiguous(),
        norm_w=torch.ones(D, device=dev), comp_bt=comp_bt, ring_pages=ring_pages,
        cos_sin=torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).to(torch.float32).to(dev),
        pool=torch.zeros((pages * 64, D), dtype=torch.bfloat16, device=dev),
        q=torch.randn(B, heads, D, device=dev, generator=g).to(torch.bfloat16),
        sinks=torch.randn(heads, device=dev, generator=g),
        q_pos=torch.full((B,), ctx - 1, dtype=torch.int64, device=dev),
        req=torch.arange(B, dtype=torch.int32, device=dev),
        idx=torch.empty((B, width), dtype=torch.int32, device=dev),
        lens=torch.empty(B, dtype=torch.int32, device=dev),
        out=torch.empty((B, heads, 512), dtype=torch.bfloat16, device=dev),
        lse=torch.empty((B, heads), dtype=torch.float32, device=dev),
        ws=ops.hca_write_workspace(B, D, dev, max_query_len=ctx),
    )
    st["dec_ws"] = ops.decode_workspace(B, heads, width, dev)
    return st


def hca_small_step(ops, st):
    """The bf16 HCA write of every token (rows, compressed spans, window
    ring), the decode rows' indices and the 16-head decode."""
    ops.hca_write(st["latent"], st["kv_score"], st["slots"], st["positions"], st["token_seq"], st["qsl"], st["ctx"],
                  st["state"], st["state_slot"], st["ape"], st["norm_w"], 1e-6, st["cos_sin"], st["comp_bt"],
                  st["ring_pages"], st["ring"], st["pool"], workspace=st["ws"])
    ops.hca_decode_indices(st["q_pos"], st["req"], st["comp_bt"], st["ring_pages"], st["ring"], st["idx"], st["lens"])
    ops.sparse_mla_decode(st["q"], st["pool"], st["idx"], st["scale"], st["out"], st["lse"], sinks=st["sinks"],
                          lengths=st["lens"], cache_bf16=True, workspace=st["dec_ws"])


def measure_hca_small(torch, ops, seed: int, reps: int = 20) -> dict:
    st = build_hca_small(torch, ops, seed)
    ms = time_ms(torch, lambda: hca_small_step(ops, st), reps)
    T, D, B = st["T"], st["D"], st["B"]
    spans = B * (st["ctx"] // 128)
    # rows in (bf16) and out (bf16), kv || score in, compressed and ring rows
    # out, the state ring's last 256 rows, then the decode's rows and q / out
    write = T * D * 2 * 2 + T * 2 * D * 2 + spans * D * 2 + B * st["ring"] * D * 2 + B * 256 * 2 * D * 2
    dec = B * st["width"] * D * 2 + B * st["heads"] * (D * 2 + 512 * 2 + 4)
    return {
        "workload": f"hca_layer_bf16_b{B}_ctx{st['ctx']}_h{st['heads']}",
        "ms": round(ms, 4), "bytes": write + dec,
        "GB/s": round((write + dec) / (ms * 1e-3) / 1e9, 1),
        "frac": round((write + dec) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "what": "ekv_hca_write_bf16 of 4 x 4096 tokens (rows, 128 compressed spans, window ring) + index rows + "
                "16-head sparse decode over 32 + 128 bf16 rows per sequence, events around the three calls",
    }


# --------------------------------------------------------------------------- HCA decode (config 2)
def build_hca_decode(torch, ops, seed: int, B: int = 64, ctx_lo: int = 8192, ctx_hi: int = 131072, D: int = 576,
                     ring: int = 128, ctxs: list | None = None, rows_per_seq: int = 1, extra_tokens: int = 0):
    """HCA-layer decode step state: B sequences with seeded contexts in
    [ctx_lo, ctx_hi) (or the given ctxs), their compressed entries and window
    rings as random fp8 rows (fp32 scale 2^-8) in permuted pages, and
    rows_per_seq new tokens each (the token and its drafts, one query row
    each).  Synthetic inputs."""
    dev = torch.device("cuda:0")
    gc = torch.Generator().manual_seed(seed + 2)
    gd = torch.Generator(device=dev).manual_seed(seed + 2)
    if ctxs is not None:
        B = len(ctxs)
        ctx = torch.tensor(ctxs, dtype=torch.int64)
        ctx_hi = int(ctx.max()) + 1
    else:
        ctx = torch.randint(ctx_lo, ctx_hi, (B,), generator=gc).to(torch.int64)
    ctx_hi += extra_tokens
    R = rows_per_seq
    T = B * R
    spans = ctx_hi // 128 + 1
    comp_pages = (spans + 63) // 64
    ring_pp = (ring + 63) // 64
    lat_pp = 1 + (extra_tokens + R + 63) // 64  # pages for the new tokens' own rows
    pages = B * (comp_pages + ring_pp + lat_pp)
    perm = torch.randperm(pages, generator=gc).to(torch.int32)
    comp_bt = perm[: B * comp_pages].view(B, comp_pages).to(dev)
    ring_pages = perm[B * comp_pages: B * (comp_pages + ring_pp)].view(B, ring_pp).to(dev)
    lat_bt = perm[B * (comp_pages + ring_pp):].view(B, lat_pp).to(torch.int64)
    # the new tokens: the last R positions of each context
    positions = ctx.repeat_interleave(R) - R + torch.arange(R).repeat(B)
    base = (ctx - R)  # first new position per sequence; its rows go to the sequence's own pages
    rel = positions - base.repeat_interleave(R)
    slots = (lat_bt[torch.arange(B).repeat_interleave(R), rel // 64] * 64 + rel % 64).to(dev)
    codes = torch.randint(0, 256, (pages, 64 * D), device=dev, dtype=torch.uint8, generator=gd)
    codes -= ((codes & 0x7F) == 0x7F).to(torch.uint8)  # no NaN codes
    scales = torch.full((pages, 64), 2.0 ** -8, device=dev, dtype=torch.float32)
    ang = (torch.arange(spans, dtype=torch.float64)[:, None] * 128.0) * (
        1.6e5 ** (-torch.arange(32, dtype=torch.float64) * 2.0 / 64))[None, :]
    width = (ctx_hi // 128) + ring
    rnd = lambda *s: torch.randn(*s, device=dev, generator=gd).to(torch.bfloat16)  # noqa: E731
    st = dict(
        B=B, T=T, R=R, D=D, ring=ring, ctx=ctx, width=width, base=base, lat_bt=lat_bt,
        pool=torch.cat([codes, scales.view(torch.uint8)], dim=1).contiguous(),
        latent=rnd(T, D), kv_score=rnd(T, 2 * D), state=rnd(B + 2, 256, 2 * D),
        state_slot=torch.randperm(B + 2, generator=gc)[:B].to(torch.int32).to(dev),
        ape=(torch.randn(128, D, device=dev, generator=gd) * 0.5).contiguous(),
        norm_w=(1.0 + 0.1 * torch.randn(D, device=dev, generator=gd)).contiguous(),
        cos_sin=torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).to(torch.float32).to(dev),
        comp_bt=comp_bt, ring_pages=ring_pages, slots=slots, positions=positions.to(dev),
        token_seq=torch.arange(B, dtype=torch.int32, device=dev).repeat_interleave(R),
        qsl=(torch.arange(B + 1, dtype=torch.int32) * R).to(dev),
        req=torch.arange(B, dtype=torch.int32, device=dev).repeat_interleave(R),
        q=rnd(T, 64, D), sinks=torch.randn(64, device=dev, generator=gd),
        idx=torch.empty((T, width), dtype=torch.int32, device=dev),
        lens=torch.empty(T, dtype=torch.int32, device=dev),
        out=torch.empty((T, 64, 512), dtype=torch.bfloat16, device=dev),
        lse=torch.empty((T, 64), dtype=torch.float32, device=dev),
    )
    st["dec_ws"] = ops.decode_workspace(T, 64, width, dev)
    st["write_ws"] = ops.hca_write_workspace(B, D, dev)
    return st


def hca_decode_step(ops, st):
    """One HCA decode step: the new token's write (latent row, window ring,
    state ring; the spans it completes are compressed) and its index rows
    (compressed entries, then the window) in one launch, then the 64-head
    decode."""
    ops.hca_write_step(st["latent"], st["kv_score"], st["slots"], st["positions"], st["token_seq"], st["qsl"],
                       st["R"], st["state"], st["state_slot"], st["ape"], st["norm_w"], 1e-6, st["cos_sin"],
                       st["comp_bt"], st["ring_pages"], st["ring"], st["pool"], 128, st["idx"], st["lens"],
                       workspace=st["write_ws"])
    ops.sparse_mla_decode(st["q"], st["pool"], st["idx"], 256 ** -0.5, st["out"], st["lse"], sinks=st["sinks"],
                          lengths=st["lens"], workspace=st["dec_ws"])


def time_ms(torch, step, reps: int, warmup: int = 3) -> float:
    """Average milliseconds of step() over reps calls (events on the current stream)."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        step()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def graph_ms(torch, step, reps: int) -> float:
    """Average milliseconds of replays of a HIP graph captured from one call of
    step() (warmed up on a side stream first, as capture requires).  The
    step's kernels take fixed workspaces and never synchronize the host, so
    a replay runs exactly the eager step's launches."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    ms = time_ms(torch, g.replay, reps)
    del g
    return ms


def hca_decode_bytes(st) -> dict:
    """Algorithmic bytes of one HCA decode step: each query row's compressed
    entries and window rows (580 B each), q / out / lse, and the new tokens'
    appends (latent in, row and ring row out, kv || score in, state row out)."""
    D, T = st["D"], st["T"]
    seq = st["positions"].cpu() + 1
    rows = int((seq // 128 + seq.clamp(max=128)).sum())
    gather = rows * (D + 4)
    q_out = T * 64 * D * 2 + T * 64 * 512 * 2 + T * 64 * 4
    append = T * (D * 2 + 2 * (D + 4) + 2 * D * 2 * 2)
    return {"rows": rows, "gather": gather, "q_out": q_out, "append": append, "total": gather + q_out + append}


def measure_hca_decode(torch, ops, seed: int, reps: int = 50, ctxs: list | None = None, label: str | None = None) -> dict:
    st = build_hca_decode(torch, ops, seed, ctxs=ctxs)
    ms_eager = time_ms(torch, lambda: hca_decode_step(ops, st), reps)
    ms_graph = graph_ms(torch, lambda: hca_decode_step(ops, st), reps)
    ms = ms_graph  # the serving mode: the step captured once and replayed
    by = hca_decode_bytes(st)
    workload = label or f"hca_decode_b{st['B']}_ctx8192-131072"
    return {
        "workload": workload,
        "kernels": "hca_write_small_kernel<576> (the new tokens' rows, ring, state; spans they complete; the "
                   "index rows) + sparse_decode_kernel<576> + decode_combine_kernel",
        "ms": round(ms, 4),
        "ms_graph": round(ms_graph, 4),
        "ms_eager": round(ms_eager, 4),
        "launch": "ms = a HIP graph replaying one captured step (ms_graph, the serving mode); ms_eager = the "
                  "same step launched eagerly",
        "rows_per_step": by.pop("rows"),
        "bytes": by,
        "GB/s": round(by["total"] / (ms * 1e-3) / 1e9, 1),
        "frac": round(by["total"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "tok_per_s": round(st["T"] / (ms * 1e-3), 1),
        "traffic": {"kernel": "sparse_decode_kernel<576>", "bytes": traffic_of(workload, "sparse_decode_kernel<576>")},
    }


# --------------------------------------------------------------------------- MTP (config 5)
MTP_CTXS = [262144] * 8 + [1048576]
MTP_ROWS = 3  # the token and its 2 draft tokens
MTP_ACCEPT = 0.7
MTP_STEPS = 13  # 3 warmup + 10 timed


def mtp_schedule(ctxs: list, steps: int, seed: int):
    """Per step, the first query position of each sequence: the step's rows
    are that position and the next two (token + 2 drafts).  Draft 1 is
    accepted with p = 0.7, draft 2 (if draft 1 was) with p = 0.7; the next
    step starts after the last accepted row, so the rejected drafts'
    positions are written again (re-appended).  Returns (first positions
    [steps, S], accepted tokens per step)."""
    import numpy as np

    rng = np.random.default_rng(seed + 5)
    first = np.array(ctxs, np.int64) - MTP_ROWS
    firsts, accepted = [], []
    for _ in range(steps):
        firsts.append(first.copy())
        a1 = rng.random(len(ctxs)) < MTP_ACCEPT
        a2 = a1 & (rng.random(len(ctxs)) < MTP_ACCEPT)
        acc = 1 + a1.astype(np.int64) + a2.astype(np.int64)
        accepted.append(int(acc.sum()))
        first = first + acc
    return np.stack(firsts), accepted


def measure_mtp(torch, ops, seed: int, steps: int = MTP_STEPS, warm: int = 3) -> dict:
    """Multi-token-prediction decode at 8 x 262,144 + 1 x 1,048,576 contexts,
    3 query rows per sequence, drafts accepted with p = 0.7 and the rejected
    ones re-appended at the next step: a DSA layer's and an HCA layer's
    steps measured over the same accept/reject schedule, and the model step
    composed from them (6 DSA + 37 HCA layers)."""
    S, R = len(MTP_CTXS), MTP_ROWS
    firsts, accepted = mtp_schedule(MTP_CTXS, steps, seed)
    grow = int(firsts[-1].max() - (max(MTP_CTXS) - R)) + 64
    dev = torch.device("cuda:0")
    offs = torch.arange(R, device=dev).repeat(S)
    pos_steps = [torch.from_numpy(f).to(dev).repeat_interleave(R) + offs for f in firsts]

    st = build_dsa_decode(torch, ops, MTP_CTXS, seed, rows_per_seq=R, spike_frac=0.0, extra_tokens=grow)
    req = st["req_ids"].long()
    dsa_pos = [p.contiguous() for p in pos_steps]
    dsa_slots = [(st["block_table"][req, p // 64].to(torch.int64) * 64 + p % 64).contiguous() for p in pos_steps]

    def dsa_at(i):
        st["positions"], st["slots"] = dsa_pos[i], dsa_slots[i]
        dsa_step(ops, st)

    dsa_ms = sequence_ms(torch, dsa_at, steps, warm)
    pos0 = pos_steps[0].cpu()
    n_row = (pos0 + 1 - 128).clamp(min=0)
    k_once = sum(max(c - 128, 0) for c in MTP_CTXS) * 132  # each sequence's keys read once
    k_rows = int(n_row.sum()) * 132                       # read per query row, as this build does
    gather = int((n_row.clamp(max=2048) + (pos0 + 1).clamp(max=128)).sum()) * 580
    T = S * R
    qo = T * (64 * 576 * 2 + 64 * 512 * 2 + 64 * 128 * 2 + 64 * 2 + 64 * 4)
    del st
    torch.cuda.empty_cache()
    # the window ring holds the 128-row window of every query row (128 + R - 1
    # rows), in whole 64-row pages
    sh = build_hca_decode(torch, ops, seed, ctxs=MTP_CTXS, rows_per_seq=R, ring=64 * ((128 + R - 1 + 63) // 64),
                          extra_tokens=grow)
    base = sh["base"].to(dev).repeat_interleave(R)
    lat_bt = sh["lat_bt"].to(dev)
    sreq = torch.arange(S, device=dev).repeat_interleave(R)
    hca_slots = [(lat_bt[sreq, (p - base) // 64] * 64 + (p - base) % 64).contiguous() for p in pos_steps]

    def hca_at(i):
        sh["positions"], sh["slots"] = dsa_pos[i], hca_slots[i]
        hca_decode_step(ops, sh)

    hca_ms = sequence_ms(torch, hca_at, steps, warm)
    sh["positions"] = dsa_pos[0]
    hb = hca_decode_bytes(sh)
    del sh
    torch.cuda.empty_cache()
    step_ms = MODEL_LAYERS["dsa"] * dsa_ms + MODEL_LAYERS["hca"] * hca_ms
    tok_step = sum(accepted[warm:]) / (steps - warm)  # accepted tokens per step, drawn
    dsa_total = k_once + gather + qo
    return {
        "workload": f"mtp_decode_{S}seq_{R}rows_8x262144_1x1048576",
        "accept": f"drafts accepted with p={MTP_ACCEPT} (draft 2 only after draft 1); rejected drafts re-appended "
                  f"at the next step; {tok_step:.2f} tokens accepted per step over the timed steps",
        "dsa_layer": {
            "ms": round(dsa_ms, 4),
            "bytes": {"indexer_k_once": k_once, "indexer_k_per_row": k_rows, "gather": gather, "q_out": qo,
                      "total": dsa_total},
            "GB/s": round(dsa_total / (dsa_ms * 1e-3) / 1e9, 1),
            "GB/s_per_row_k": round((k_rows + gather + qo) / (dsa_ms * 1e-3) / 1e9, 1),
        },
        "hca_layer": {
            "ms": round(hca_ms, 4), "rows_per_step": hb.pop("rows"), "bytes": hb,
            "GB/s": round(hb["total"] / (hca_ms * 1e-3) / 1e9, 1),
        },
        "model_step_ms": round(step_ms, 3),
        "model_step": "composed: 6 x dsa_layer.ms + 37 x hca_layer.ms (the attention KV path only)",
        "query_rows_per_s": round(T / (step_ms * 1e-3), 1),
        "tok_per_s": round(tok_step / (step_ms * 1e-3), 1),
    }


def sequence_ms(torch, step_at, steps: int, warm: int) -> float:
    """Average milliseconds of step_at(i) for i in [warm, steps) after running
    steps 0 .. warm-1 untimed (events on the current stream)."""
    for i in range(warm):
        step_at(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(warm, steps):
        step_at(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (steps - warm)


# --------------------------------------------------------------------------- CPU baselines
def _cpu_workers() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _cpu_dsa_row(args):
    """Oracle of one DSA query row: exact scores of its n keys, top-2048,
    64-head decode over 2176 gathered rows.  Synthetic inputs of the
    headline's shape (seeded per row)."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    from oracle import decode as od
    from oracle import indexer as oi
    from oracle.fp8 import bf16_round, decode_e4m3

    from oracle.fp8 import quantize_rows

    ctx, seed = args
    rng = np.random.default_rng(seed)
    n = max(ctx - 128, 0)
    # N(0,1) key rows quantized as the K insert does; 5% of them one spike row
    codes, kscale = quantize_rows(bf16_round(rng.standard_normal((n, 128)).astype(np.float32)))
    spike = rng.random(n) < 0.05
    codes[spike], kscale[spike] = codes[0], kscale[0]
    q = bf16_round(rng.standard_normal((64, 128)).astype(np.float32))
    w = bf16_round(rng.standard_normal(64).astype(np.float32))
    lat_codes = rng.integers(0, 256, (2176, 576)).astype(np.uint8)
    lat_codes[(lat_codes & 0x7F) == 0x7F] ^= 1
    rows = decode_e4m3(lat_codes).astype(np.float64) * 2.0 ** -8
    qm = bf16_round(rng.standard_normal((1, 64, 576)).astype(np.float32))
    sinks = rng.standard_normal(64).astype(np.float32)
    t0 = time.perf_counter()
    qc, wf = oi.quantize_q(q[None], w[None])
    sc = oi.exact_scores(qc[0], wf[0], codes, kscale)
    top = oi.topk_ascending(sc, 2048)
    idx = np.concatenate([top, np.arange(n, n + 128)])[None]
    idx = np.where(idx >= 0, idx % 2176, -1)
    od.sparse_mla_decode(qm, lambda s: rows[s], idx, 256 ** -0.5, 512, sinks)
    return time.perf_counter() - t0


def _cpu_hca_write_seq(args):
    """Oracle of one sequence's chunked-prefill write: quantize its rows,
    compress every span the chunk completes, the window ring."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    from oracle import hca as oh
    from oracle import indexer as oi
    from oracle.fp8 import bf16_round, quantize_rows

    chunk, off, D, seed = args
    rng = np.random.default_rng(seed)
    lat = bf16_round(rng.standard_normal((chunk, D)).astype(np.float32))
    kvs = bf16_round(rng.standard_normal((chunk + 128, 2 * D)).astype(np.float32))
    ape = (rng.standard_normal((128, D)) * 0.5).astype(np.float32)
    norm_w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    t0 = time.perf_counter()
    quantize_rows(lat)
    first, last = off // 128, (off + chunk) // 128
    for j in range(first, last):
        r0 = 128 * j - off + 128  # kvs row of position 128 j (state rows before the chunk start at row 0..127)
        cs = oi.rope_cos_sin(np.array([128 * j]), 64, 1.6e5)[0]
        y = oh.compress_span(kvs[r0:r0 + 128, :D], kvs[r0:r0 + 128, D:], ape, norm_w, 1e-6, cs)
        quantize_rows(y[None])
    return time.perf_counter() - t0


def _cpu_hca_decode_row(args):
    """Oracle of one HCA decode row: 64-head decode over its compressed
    entries and 128-row window, plus the new row's quantization."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    from oracle import decode as od
    from oracle.fp8 import bf16_round, decode_e4m3, quantize_rows

    ctx, seed = args
    rng = np.random.default_rng(seed)
    n = ctx // 128 + 128
    codes = rng.integers(0, 256, (n, 576)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] ^= 1
    q = bf16_round(rng.standard_normal((1, 64, 576)).astype(np.float32))
    sinks = rng.standard_normal(64).astype(np.float32)
    new = bf16_round(rng.standard_normal((1, 576)).astype(np.float32))
    t0 = time.perf_counter()
    quantize_rows(new)
    rows = decode_e4m3(codes).astype(np.float64) * 2.0 ** -8
    od.sparse_mla_decode(q, lambda s: rows[s], np.arange(n)[None], 256 ** -0.5, 512, sinks)
    return time.perf_counter() - t0


def _cpu_hca_small_seq(args):
    """Oracle of one sequence of the small bf16 HCA layer workload: its 4096
    rows into a bf16 pool, its 32 spans compressed, the window ring, then
    its 16-head decode over 32 + 128 rows."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    from oracle import decode as od
    from oracle import hca as oh
    from oracle import indexer as oi
    from oracle.fp8 import bf16_from_bits, bf16_round

    ctx, D, heads, seed = args
    rng = np.random.default_rng(seed)
    lat = bf16_round(rng.standard_normal((ctx, D)).astype(np.float32))
    kvs = bf16_round((rng.standard_normal((ctx, 2 * D)) * 1.28).astype(np.float32))
    ape = (rng.standard_normal((128, D)) * 0.02).astype(np.float32)
    q = bf16_round(rng.standard_normal((1, heads, D)).astype(np.float32))
    sinks = rng.standard_normal(heads).astype(np.float32)
    pages = ctx // 64 + 3
    bt = rng.permutation(pages).astype(np.int32)
    comp_bt, ring_pages = bt[None, -3:-2], bt[None, -2:]
    pos = np.arange(ctx, dtype=np.int64)
    slots = bt[pos // 64].astype(np.int64) * 64 + pos % 64
    cs = oi.rope_cos_sin(np.arange(ctx // 128 + 1) * 128, 64, 1.6e5)
    t0 = time.perf_counter()
    st = oh.HcaState(pages, D, 1, bf16=True)
    oh.hca_write(st, lat, kvs, pos, np.zeros(ctx, np.int32), np.array([0, ctx], np.int32), slots, ring_pages, 128,
                 comp_bt, np.zeros(1, np.int32), ape, np.ones(D, np.float32), 1e-6, cs)
    idx, lens = oh.hca_decode_indices(np.array([ctx - 1]), np.zeros(1, np.int32), comp_bt, ring_pages, 128,
                                      ctx // 128 + 128)
    vals = bf16_from_bits(st.pool.view(np.uint16).reshape(-1, D))
    od.sparse_mla_decode(q, lambda s: od.gather_rows_bf16(vals, s), idx, D ** -0.5, 512, sinks, lengths=lens)
    return time.perf_counter() - t0


def _pool_run(fn, jobs):
    import multiprocessing as mp

    workers = min(_cpu_workers(), len(jobs))
    t0 = time.perf_counter()
    with mp.get_context("fork").Pool(workers) as pool:
        busy = pool.map(fn, jobs, chunksize=1)
    return time.perf_counter() - t0, sum(busy), workers


def cpu_baselines(B: int, ctx: int, seed: int) -> dict:
    """The numpy oracle on the host's cores (a process pool, one job per
    query row or sequence), each on the full workload of its leg.  Run
    before the GPU is initialized."""
    import numpy as np

    out = {}
    wall, busy, workers = _pool_run(_cpu_dsa_row, [(ctx, seed * 1000 + r) for r in range(B)])
    by = dsa_bytes(B, ctx)["total"]
    out["dsa"] = {
        "value": round(by / wall / 1e9, 4), "unit": "GB/s", "cores": workers, "kind": "port",
        "sample": f"the whole headline step on the CPU: {B} query rows at ctx {ctx} (exact scores of "
                  f"{max(ctx - 128, 0)} N(0,1) keys each with 5% identical spike rows, top-2048, 64-head decode "
                  f"over 2176 rows), numpy oracle, one row per job on {workers} processes (the GPU box's CPU share "
                  f"is 16 cores): {wall:.2f} s wall, {busy:.1f} core-s",
        "tok_per_s": round(B / wall, 3), "ms_per_step": round(wall * 1e3, 1),
    }
    rng = np.random.default_rng(seed + 1)
    offs = rng.integers(0, 65536, 16)
    wall, busy, workers = _pool_run(_cpu_hca_write_seq, [(8192, int(o), 576, seed * 1000 + i) for i, o in
                                                         enumerate(offs)])
    spans = int(((offs + 8192) // 128 - offs // 128).sum())
    by = hca_write_bytes(16 * 8192, 576, 16, spans)
    out["hca_write"] = {
        "value": round(by["with_kv_score"] / wall / 1e9, 4), "unit": "GB/s", "cores": workers, "kind": "port",
        "sample": f"the whole chunked-prefill write on the CPU: 16 sequences x 8192 rows quantized and {spans} spans "
                  f"compressed, numpy oracle, one sequence per job on {workers} processes: {wall:.2f} s wall, "
                  f"{busy:.1f} core-s",
        "ms": round(wall * 1e3, 1),
    }
    wall, busy, workers = _pool_run(_cpu_hca_small_seq, [(4096, 576, 16, seed * 1000 + 7 + i) for i in range(4)])
    out["hca_small"] = {
        "value": round(4 / wall, 3), "unit": "sequences/s", "cores": workers, "kind": "port",
        "sample": f"the whole small bf16 HCA layer step on the CPU: 4 sequences x 4096 rows into a bf16 pool, 128 "
                  f"spans compressed, window ring, 16-head decode over 32 + 128 rows, numpy oracle, one sequence per "
                  f"job on {workers} processes: {wall:.2f} s wall, {busy:.1f} core-s",
        "ms": round(wall * 1e3, 1),
    }
    ctxs = rng.integers(8192, 131072, 64)
    wall, busy, workers = _pool_run(_cpu_hca_decode_row, [(int(c), seed * 1000 + i) for i, c in enumerate(ctxs)])
    rows = int((ctxs // 128 + 128).sum())
    byd = rows * 580 + 64 * (64 * 576 * 2 + 64 * 512 * 2 + 64 * 4)
    out["hca_decode"] = {
        "value": round(byd / wall / 1e9, 4), "unit": "GB/s", "cores": workers, "kind": "port",
        "sample": f"the whole 64-row HCA decode step on the CPU ({rows} index entries), numpy oracle, one row per "
                  f"job on {workers} processes: {wall:.2f} s wall, {busy:.1f} core-s",
        "tok_per_s": round(64 / wall, 3),
    }
    return out


# --------------------------------------------------------------------------- main
def time_dsa(torch, ops, st, steps: int, warmup: int):
    """(graph-replay ms, eager ms, indexer top-k call ms, decode call ms) of the
    DSA step on `st`: `steps` eager steps with events around the top-k and
    decode calls, then `steps` replays of one captured step."""
    torch.cuda.synchronize()
    for _ in range(warmup):
        dsa_step(ops, st)
    torch.cuda.synchronize()
    evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(4)) for _ in range(steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for i in range(steps):
        dsa_step(ops, st, evs[i])
    t_end.record()
    torch.cuda.synchronize()
    ms_eager = t_start.elapsed_time(t_end) / steps
    # the timed steps: replays of one captured step (the whole DSA step is
    # graph-capturable: fixed workspaces, no host synchronization)
    ms_step = graph_ms(torch, lambda: dsa_step(ops, st), steps)
    filt_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
    dec_ms = sum(e[2].elapsed_time(e[3]) for e in evs) / steps
    return ms_step, ms_eager, filt_ms, dec_ms


def model_layer_kinds() -> list:
    """Attention kind of each of the model's 43 layers: 6 DSA, 37 HCA.
    Which layers are DSA is a checkpoint setting (compress_ratios); here
    they are spread evenly (layer i is DSA when i % 7 == 3)."""
    kinds = ["dsa" if i % 7 == 3 else "hca" for i in range(MODEL_LAYERS["dsa"] + MODEL_LAYERS["hca"])]
    assert kinds.count("dsa") == MODEL_LAYERS["dsa"]
    return kinds


def measure_model_step(torch, ops, args, reps: int = 10) -> dict:
    """The model's attention KV path for one decode step as a serving engine
    runs it: the 43 layers' steps at the headline batch and context, in
    layer order, each layer with its own caches and inputs (its own seed: a
    DSA layer's keys carry their own +4 sigma spikes), captured in one HIP
    graph and replayed (`ms`); `ms_eager` = the same launches eagerly."""
    layers = []
    for i, kind in enumerate(model_layer_kinds()):
        seed = args.seed + 1000 + i
        if kind == "dsa":
            layers.append((kind, build_dsa_decode(torch, ops, [args.ctx] * args.batch, seed)))
        else:
            layers.append((kind, build_hca_decode(torch, ops, seed, ctxs=[args.ctx] * args.batch)))
    torch.cuda.synchronize()

    def step():
        for kind, st in layers:
            if kind == "dsa":
                dsa_step(ops, st)
            else:
                hca_decode_step(ops, st)

    ms_eager = time_ms(torch, step, reps)
    ms_graph = graph_ms(torch, step, reps)
    del layers
    return {"ms": round(ms_graph, 4), "ms_eager": round(ms_eager, 4),
            "layers": f"{MODEL_LAYERS['dsa']} DSA + {MODEL_LAYERS['hca']} HCA, layer i DSA when i % 7 == 3",
            "measured": "the 43 layers' DSA / HCA decode steps (each layer its own caches) captured in one HIP "
                        "graph and replayed; ms_eager = the same launches eagerly"}


def measure_dsa_random_row(torch, ops, args) -> dict:
    """The DSA step at the headline shape on uniformly random key codes with
    one random spike row in 5% of the positions (its score is random, so it
    ties the threshold of only some rows)."""
    st = build_dsa_decode(torch, ops, [args.ctx] * args.batch, args.seed, spikes="random_row")
    ms_step, ms_eager, filt_ms, dec_ms = time_dsa(torch, ops, st, args.steps, args.warmup)
    by = dsa_bytes(args.batch, args.ctx)
    del st
    return {
        "workload": f"dsa_decode_b{args.batch}_ctx{args.ctx}_random_spike_row",
        "ms": round(ms_step, 4), "ms_eager": round(ms_eager, 4),
        "GB/s": round(by["total"] / (ms_step * 1e-3) / 1e9, 1),
        "frac": round(by["total"] / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "indexer_topk_ms": round(filt_ms, 4), "decode_ms": round(dec_ms, 4),
        "what": "the headline DSA step (graph replays) on uniformly random fp8 key codes at scale 2^-8 with one "
                "random key row copied into 5% of the positions",
    }


def measure_dsa(torch, ops, args, line: dict) -> None:
    st = build_dsa_decode(torch, ops, [args.ctx] * args.batch, args.seed)
    if args.copy_mb > 0:
        src = torch.ones(args.copy_mb << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        del src, dst
    ms_step, ms_eager, filt_ms, dec_ms = time_dsa(torch, ops, st, args.steps, args.warmup)
    by = dsa_bytes(args.batch, args.ctx)
    gbs = by["total"] / (ms_step * 1e-3) / 1e9
    n = max(args.ctx - 128, 0)
    filt_gbs = by["indexer_k"] / (filt_ms * 1e-3) / 1e9
    filt_tflops = args.batch * n * 64 * 128 * 2 / (filt_ms * 1e-3) / 1e12
    # decode contractions: S = Q K^T over the 576-wide rows and O = P V over
    # their first 512 columns (twice: the hi and lo bf16 parts of P), 64 heads
    # x 2176 rows per query row
    dec_flops = args.batch * 64 * (min(n, 2048) + min(args.ctx, 128)) * (576 + 2 * 512) * 2
    workload = f"dsa_decode_b{args.batch}_ctx{args.ctx}"
    traffic = traffic_of(workload, HEADLINE_KERNEL)
    line.update({
        "value": round(gbs, 2),
        "unit": "GB/s",
        "pct_of_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_eager": round(ms_eager, 4),
        "launch": "hip_graph: the timed steps replay one captured DSA step (the indexer top-k with the "
                  "step's prologue folded into its launch and the merged rows, decode, combine); "
                  "ms_per_step_eager = the same steps launched eagerly",
        "tok_per_s_dsa_layer": round(args.batch / (ms_step * 1e-3), 1),
        "config": {
            "workload": workload,
            "batch": args.batch, "ctx": args.ctx, "index_topk": 2048, "window": 128, "heads": 64,
            "latent_dim": 576, "indexer": "64x128 fp8", "kv_cache": "fp8 e4m3 + fp32 per-token scale",
            "keys": "N(0,1) rows through the K insert; per sequence 5% of the scored positions hold a spike row "
                    "whose exact score is mean + 4 sigma of the row's ordinary scores (every row's top-2048 ends in "
                    "a lowest-index tie among its spikes)",
            "spike_sigma": [min(st["spikes"]["sigma"]), max(st["spikes"]["sigma"])],
            "spikes_per_row": round(sum(st["spikes"]["per_row"]) / len(st["spikes"]["per_row"]), 1),
            "bytes_per_step": by,
        },
        "roofline": {
            "kernel": f"ekv_dsa_decode_prologue_topk_merged = {HEADLINE_KERNEL} (the step's prologue -- q and k "
                      "prep, K and latent appends, q quantization -- folded into the one-launch top-k: fp8-MFMA "
                      "filter over every key row, candidate bound, exact scoring of the candidates, exact "
                      "top-2048 and the merged rows), timed by events around the call",
            "bound": "hbm",
            "achieved": round(filt_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(filt_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": f"{TRAFFIC_FILE.relative_to(ROOT)} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this "
                              "workload, scaled by a plain copy's readings)" if traffic else None,
            "traffic_vs_algorithmic": round(traffic / by["indexer_k"], 4) if traffic else None,
            "ms": round(filt_ms, 4),
            "bytes_per_launch": by["indexer_k"],
            "mfma_fp8_tflops_algorithmic": round(filt_tflops, 1),
            "mfma": mfma_report(workload, HEADLINE_KERNEL, filt_ms),
        },
        "decode": {
            "kernels": "sparse_decode_kernel<576> + decode_combine_kernel (ekv_sparse_mla_decode), timed by events "
                       "around the call",
            "ms": round(dec_ms, 4),
            "bytes": by["gather"],
            "GB/s_gather": round(by["gather"] / (dec_ms * 1e-3) / 1e9, 1),
            "mfma_bf16_tflops_algorithmic": round(dec_flops / (dec_ms * 1e-3) / 1e12, 1),
            "mfma": mfma_report(workload, "sparse_decode_kernel<576>", None),
        },
    })


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU (one DP rank's share of the attention "
                                   "work); --gpus must be 1", "n_gpus": args.gpus}))
        sys.exit(2)
    # CPU baselines first: the process pool forks before the GPU is touched
    cpu = None
    if not args.no_cpu_baseline and args.only is None:
        cpu = cpu_baselines(args.batch, args.ctx, args.seed)
    import torch
    from ernie_kv import ops

    torch.cuda.init()
    if args.only is not None:
        if args.only == "dsa":
            line = {}
            measure_dsa(torch, ops, args, line)
            print(json.dumps(line), flush=True)
            return
        if args.only == "dsa_random_row":
            print(json.dumps(measure_dsa_random_row(torch, ops, args)), flush=True)
            return
        if args.only == "model":  # the 43 layers' step in one graph
            print(json.dumps(measure_model_step(torch, ops, args)), flush=True)
            return
        if args.only == "hca_layer":  # the HCA decode step at the headline batch and context
            print(json.dumps(measure_hca_decode(torch, ops, args.seed, ctxs=[args.ctx] * args.batch,
                                                label=f"hca_decode_b{args.batch}_ctx{args.ctx}")), flush=True)
            return
        leg = {"hca_write": measure_hca_write, "hca_decode": measure_hca_decode, "mtp": measure_mtp,
               "hca_small": measure_hca_small,
               "indexer_fp4": measure_indexer_fp4, "dsa_prefill": measure_dsa_prefill,
               "pages": measure_pages}[args.only]
        print(json.dumps(leg(torch, ops, args.seed)), flush=True)
        return
    line = {"metric": METRIC}
    measure_dsa(torch, ops, args, line)
    torch.cuda.empty_cache()
    # the HCA layers' decode step at the headline shape, for the model step
    hca_head = measure_hca_decode(torch, ops, args.seed, ctxs=[args.ctx] * args.batch,
                                  label=f"hca_decode_b{args.batch}_ctx{args.ctx}")
    torch.cuda.empty_cache()
    # both layer types as graph replays (the serving mode), composed
    dsa_ms = line["ms_per_step"]
    hca_ms = hca_head["ms_graph"]
    composed_ms = MODEL_LAYERS["dsa"] * dsa_ms + MODEL_LAYERS["hca"] * hca_ms
    model = measure_model_step(torch, ops, args)
    torch.cuda.empty_cache()
    model_ms = model["ms"]
    line.update({
        "tok_per_s": round(args.batch / (model_ms * 1e-3), 1),
        "model_step": {**model,
                       "composed_ms": round(composed_ms, 4),
                       "composed": "6 x the DSA step + 37 x the HCA decode step (hca_layer) at the same batch and "
                                   "context, each timed as replays of its own one-layer graph",
                       "dsa_ms": round(dsa_ms, 4), "hca_ms": round(hca_ms, 4),
                       "hca_layer": hca_head},
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8", "data": "synthetic",
    })
    line["dsa_random_spike_row"] = measure_dsa_random_row(torch, ops, args)
    torch.cuda.empty_cache()
    if not args.no_hca:
        line["hca_small"] = measure_hca_small(torch, ops, args.seed)
        torch.cuda.empty_cache()
        line["hca_write"] = measure_hca_write(torch, ops, args.seed)
        torch.cuda.empty_cache()
        line["hca_decode"] = measure_hca_decode(torch, ops, args.seed)
    if not args.no_mtp:
        torch.cuda.empty_cache()
        line["mtp"] = measure_mtp(torch, ops, args.seed)
    if not args.no_fp4:
        torch.cuda.empty_cache()
        line["indexer_fp4"] = measure_indexer_fp4(torch, ops, args.seed, B=args.batch, ctx=args.ctx)
    if not args.no_prefill:
        torch.cuda.empty_cache()
        line["dsa_prefill"] = measure_dsa_prefill(torch, ops, args.seed)
    if not args.no_pages:
        torch.cuda.empty_cache()
        line["pages"] = measure_pages(torch, ops, args.seed)
    if cpu is not None:
        line["cpu_baseline"] = cpu["dsa"]
        if "hca_write" in line:
            line["hca_write"]["cpu_baseline"] = cpu["hca_write"]
        if "hca_decode" in line:
            line["hca_decode"]["cpu_baseline"] = cpu["hca_decode"]
        if "hca_small" in line:
            line["hca_small"]["cpu_baseline"] = cpu["hca_small"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
