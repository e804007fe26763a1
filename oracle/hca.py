"""HCA write path: append + fp8 quant, 128->1 span compressor, window ring (oracle).

Reference: the HCA layer (``src/vllm_ernie/models/ernie5_5/nvidia/attention.py``
``:398-408, 471-539``) hands the projected compressor input ``kv_score`` (the
``compressor.fused_wkv_wgate`` output, ``nvidia/model.py:684-685``) and the
per-token latent to upstream ``DeepseekV4Attention._prepare_and_attn_fn``,
which appends the latent by ``slot_mapping`` and runs ``DeepseekCompressor``
(state cache + ``c128_boundary``).  vLLM 0.32.0 is absent, so the compressor
below is a restatement of the DeepSeek-V4 compressor as described by its call
sites -- **parity unpinned** against upstream; it is pinned against closed
forms (constant gate -> mean, one-hot gate -> copy, permutation invariance) and
an fp64 brute force in ``tests/test_oracle_paths.py``.  Its RoPE pairing
(interleaved pairs of the last 64 channels, rotated forward) is pinned by the
reference's own inverse rotation of these rows (``_vha_inv_rope_quant_kernel``,
``attention.py:166-229``, restated in ``oracle.quant``), which undoes it; the
rotation position 128 j of compressed entry j stays parity unpinned.

Compressor of span j (positions 128j .. 128j+127), per channel c < D: the
softmax over the span of g_i = fl32(score_i[c] + ape[i, c]) weights kv_i[c].
It is evaluated in one pass, as an online softmax over 4 interleaved row
groups (group r holds rows r, r+4, ..., r+124) in chunks of 4 of a group's
rows, then a fixed-order merge of the groups.  A group's shift m_r moves (and
its sums are rescaled) only when a chunk's max exceeds it by more than
SLACK = 8, so every term is at most e**8::

    for r in 0..3:
        m_r, Z_r, N_r = -inf, 0, 0
        for each chunk C of group r's rows, in order:
            mc = max(m_r, max_{i in C} g_i)
            if mc > fl32(m_r + SLACK):
                s = exp_ekv(fl32(m_r - mc));  Z_r = fl32(Z_r * s);  N_r = fl32(N_r * s);  m_r = mc
            for i in C, in order:
                e = exp_ekv(fl32(g_i - m_r))
                Z_r = fl32(Z_r + e);  N_r = fma(e, kv_i[c], N_r)
    M = max_r m_r;  Z, N = 0, 0
    for r in 0..3:  s = exp_ekv(fl32(m_r - M));  Z = fma(Z_r, s, Z);  N = fma(N_r, s, N)
    x_c = fl32(N / Z)
    RMSNorm over D (eps from rms_norm_eps), sums in the kernel's order
    RoPE (interleaved pairs) on channels D-64..D-1 at position 128j
    UE8M0 fp8 quant -> compressed row j

``exp_ekv`` is this build's own exp: ``2**n * P(f)`` with ``n = rint(x*log2 e)``,
``f = x*log2 e - n`` and ``P`` a degree-5 polynomial fit of ``2**f`` (``EXP_C``)
evaluated by Horner in fp32 with fused multiply-adds, flushing to 0 below
``2**-125``.  ``fma(a, b, c)`` is ``a*b + c`` with one fp32 rounding (``fma32``
below).  The kernel evaluates the same operations.

State: the kv_score rows of a sequence's most recent 256 positions live in a
ring ``state[state_slot, pos % 256]`` so a span that completes in a later call
(or is re-completed after an MTP rollback) can be recompressed.
Window ring: the fp8 rows of the most recent ``R`` positions (``R`` a multiple
of 64, >= 128 + draft tokens) in pages named by ``ring_pages[seq]``.
"""

from __future__ import annotations

import math

import numpy as np

from .fp8 import bf16_bits, bf16_round, quantize_rows
from .paged import PAGE_TOKENS, write_fp8_rows

SPAN = 128
STATE_RING = 256
WINDOW = 128

LOG2E = np.float32(1.0 / math.log(2.0))
# P(f) ~ 2**f on [-1/2, 1/2]: degree 5, P(0) = 1 exactly, fp32 coefficients
# fit to the relative error of the fp32 evaluation; within 2x of the exact
# minimax error (9.1e-8) and, evaluated in fp32 Horner with fused
# multiply-adds, below 2.2e-7 relative error.  tests/test_oracle_paths.py
# re-derives the minimax fit by a Remez exchange and checks these bounds.
EXP_C = [np.float32(float.fromhex(h)) for h in (
    "0x1.0p+0", "0x1.62e428p-1", "0x1.ebf918p-3", "0x1.c6b6e4p-5", "0x1.3d0c52p-7", "0x1.5c08e6p-10")]


def fma32(a, b, c) -> np.ndarray:
    """fp32 fused multiply-add ``round_fp32(a*b + c)`` with one rounding
    (nearest-even), for finite fp32 inputs whose result is a normal fp32.

    ``a*b`` is exact in fp64 (48 significant bits); ``s = fl64(a*b + c)`` and
    its exact remainder ``err`` (Knuth's TwoSum) give the exact sum
    ``s + err``.  Rounding ``s`` to fp32 is then the correct rounding of the
    exact sum unless ``s`` sits exactly halfway between two fp32 neighbours
    and ``err != 0``; in that case the neighbour on ``err``'s side is the
    correctly rounded result."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    p = a64 * b64
    s = p + c64
    bb = s - p
    err = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    d = s - r.astype(np.float64)
    toward = np.where(d > 0, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
    other = np.nextafter(r, toward).astype(np.float32)
    mid = (d != 0) & (s == (r.astype(np.float64) + other.astype(np.float64)) * 0.5)
    # at a midpoint r is the even neighbour; err decides between r and other
    pick_other = mid & (err != 0) & (np.sign(err) == np.sign(d))
    return np.where(pick_other, other, r).astype(np.float32)


def exp_ekv(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    t = (x * LOG2E).astype(np.float32)
    n = np.rint(t).astype(np.float32)
    f = (t - n).astype(np.float32)
    p = np.broadcast_to(EXP_C[5], f.shape).astype(np.float32)
    for k in range(4, -1, -1):
        p = fma32(p, f, EXP_C[k])
    out = np.ldexp(p, np.clip(n, -200, 200).astype(np.int32)).astype(np.float32)
    return np.where(t < np.float32(-125.0), np.float32(0.0), out).astype(np.float32)


ROW_GROUPS = 4           # interleaved row groups of the online softmax
CHUNK = 4                # rows of a group per online-softmax step
SLACK = np.float32(8.0)  # a chunk max above shift + SLACK moves the shift


def span_softmax_sum(g: np.ndarray, kv: np.ndarray) -> np.ndarray:
    """sum_i softmax_i(g) * kv_i per channel, in the one-pass order above
    (``g, kv [..., 128, D]`` fp32, any leading span dimensions; returns
    ``x [..., D]``)."""
    f32 = np.float32
    shape = g.shape[:-2] + g.shape[-1:]
    ms, Zs, Ns = [], [], []
    with np.errstate(invalid="ignore", over="ignore"):
        for r in range(ROW_GROUPS):
            m = np.full(shape, -np.inf, f32)
            Z = np.zeros(shape, f32)
            N = np.zeros(shape, f32)
            rows = np.arange(r, SPAN, ROW_GROUPS)
            for k0 in range(0, len(rows), CHUNK):
                chunk = rows[k0 : k0 + CHUNK]
                mc = np.maximum(m, g[..., chunk, :].max(axis=-2))
                move = mc > (m + SLACK).astype(f32)
                s = exp_ekv((m - mc).astype(f32))
                Z = np.where(move, (Z * s).astype(f32), Z)
                N = np.where(move, (N * s).astype(f32), N)
                m = np.where(move, mc, m)
                for i in chunk:
                    e = exp_ekv((g[..., i, :] - m).astype(f32))
                    Z = (Z + e).astype(f32)
                    N = fma32(e, kv[..., i, :], N)
            ms.append(m), Zs.append(Z), Ns.append(N)
        M = np.max(np.stack(ms), axis=0)
        Z = np.zeros(shape, f32)
        N = np.zeros(shape, f32)
        for r in range(ROW_GROUPS):
            s = exp_ekv((ms[r] - M).astype(f32))
            Z = fma32(Zs[r], s, Z)
            N = fma32(Ns[r], s, N)
    return (N / Z).astype(f32)


def compress_span(
    kv: np.ndarray,
    score: np.ndarray,
    ape: np.ndarray,
    norm_w: np.ndarray,
    eps: float,
    cos_sin: np.ndarray,
) -> np.ndarray:
    """The compressed row (fp32 before quant) of each span: ``kv, score
    [..., 128, D]`` (bf16 values) and ``cos_sin [..., 64]`` with the same
    leading span dimensions (none for one span); returns ``[..., D]``."""
    f32 = np.float32
    kv = np.asarray(kv, f32)
    D = kv.shape[-1]
    g = (np.asarray(score, f32) + np.asarray(ape, f32)).astype(f32)
    x = span_softmax_sum(g, kv)
    sq = (x * x).astype(f32).reshape(x.shape[:-1] + (D // 4, 4))
    part = np.zeros(sq.shape[:-1], f32)
    for k in range(4):
        part = (part + sq[..., k]).astype(f32)
    S = np.zeros(x.shape[:-1], f32)
    for q in range(D // 4):
        S = (S + part[..., q]).astype(f32)
    ms = (S / f32(D)).astype(f32)
    r = (f32(1.0) / np.sqrt((ms + f32(eps)).astype(f32))).astype(f32)
    y = ((x * r[..., None]).astype(f32) * np.asarray(norm_w, f32)).astype(f32)
    cs = np.asarray(cos_sin, f32)
    x0 = y[..., D - 64 :: 2].copy()
    x1 = y[..., D - 63 :: 2].copy()
    c, s = cs[..., :32], cs[..., 32:64]
    y[..., D - 64 :: 2] = ((x0 * c).astype(f32) - (x1 * s).astype(f32)).astype(f32)
    y[..., D - 63 :: 2] = ((x0 * s).astype(f32) + (x1 * c).astype(f32)).astype(f32)
    return y


def ring_slot(ring_pages: np.ndarray, seq: int, pos: int, ring: int) -> int:
    r = pos % ring
    return int(ring_pages[seq, r // PAGE_TOKENS]) * PAGE_TOKENS + r % PAGE_TOKENS


def comp_slot(comp_block_table: np.ndarray, seq: int, j: int) -> int:
    return int(comp_block_table[seq, j // PAGE_TOKENS]) * PAGE_TOKENS + j % PAGE_TOKENS


class HcaState:
    """Numpy model of every buffer the HCA write path touches."""

    def __init__(self, num_pages: int, dim: int, num_state: int, stride: int | None = None, bf16: bool = False):
        """``bf16``: a pool of bf16 rows (64 rows of ``dim`` bf16 values a
        page, no scales; the non-fp8 HCA cache) instead of fp8 rows with
        per-token scales."""
        self.dim = dim
        self.bf16 = bf16
        if stride is None:
            stride = PAGE_TOKENS * (2 * dim if bf16 else dim + 4)
        self.pool = np.zeros((num_pages, stride), dtype=np.uint8)
        self.state = np.zeros((num_state, STATE_RING, 2 * dim), dtype=np.float32)

    def store(self, slots, rows: np.ndarray) -> None:
        """Rows ``[n, dim]`` (fp32 values) into their slots: UE8M0 fp8 with
        per-token scales, or rounded to bf16 (nearest even) in a bf16 pool;
        negative slots are skipped."""
        rows = np.asarray(rows, np.float32)
        if not self.bf16:
            codes, scale = quantize_rows(rows)
            write_fp8_rows(self.pool, slots, codes, scale, self.dim)
            return
        bits = bf16_bits(rows).view(np.uint8).reshape(len(rows), 2 * self.dim)
        for i, slot in enumerate(np.asarray(slots, np.int64)):
            if slot >= 0:
                off = (slot % PAGE_TOKENS) * 2 * self.dim
                self.pool[slot // PAGE_TOKENS, off:off + 2 * self.dim] = bits[i]


def hca_write(
    st: HcaState,
    latent: np.ndarray,
    kv_score: np.ndarray,
    positions: np.ndarray,
    token_seq: np.ndarray,
    qsl: np.ndarray,
    slot_mapping: np.ndarray,
    ring_pages: np.ndarray | None,
    ring: int,
    comp_block_table: np.ndarray | None,
    state_slot: np.ndarray,
    ape: np.ndarray,
    norm_w: np.ndarray,
    eps: float,
    comp_cos_sin: np.ndarray,
) -> None:
    """Apply one call: compress completed spans (from the pre-call state and
    this call's rows), then append, update the ring and the state ring."""
    D = st.dim
    positions = np.asarray(positions, np.int64)
    B = len(qsl) - 1
    if comp_block_table is not None:
        spans, js, slots = [], [], []
        for b in range(B):
            t0, t1 = int(qsl[b]), int(qsl[b + 1])
            if t1 <= t0:
                continue
            p0, pl = int(positions[t0]), int(positions[t0]) + (t1 - t0) - 1
            for j in range(p0 // SPAN, (pl + 1) // SPAN):
                rows = np.empty((SPAN, 2 * D), np.float32)
                for i in range(SPAN):
                    p = SPAN * j + i
                    if p >= p0:
                        rows[i] = kv_score[t0 + p - p0]
                    else:
                        rows[i] = st.state[int(state_slot[b]), p % STATE_RING]
                spans.append(rows)
                js.append(j)
                slots.append(comp_slot(comp_block_table, b, j))
        if spans:
            rows = np.stack(spans)
            y = compress_span(rows[..., :D], rows[..., D:], ape, norm_w, eps, np.asarray(comp_cos_sin)[js])
            st.store(slots, y)
    latent = np.asarray(latent, np.float32)
    st.store(slot_mapping, latent)
    for b in range(B):
        t0, t1 = int(qsl[b]), int(qsl[b + 1])
        if t1 <= t0:
            continue
        p0 = int(positions[t0])
        pl = p0 + (t1 - t0) - 1
        for t in range(t0, t1):
            p = p0 + (t - t0)
            if ring_pages is not None and p > pl - ring:
                st.store([ring_slot(ring_pages, b, p, ring)], latent[t : t + 1])
            if comp_block_table is not None and p > pl - STATE_RING:
                st.state[int(state_slot[b]), p % STATE_RING] = kv_score[t]


def hca_decode_indices(
    positions: np.ndarray,
    req_ids: np.ndarray,
    comp_block_table: np.ndarray,
    ring_pages: np.ndarray,
    ring: int,
    width: int,
    window: int = WINDOW,
    call_qsl: np.ndarray | None = None,
    call_slots: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """Global slots ``[comp 0..n_c-1 | window p-w+1..p | -1...]`` and lengths.
    With the call's ``call_qsl`` / ``call_slots``, window positions at or
    after the first call position of the row's request are that token's
    slot, older ones ring slots."""
    T = len(positions)
    out = np.full((T, width), -1, dtype=np.int32)
    lens = np.zeros(T, dtype=np.int32)
    for t in range(T):
        p = int(positions[t])
        b = int(req_ids[t])
        n_c = (p + 1) // SPAN
        w = min(p + 1, window)
        assert n_c + w <= width
        for j in range(n_c):
            out[t, j] = comp_slot(comp_block_table, b, j)
        first = int(positions[int(call_qsl[b])]) if call_slots is not None else None
        for i in range(w):
            q = p - w + 1 + i
            if first is not None and q >= first:
                s = int(call_slots[int(call_qsl[b]) + q - first])
                out[t, n_c + i] = s if s >= 0 else -1
            else:
                out[t, n_c + i] = ring_slot(ring_pages, b, q, ring)
        lens[t] = n_c + w
    return out, lens


def bf16_values(x: np.ndarray) -> np.ndarray:
    return bf16_round(np.asarray(x, np.float32))
