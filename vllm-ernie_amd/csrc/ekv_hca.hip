// HCA 128->1 span compressor (the C128 compression of an HCA layer).
//
// One workgroup per span that completes in this call: the span's 128 rows of
// kv_score (the compressor projection [kv | score], bf16) come from this
// call's input for positions >= the sequence's first new position, and from
// the per-sequence state ring (positions % 256) for earlier positions.  Per
// channel c the workgroup forms the softmax over the span of
// g_i = score_i[c] + ape[i, c] weighting kv_i[c], in one pass: an online
// softmax per row group (group r holds rows r, r+4, ..., r+124), in chunks of
// 4 of the group's rows,
//
//   mc = max(m, g over the chunk)
//   if mc > m + 8:  s = exp_ekv(m - mc);  Z *= s;  N *= s;  m = mc
//   per row in order:  e = exp_ekv(g_i - m);  Z += e;  N = fma(e, kv_i[c], N)
//
// then the groups merged in order, M = max_r m_r, Z = fma(Z_r, s_r, Z),
// N = fma(N_r, s_r, N) with s_r = exp_ekv(m_r - M), and x_c = N / Z.
// Then RMSNorm over the row (sum of squares: per lane over its 4 channels,
// then thread 0 over the lanes in order), interleaved RoPE on the last 64
// channels at position 128*j (cos/sin table row j), and the per-token UE8M0
// fp8 quant; the row is written to the compressed page slot of span j.
//
// Must run before ekv_hca_append of the same call (the append overwrites the
// state ring rows this kernel may still read).  Built with -ffp-contract=off
// (the only fused multiply-adds are the explicit ones) and correctly rounded
// fp32 division / square root: the CPU oracle evaluates the same operations
// in the same order.
#include "ekv_common.h"
#include "ekv_internal.h"
#include "ekv_rows.h"

namespace ekv {

// exp(x) for x <= 88 as 2**n * P(f): n = rint(x * log2 e), f = x * log2 e - n,
// P a degree-5 polynomial fit of 2**f on [-1/2, 1/2] (Remez exchange on the
// relative error, fp32 coefficients, P(0) = 1), Horner with fused
// multiply-adds; 0 when x * log2 e < -125.  Branch-free: the polynomial is
// evaluated for every x and the flush is a select.
__device__ __forceinline__ float exp_ekv(float x) {
  const float t = x * 0x1.715476p+0f;
  const float n = rintf(t);
  const float f = t - n;
  float p = 0x1.5c08e6p-10f;
  p = __builtin_fmaf(p, f, 0x1.3d0c52p-7f);
  p = __builtin_fmaf(p, f, 0x1.c6b6e4p-5f);
  p = __builtin_fmaf(p, f, 0x1.ebf918p-3f);
  p = __builtin_fmaf(p, f, 0x1.62e428p-1f);
  p = __builtin_fmaf(p, f, 0x1.0p+0f);
  const float r = ldexpf(p, static_cast<int>(n));
  return t < -125.0f ? 0.0f : r;
}

struct CompressArgs {
  const uint16_t* kv_score;  // [T, kvs_stride] bf16: kv (D) | score (D)
  int64_t kvs_stride;
  const int64_t* positions;  // [T]
  const int32_t* qsl;        // [B + 1]
  const uint16_t* state;     // [num_state, 256, 2D] bf16
  const int32_t* state_slot; // [B]
  int32_t num_state;
  const float* ape;          // [128, D]
  const float* norm_w;       // [D]
  float eps;
  const float* cos_sin;      // [max_spans, 64]: cos[32] | sin[32]
  int32_t max_spans;
  const int32_t* comp_bt;    // [B, comp_bt_stride]
  int32_t comp_bt_stride;
  uint8_t* pool;             // [num_pages, page_stride]
  int64_t page_stride;
  int64_t num_pages;
  // Decode-sized writes with a workspace: a span is compressed by D / 64
  // four-wave workgroups (null: one workgroup per span).
  uint32_t* span_count;      // [B] arrivals per span (zero between calls)
  float* span_x;             // [B, D] softmax results
  float* span_part;          // [B, D/4] sums of squares per channel quad
  // pools of bf16 rows (page = 64 rows of D bf16 values, no scales): the
  // compressed row is stored rounded to bf16 (nearest even), not quantized
  int32_t bf16_rows;
};

// 4 channels of a compressed row as bf16 (round to nearest even), 8 bytes.
__device__ __forceinline__ uint2 bf16x4_pack(float y0, float y1, float y2, float y3) {
  return make_uint2(f32_to_bf16(y0) | (static_cast<uint32_t>(f32_to_bf16(y1)) << 16),
                    f32_to_bf16(y2) | (static_cast<uint32_t>(f32_to_bf16(y3)) << 16));
}

// Third descriptor word of a raw (unswizzled, unformatted) buffer resource.
constexpr int kBufferWord3 = 0x00020000;

constexpr int kRowGroups = 4;  // interleaved row groups: group r holds rows r, r+4, ...
constexpr int kChunk = 4;      // rows of a group per online-softmax step
constexpr int kGroupRows = kSpan / kRowGroups;

// Online-softmax state of one lane: 4 channels of one row group.
struct SoftmaxState {
  float m[4], Z[4], N[4];
};

__device__ __forceinline__ void bf16x4(uint2 v, float (&f)[4]) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
}

constexpr float kShiftSlack = 8.0f;  // a chunk max above shift + slack moves the shift

// Gate values g = score + ape of one chunk of kChunk rows (in group order).
__device__ __forceinline__ void gate_chunk(const uint2 (&sc)[kChunk], const float4 (&ap)[kChunk],
                                           float (&g)[kChunk][4]) {
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    float f[4];
    bf16x4(sc[u], f);
    g[u][0] = f[0] + ap[u].x;
    g[u][1] = f[1] + ap[u].y;
    g[u][2] = f[2] + ap[u].z;
    g[u][3] = f[3] + ap[u].w;
  }
}

// One chunk's terms: the shift m moves to the running max (and the sums are
// rescaled) only when the chunk's max exceeds it by more than kShiftSlack --
// a wave-uniform branch, rarely taken after the first chunk, which sets m
// without rescaling (its sums are still 0) -- then the rows' terms in order.
template <bool kFirst>
__device__ __forceinline__ void softmax_terms(SoftmaxState& s, const float (&g)[kChunk][4],
                                              const uint2 (&kv)[kChunk]) {
  float mc[4];
  bool move = false;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mc[k] = s.m[k];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) mc[k] = fmaxf(mc[k], g[u][k]);
    if (kFirst) s.m[k] = mc[k];
    else move |= mc[k] > s.m[k] + kShiftSlack;
  }
  if (!kFirst && __builtin_amdgcn_ballot_w64(move) != 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool mv = mc[k] > s.m[k] + kShiftSlack;
      const float r = exp_ekv(s.m[k] - mc[k]);
      s.Z[k] = mv ? s.Z[k] * r : s.Z[k];
      s.N[k] = mv ? s.N[k] * r : s.N[k];
      s.m[k] = mv ? mc[k] : s.m[k];
    }
  }
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    float v[4];
    bf16x4(kv[u], v);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float e = exp_ekv(g[u][k] - s.m[k]);
      s.Z[k] = s.Z[k] + e;
      s.N[k] = __builtin_fmaf(e, v[k], s.N[k]);
    }
    if (u + 1 < kChunk) __builtin_amdgcn_sched_barrier(0);  // one row's exps at a time: fewer live temporaries
  }
}

// softmax_terms for one channel (the same operations in the same order).
template <bool kFirst>
__device__ __forceinline__ void softmax_terms1(float& m, float& Z, float& N, const float (&g)[kChunk],
                                               const float (&kv)[kChunk]) {
  float mc = m;
#pragma unroll
  for (int u = 0; u < kChunk; ++u) mc = fmaxf(mc, g[u]);
  if (kFirst) {
    m = mc;
  } else {
    const bool mv = mc > m + kShiftSlack;
    if (__builtin_amdgcn_ballot_w64(mv) != 0) {
      const float r = exp_ekv(m - mc);
      Z = mv ? Z * r : Z;
      N = mv ? N * r : N;
      m = mv ? mc : m;
    }
  }
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    const float e = exp_ekv(g[u] - m);
    Z = Z + e;
    N = __builtin_fmaf(e, kv[u], N);
  }
}

// Workgroup-shared scratch of compress_span.
template <int D>
struct CompressLds {
  __align__(16) float part[D / 4];
  float wmax[D / 64];
  float rn;
  int last;
};

// The softmax of span j of a sequence (first row t0 at position p0, state
// slot st) for the 4 channels 4 quad .. 4 quad + 3, row group lane / 16 of
// this lane, merged over the 4 row groups in order: every lane of a column
// (lanes l, l+16, l+32, l+48 of the wave, which must share quad) ends with the
// same x, and part = their sum of squares in channel order.  Every
// kv_score element is read from memory once: the softmax is an online one per
// (row group, channel).  kRingPipe: spans that start in the state ring get
// the input path's load pipeline too (at the cost of more registers).
template <int D, bool kRingPipe>
__device__ __forceinline__ void span_softmax(const CompressArgs& a, int quad, int t0, int64_t p0, int64_t j, int st,
                                             float (&x)[4], float& part) {
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4;  // row group r
  const int c0 = 4 * quad;

  SoftmaxState sm;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    sm.m[k] = -INFINITY;
    sm.Z[k] = 0.0f;
    sm.N[k] = 0.0f;
  }
  // Row i of the span: this call's input for positions >= p0, else the
  // state ring (positions % 256), whose rows of span j are consecutive from
  // (j % 2) * 128; without a ring those rows count as score 0, kv 0.
  const int64_t split64 = p0 - j * kSpan;
  const __amdgpu_buffer_rsrc_t ape_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.ape), 0, kSpan * 4 * D, kBufferWord3);
  const uint32_t ape_off = static_cast<uint32_t>(grp * 4 * D + 4 * c0);
  auto load_ape = [&](int i0) -> float4 {  // row i0 + grp
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(ape_rsrc, ape_off, i0 * (4 * D), 0);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
  };
  if (split64 <= 0) {
    // Every row from the input, row i at t0 - split64 + i, loaded through a
    // buffer resource: uniform base, the lane's constant byte offset (its
    // row group's row, its channels), a uniform row offset.  Chunk c + 1's
    // kv rows are loaded (double-buffered) before chunk c is consumed, its
    // score and ape rows as soon as chunk c's gate values are formed (into
    // the same registers); the scheduling barriers keep the loads where they
    // are issued and keep the compiler from hoisting more.
    const uint32_t in_row = static_cast<uint32_t>(a.kvs_stride) * 2u;
    const __amdgpu_buffer_rsrc_t in_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.kv_score + (t0 - split64) * a.kvs_stride), 0, kSpan * in_row, kBufferWord3);
    const uint32_t kv_off = static_cast<uint32_t>(grp) * in_row + 2u * c0;
    const uint32_t sc_off = kv_off + 2u * D;
    auto load2 = [&](uint32_t off, int i0) -> uint2 {  // row i0 + grp
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(in_rsrc, off, i0 * in_row, 0);
      return make_uint2(v[0], v[1]);
    };
    constexpr int kSteps = kGroupRows / kChunk;  // chunks per row group
    uint2 sc[kChunk], kv[2][kChunk];
    float4 ap[kChunk];
    auto issue_kv = [&](int step, uint2 (&k_)[kChunk]) {
#pragma unroll
      for (int u = 0; u < kChunk; ++u) k_[u] = load2(kv_off, kRowGroups * (step * kChunk + u));
    };
    auto issue_gate = [&](int step) {
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        const int i0 = kRowGroups * (step * kChunk + u);
        sc[u] = load2(sc_off, i0);
        ap[u] = load_ape(i0);
      }
    };
    issue_kv(0, kv[0]);
    issue_gate(0);
#pragma unroll
    for (int step = 0; step < kSteps; ++step) {
      const int cur = step & 1;
      if (step + 1 < kSteps) issue_kv(step + 1, kv[cur ^ 1]);
      __builtin_amdgcn_sched_barrier(0);
      float g[kChunk][4];
      gate_chunk(sc, ap, g);
      __builtin_amdgcn_sched_barrier(0);
      if (step + 1 < kSteps) issue_gate(step + 1);  // into the score / ape registers just consumed
      __builtin_amdgcn_sched_barrier(0);
      if (step == 0) softmax_terms<true>(sm, g, kv[cur]);
      else softmax_terms<false>(sm, g, kv[cur]);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else if constexpr (kRingPipe) {
    // The span's first rows precede this call: rows i < split64 come from
    // the state ring, the others from the input.  Same arithmetic and the
    // same pipeline as above (next chunk's kv rows in flight while a chunk is
    // consumed, its score and ape rows issued once the gate values are
    // formed), with per-lane row addresses: lane bases of row group grp in
    // the ring (row i at ring + i * 2D) and in the input (row i at input +
    // (i - split) * stride); a row before the call without a ring reads the
    // call's first row and counts as 0.
    const int split = static_cast<int>(split64);
    const bool has_state = st >= 0 && st < a.num_state;
    const uint16_t* ring = (has_state ? a.state + (static_cast<int64_t>(st) * kStateRing + (j & 1) * kSpan) * (2 * D)
                                      : a.kv_score + t0 * a.kvs_stride - grp * (2 * D)) +
                           grp * (2 * D) + c0;
    const uint16_t* input = a.kv_score + (t0 - split + grp) * a.kvs_stride + c0;
    auto load_row = [&](int i0, int col) -> uint2 {  // row i0 + grp, channels col + c0 ..
      const bool from_ring = i0 + grp < split;
      const uint16_t* r = from_ring ? ring + (has_state ? i0 * (2 * D) : 0) : input + i0 * a.kvs_stride;
      const uint2 v = *reinterpret_cast<const uint2*>(r + col);
      return (from_ring && !has_state) ? make_uint2(0, 0) : v;
    };
    constexpr int kSteps = kGroupRows / kChunk;
    uint2 sc[kChunk], kv[2][kChunk];
    float4 ap[kChunk];
    auto issue_kv = [&](int step, uint2 (&k_)[kChunk]) {
#pragma unroll
      for (int u = 0; u < kChunk; ++u) k_[u] = load_row(kRowGroups * (step * kChunk + u), 0);
    };
    auto issue_gate = [&](int step) {
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        const int i0 = kRowGroups * (step * kChunk + u);
        sc[u] = load_row(i0, D);
        ap[u] = load_ape(i0);
      }
    };
    issue_kv(0, kv[0]);
    issue_gate(0);
#pragma unroll
    for (int step = 0; step < kSteps; ++step) {
      const int cur = step & 1;
      if (step + 1 < kSteps) issue_kv(step + 1, kv[cur ^ 1]);
      __builtin_amdgcn_sched_barrier(0);
      float g[kChunk][4];
      gate_chunk(sc, ap, g);
      __builtin_amdgcn_sched_barrier(0);
      if (step + 1 < kSteps) issue_gate(step + 1);
      __builtin_amdgcn_sched_barrier(0);
      if (step == 0) softmax_terms<true>(sm, g, kv[cur]);
      else softmax_terms<false>(sm, g, kv[cur]);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    // The span's first rows precede this call: rows i < split64 come from
    // the state ring.  Same arithmetic, plain per-row addressing.
    const int split = static_cast<int>(split64);
    const bool has_state = st >= 0 && st < a.num_state;
    auto load_row = [&](int i, int col) -> uint2 {
      const uint16_t* r;
      if (i >= split) r = a.kv_score + (t0 + (i - split)) * a.kvs_stride;
      else if (has_state) r = a.state + (static_cast<int64_t>(st) * kStateRing + (j & 1) * kSpan + i) * (2 * D);
      else return make_uint2(0, 0);
      return *reinterpret_cast<const uint2*>(r + col + c0);
    };
    for (int step = 0; step < kGroupRows / kChunk; ++step) {
      uint2 sc[kChunk], kv[kChunk];
      float4 ap[kChunk];
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        const int i0 = kRowGroups * (step * kChunk + u);
        sc[u] = load_row(i0 + grp, D);
        kv[u] = load_row(i0 + grp, 0);
        ap[u] = load_ape(i0);
      }
      float g[kChunk][4];
      gate_chunk(sc, ap, g);
      if (step == 0) softmax_terms<true>(sm, g, kv);
      else softmax_terms<false>(sm, g, kv);
    }
  }

  // Merge the 4 row groups in order (lanes l, l+16, l+32, l+48 of a wave).
  part = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float m_g[kRowGroups];
#pragma unroll
    for (int r = 0; r < kRowGroups; ++r) m_g[r] = __shfl(sm.m[k], (lane & 15) + 16 * r);
    float M = m_g[0];
#pragma unroll
    for (int r = 1; r < kRowGroups; ++r) M = fmaxf(M, m_g[r]);
    float Z = 0.0f, N = 0.0f;
#pragma unroll
    for (int r = 0; r < kRowGroups; ++r) {
      const float s = exp_ekv(m_g[r] - M);
      Z = __builtin_fmaf(__shfl(sm.Z[k], (lane & 15) + 16 * r), s, Z);
      N = __builtin_fmaf(__shfl(sm.N[k], (lane & 15) + 16 * r), s, N);
    }
    x[k] = __fdiv_rn(N, Z);
    part = part + x[k] * x[k];
  }
}

// Compress span j of sequence b (first row t0 at position p0, state slot st)
// with one workgroup of D threads.  Wave w owns channels 64w .. 64w+63;
// lane l of it owns the 4 channels 64w + 4 (l % 16) + 0..3 of row group
// l / 16 (span_softmax), then the row is finished: RMSNorm (the quads' sums
// of squares added in quad order by one thread), RoPE, quant.  Every thread
// of the workgroup must call it (it synchronizes).
template <int D, bool kRingPipe>
__device__ __forceinline__ void compress_span(const CompressArgs& a, CompressLds<D>& ls, int b, int t0, int64_t p0,
                                              int64_t j, int st) {
  constexpr int kWaves = D / 64;
  constexpr int kQuads = D / 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int grp = lane >> 4;                            // row group r
  const int quad = (tid >> 6) * 16 + (lane & 15);       // channel quad
  const int c0 = 4 * quad;
  float x[4], part;
  span_softmax<D, kRingPipe>(a, quad, t0, p0, j, st, x, part);
  // the row's page, requested before the norm
  const int64_t cpage = a.comp_bt[static_cast<int64_t>(b) * a.comp_bt_stride + j / kPageTokens];
  // From here on the lanes of row group 0 carry the row: quad q's channels.
  const bool owner = grp == 0;
  if (owner) ls.part[quad] = part;
  __syncthreads();
  if (tid == 0) {
    float S = 0.0f;
    for (int q = 0; q < kQuads; q += 4) {
      const float4 v = *reinterpret_cast<const float4*>(&ls.part[q]);
      S = S + v.x; S = S + v.y; S = S + v.z; S = S + v.w;
    }
    const float ms = __fdiv_rn(S, static_cast<float>(D));
    ls.rn = __fdiv_rn(1.0f, __fsqrt_rn(ms + a.eps));
  }
  __syncthreads();
  const float rn = ls.rn;
  const float4 w = *reinterpret_cast<const float4*>(a.norm_w + c0);
  float y[4] = {(x[0] * rn) * w.x, (x[1] * rn) * w.y, (x[2] * rn) * w.z, (x[3] * rn) * w.w};
  if (c0 >= D - 64) {
    const float* cs = a.cos_sin + j * 64;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int pi = (c0 - (D - 64)) / 2 + q;
      const float cz = cs[pi], sz = cs[32 + pi];
      const float x0 = y[2 * q], x1 = y[2 * q + 1];
      y[2 * q] = x0 * cz - x1 * sz;
      y[2 * q + 1] = x0 * sz + x1 * cz;
    }
  }
  float amax = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
  amax = wave_max_xor(amax, 64);  // the row-group copies are equal
  if (lane == 0) ls.wmax[tid >> 6] = amax;
  __syncthreads();
  amax = ls.wmax[0];
#pragma unroll
  for (int wv = 1; wv < kWaves; ++wv) amax = fmaxf(amax, ls.wmax[wv]);
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  const int64_t slot = cpage * kPageTokens + j % kPageTokens;
  if (slot < 0 || slot >= a.num_pages * kPageTokens) return;
  uint8_t* page = a.pool + (slot / kPageTokens) * a.page_stride;
  const int64_t off = slot % kPageTokens;
  if (a.bf16_rows) {
    if (owner) *reinterpret_cast<uint2*>(page + off * (2 * D) + 2 * c0) = bf16x4_pack(y[0], y[1], y[2], y[3]);
    return;
  }
  if (owner) {
    const uint32_t lo = f32x2_to_fp8(y[0] * inv, y[1] * inv);
    const uint32_t hi = f32x2_to_fp8(y[2] * inv, y[3] * inv);
    *reinterpret_cast<uint32_t*>(page + off * D + c0) = lo | (hi << 16);
  }
  if (tid == 0) *reinterpret_cast<float*>(page + kPageTokens * D + off * 4) = exp2i(e);
}

// compress_span split over D / 64 four-wave workgroups (decode-sized calls
// with a workspace, one slot per sequence): workgroup k takes channels
// [64 k, 64 k + 64), one per lane -- wave w channels 64 k + 16 w .. + 15,
// lane l of row group l / 16 -- so each lane runs one channel's online
// softmax over its group's 32 rows, and a span's work spreads over D / 64
// CUs.  It writes its softmax results and its channel quads' sums of squares
// to the workspace; the last of the span's workgroups to arrive reads all of
// them and finishes the row (finish_span_block).  Every operation on a
// channel, and the order of the sums, is compress_span's, so the bytes are
// too.  Every thread of the workgroup must call it (it synchronizes).
constexpr int kPartThreads = 256;

template <int D>
__device__ __forceinline__ void finish_span_block(const CompressArgs& a, CompressLds<D>& ls, int b, int64_t j);

template <int D>
__device__ __forceinline__ void compress_span_part(const CompressArgs& a, CompressLds<D>& ls, int b, int k, int t0,
                                                   int64_t p0, int64_t j, int st) {
  constexpr int kParts = D / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int grp = lane >> 4;
  const int c = 64 * k + 16 * wave + (lane & 15);  // this lane's channel

  // Row i = i0 + grp of the span: the state ring's row (j % 2) * 128 + i
  // for i < split, else the call's input row i - split.  Both come through
  // buffer resources, so a row is two unconditional loads whose
  // out-of-range offsets read 0 (an input offset below the call's first
  // row wraps past its end; without a ring the ring resource is empty, and
  // such rows count as 0), and the lane keeps one of the two.
  const int64_t split64 = p0 - j * kSpan;
  const int split = static_cast<int>(split64 < 0 ? 0 : split64);
  const bool has_state = st >= 0 && st < a.num_state;
  const uint32_t in_row = static_cast<uint32_t>(a.kvs_stride) * 2u;
  // (uniform values: the resources must live in scalar registers)
  const uint32_t n_in = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(a.qsl[b + 1] - t0));
  const __amdgpu_buffer_rsrc_t in_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.kv_score + static_cast<int64_t>(t0) * a.kvs_stride), 0, n_in * in_row, kBufferWord3);
  const __amdgpu_buffer_rsrc_t ring_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      has_state ? const_cast<uint16_t*>(a.state + (static_cast<int64_t>(st) * kStateRing + (j & 1) * kSpan) * (2 * D))
                : const_cast<uint16_t*>(a.kv_score),
      0, has_state ? kSpan * 2 * D * 2 : 0, kBufferWord3);
  const uint32_t ring_lane = static_cast<uint32_t>((grp * 2 * D + c) * 2);
  const uint32_t in_lane = static_cast<uint32_t>(grp) * in_row + static_cast<uint32_t>(c) * 2u;
  auto ring_off = [&](int i0, int col) { return ring_lane + (i0 * 2 * D + col) * 2; };
  auto in_off = [&](int i0, int col) {
    return in_lane + static_cast<uint32_t>((i0 - split) * static_cast<int>(in_row)) + col * 2;
  };
  const float* ape = a.ape + grp * D + c;
  // The lane's 32 rows in two halves: every load of a half is issued
  // before any of it is used (two memory latencies for the span part
  // instead of one per chunk, in half the registers of one batch), and the
  // chunks are folded in order as before.
  constexpr int kHalf = kGroupRows / 2;
  float m = -INFINITY, Z = 0.0f, N = 0.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t kr[kHalf], ki[kHalf], sr[kHalf], si[kHalf];
    float ap[kHalf];
#pragma unroll
    for (int q = 0; q < kHalf; ++q) {
      const int i0 = kRowGroups * (h * kHalf + q);
      kr[q] = __builtin_amdgcn_raw_buffer_load_b16(ring_rsrc, ring_off(i0, 0), 0, 0);
      ki[q] = __builtin_amdgcn_raw_buffer_load_b16(in_rsrc, in_off(i0, 0), 0, 0);
      sr[q] = __builtin_amdgcn_raw_buffer_load_b16(ring_rsrc, ring_off(i0, D), 0, 0);
      si[q] = __builtin_amdgcn_raw_buffer_load_b16(in_rsrc, in_off(i0, D), 0, 0);
      ap[q] = ape[i0 * D];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < kHalf / kChunk; ++st) {
      const int step = h * (kHalf / kChunk) + st;
      float g[kChunk], kv[kChunk];
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        const int q = st * kChunk + u;
        const bool from_ring = kRowGroups * (h * kHalf + q) + grp < split;
        g[u] = __uint_as_float((from_ring ? sr[q] : si[q]) << 16) + ap[q];
        kv[u] = __uint_as_float((from_ring ? kr[q] : ki[q]) << 16);
      }
      if (step == 0) softmax_terms1<true>(m, Z, N, g, kv);
      else softmax_terms1<false>(m, Z, N, g, kv);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // Merge the 4 row groups in order (lanes l, l+16, l+32, l+48).
  float m_g[kRowGroups];
#pragma unroll
  for (int r = 0; r < kRowGroups; ++r) m_g[r] = __shfl(m, (lane & 15) + 16 * r);
  float M = m_g[0];
#pragma unroll
  for (int r = 1; r < kRowGroups; ++r) M = fmaxf(M, m_g[r]);
  float Zs = 0.0f, Ns = 0.0f;
#pragma unroll
  for (int r = 0; r < kRowGroups; ++r) {
    const float s = exp_ekv(m_g[r] - M);
    Zs = __builtin_fmaf(__shfl(Z, (lane & 15) + 16 * r), s, Zs);
    Ns = __builtin_fmaf(__shfl(N, (lane & 15) + 16 * r), s, Ns);
  }
  const float x = __fdiv_rn(Ns, Zs);
  // the quad's sum of squares, channel 4q first (lanes 4q' .. 4q'+3 hold it)
  const float x1 = __shfl_down(x, 1), x2 = __shfl_down(x, 2), x3 = __shfl_down(x, 3);
  float part = 0.0f;
  part = part + x * x;
  part = part + x1 * x1;
  part = part + x2 * x2;
  part = part + x3 * x3;
  if (grp == 0) {
    __hip_atomic_store(a.span_x + static_cast<int64_t>(b) * D + c, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((c & 3) == 0)
      __hip_atomic_store(a.span_part + static_cast<int64_t>(b) * (D / 4) + c / 4, part, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  handoff_wait();  // this workgroup's results are complete before it arrives (as in compress_span_slab)
  __syncthreads();
  if (tid == 0) {
    const uint32_t before = __hip_atomic_fetch_add(a.span_count + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ls.last = (before + 1u == static_cast<uint32_t>(kParts)) ? 1 : 0;
  }
  __syncthreads();
  if (!ls.last) return;
  compiler_fence();
  finish_span_block<D>(a, ls, b, j);
}

// The row of span j of sequence b (workspace slot b) from the softmax
// results and quad sums in the workspace, finished by the kPartThreads
// threads of the last workgroup to arrive as compress_span finishes it:
// RMSNorm with the quad sums added in quad order by thread 0, RoPE on the
// last 64 channels, the per-token quant.  Thread tid takes channels
// tid + kPartThreads i.  Clears the slot's arrival counter.
template <int D>
__device__ __forceinline__ void finish_span_block(const CompressArgs& a, CompressLds<D>& ls, int b, int64_t j) {
  constexpr int kPer = (D + kPartThreads - 1) / kPartThreads;
  constexpr int kWaves = kPartThreads / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  if (tid == 0) __hip_atomic_store(a.span_count + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the norm weights and the RoPE table entries of this thread's channels
  // are loaded with the workspace reads, not after the norm
  float xc[kPer], wc[kPer], cz[kPer], sz[kPer];
  const int64_t cpage = a.comp_bt[static_cast<int64_t>(b) * a.comp_bt_stride + j / kPageTokens];  // the row's page
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = tid + kPartThreads * i;
    const bool rope = c >= D - 64 && c < D;
    const int pi = rope ? (c - (D - 64)) / 2 : 0;
    xc[i] = c < D ? __hip_atomic_load(a.span_x + static_cast<int64_t>(b) * D + c, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT)
                  : 0.0f;
    wc[i] = c < D ? a.norm_w[c] : 0.0f;
    cz[i] = rope ? a.cos_sin[j * 64 + pi] : 0.0f;
    sz[i] = rope ? a.cos_sin[j * 64 + 32 + pi] : 0.0f;
  }
  if (tid < D / 4)
    ls.part[tid] = __hip_atomic_load(a.span_part + static_cast<int64_t>(b) * (D / 4) + tid, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (tid == 0) {
    float S = 0.0f;
    for (int q = 0; q < D / 4; q += 4) {
      const float4 v = *reinterpret_cast<const float4*>(&ls.part[q]);
      S = S + v.x; S = S + v.y; S = S + v.z; S = S + v.w;
    }
    const float ms = __fdiv_rn(S, static_cast<float>(D));
    ls.rn = __fdiv_rn(1.0f, __fsqrt_rn(ms + a.eps));
  }
  __syncthreads();
  const float rn = ls.rn;
  float y[kPer];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = tid + kPartThreads * i;
    float v = c < D ? (xc[i] * rn) * wc[i] : 0.0f;
    const float vp = __shfl_xor(v, 1);  // the RoPE pair (channels 2i, 2i+1)
    if (c >= D - 64 && c < D) {
      const float x0 = (c & 1) ? vp : v, x1v = (c & 1) ? v : vp;
      v = (c & 1) ? x0 * sz[i] + x1v * cz[i] : x0 * cz[i] - x1v * sz[i];
    }
    y[i] = v;
    amax = fmaxf(amax, fabsf(v));
  }
  amax = wave_max_xor(amax, 64);
  if (lane == 0) ls.wmax[wave] = amax;
  __syncthreads();
  amax = ls.wmax[0];
#pragma unroll
  for (int wv = 1; wv < kWaves; ++wv) amax = fmaxf(amax, ls.wmax[wv]);
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  const int64_t cslot = cpage * kPageTokens + j % kPageTokens;
  if (cslot < 0 || cslot >= a.num_pages * kPageTokens) return;
  uint8_t* page = a.pool + (cslot / kPageTokens) * a.page_stride;
  const int64_t off = cslot % kPageTokens;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = tid + kPartThreads * i;
    const float y1 = __shfl_down(y[i], 1), y2 = __shfl_down(y[i], 2), y3 = __shfl_down(y[i], 3);
    if (c >= D || (c & 3) != 0) continue;
    if (a.bf16_rows) {
      *reinterpret_cast<uint2*>(page + off * (2 * D) + 2 * c) = bf16x4_pack(y[i], y1, y2, y3);
    } else {
      const uint32_t lo = f32x2_to_fp8(y[i] * inv, y1 * inv);
      const uint32_t hi = f32x2_to_fp8(y2 * inv, y3 * inv);
      *reinterpret_cast<uint32_t*>(page + off * D + c) = lo | (hi << 16);
    }
  }
  if (tid == 0 && !a.bf16_rows) *reinterpret_cast<float*>(page + kPageTokens * D + off * 4) = exp2i(e);
}

// The row of span j (workspace slot `slot`, compressed slot through
// sequence b's comp_block_table row) from the softmax results and quad sums
// in the workspace, finished by one wave as compress_span finishes it:
// RMSNorm with the quad sums added in quad order by lane 0, RoPE on the last
// 64 channels, the per-token quant.  Lane l takes channels 64 i + l.  Clears
// the slot's arrival counter.  part_lds holds D / 4 floats.
template <int D>
__device__ __forceinline__ void finish_span_wave(const CompressArgs& a, float* part_lds, int64_t slot, int b,
                                                 int64_t j) {
  constexpr int kSlabs = D / 64;
  const int lane = threadIdx.x & 63;
  if (lane == 0) __hip_atomic_store(a.span_count + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float* sx = a.span_x + slot * D;
  const float* sp = a.span_part + slot * (D / 4);
  const int64_t cpage = a.comp_bt[static_cast<int64_t>(b) * a.comp_bt_stride + j / kPageTokens];  // the row's page
  for (int q = lane; q < D / 4; q += 64)
    part_lds[q] = __hip_atomic_load(sp + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float xs[kSlabs];
#pragma unroll
  for (int i = 0; i < kSlabs; ++i) xs[i] = __hip_atomic_load(sx + 64 * i + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  float rn = 0.0f;
  if (lane == 0) {
    float S = 0.0f;
    for (int q = 0; q < D / 4; q += 4) {
      const float4 v = *reinterpret_cast<const float4*>(&part_lds[q]);
      S = S + v.x; S = S + v.y; S = S + v.z; S = S + v.w;
    }
    const float ms = __fdiv_rn(S, static_cast<float>(D));
    rn = __fdiv_rn(1.0f, __fsqrt_rn(ms + a.eps));
  }
  rn = __shfl(rn, 0);
  float y[kSlabs];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kSlabs; ++i) {
    const int c = 64 * i + lane;
    float v = (xs[i] * rn) * a.norm_w[c];
    if (i == kSlabs - 1) {  // channels D - 64 .. D - 1: RoPE on the pairs (2i, 2i+1)
      const float vp = __shfl_xor(v, 1);
      const int pi = lane / 2;
      const float cz = a.cos_sin[j * 64 + pi], sz = a.cos_sin[j * 64 + 32 + pi];
      const float x0 = (lane & 1) ? vp : v, x1 = (lane & 1) ? v : vp;
      v = (lane & 1) ? x0 * sz + x1 * cz : x0 * cz - x1 * sz;
    }
    y[i] = v;
    amax = i == 0 ? fabsf(v) : fmaxf(amax, fabsf(v));
  }
  amax = wave_max_xor(amax, 64);
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  const int64_t cslot = cpage * kPageTokens + j % kPageTokens;
  if (cslot < 0 || cslot >= a.num_pages * kPageTokens) return;
  uint8_t* page = a.pool + (cslot / kPageTokens) * a.page_stride;
  const int64_t off = cslot % kPageTokens;
#pragma unroll
  for (int i = 0; i < kSlabs; ++i) {
    const float y1 = __shfl_down(y[i], 1), y2 = __shfl_down(y[i], 2), y3 = __shfl_down(y[i], 3);
    if (a.bf16_rows) {
      if ((lane & 3) == 0)
        *reinterpret_cast<uint2*>(page + off * (2 * D) + 2 * (64 * i + lane)) = bf16x4_pack(y[i], y1, y2, y3);
      continue;
    }
    if ((lane & 3) == 0) {
      const uint32_t lo = f32x2_to_fp8(y[i] * inv, y1 * inv);
      const uint32_t hi = f32x2_to_fp8(y2 * inv, y3 * inv);
      *reinterpret_cast<uint32_t*>(page + off * D + 64 * i + lane) = lo | (hi << 16);
    }
  }
  if (lane == 0 && !a.bf16_rows) *reinterpret_cast<float*>(page + kPageTokens * D + off * 4) = exp2i(e);
}

// Span j of sequence b compressed by D / 64 one-wave workgroups (prefill
// calls with a workspace): workgroup `slab` runs compress_span's wave `slab`
// -- channels 64 slab .. 64 slab + 63, 4 per lane of row group lane / 16 --
// and writes its softmax results and quad sums to workspace slot `slot`; the
// last of the span's workgroups to arrive finishes the row (finish_span_wave).
// The operations on a channel and the order of the sums are compress_span's,
// so the bytes are too.  Spans that start in the state ring take the plain
// per-row path (one per sequence at most).
template <int D>
__device__ __forceinline__ void compress_span_slab(const CompressArgs& a, float* part_lds, int64_t slot, int b,
                                                   int slab, int t0, int64_t p0, int64_t j, int st) {
  const int lane = threadIdx.x & 63;
  const int quad = 16 * slab + (lane & 15);
  float x[4], part;
  span_softmax<D, false>(a, quad, t0, p0, j, st, x, part);
  if (lane < 16) {
    float* sx = a.span_x + slot * D + 4 * quad;
#pragma unroll
    for (int k = 0; k < 4; ++k) __hip_atomic_store(sx + k, x[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.span_part + slot * (D / 4) + quad, part, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // This wave's results are complete (agent-coherent stores) before it
  // arrives; the last arriver's loads are agent-coherent and issued after its
  // add returns.  No acquire / release: their L2 write-back and invalidate on
  // every arrival would cost more than the span.
  handoff_wait();
  uint32_t before = 0;
  if (lane == 0) before = __hip_atomic_fetch_add(a.span_count + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  before = __shfl(before, 0);
  if (before + 1u != static_cast<uint32_t>(D / 64)) return;
  compiler_fence();
  finish_span_wave<D>(a, part_lds, slot, b, j);
}

// One one-wave workgroup per (channel slab, span slot, sequence), slab
// fastest: span slot x of sequence b is span p0 / 128 + x, compressed when
// this call completes it, into workspace slot b * slots + x.
template <int D>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(5)))
hca_compress_slab_kernel(CompressArgs a, int slots) {
  __shared__ __align__(16) float part_lds[D / 4];
  constexpr int kSlabs = D / 64;
  const int span_id = static_cast<int>(blockIdx.x) / kSlabs;
  const int slab = static_cast<int>(blockIdx.x) - span_id * kSlabs;
  const int b = span_id / slots;
  const int t0 = a.qsl[b];
  const int n = a.qsl[b + 1] - t0;
  if (n <= 0) return;
  const int64_t p0 = a.positions[t0];
  const int64_t j = p0 / kSpan + (span_id - b * slots);
  if (j * kSpan + kSpan - 1 > p0 + n - 1) return;  // span not completed by this call
  if (j >= a.max_spans) return;
  compress_span_slab<D>(a, part_lds, span_id, b, slab, t0, p0, j, a.state_slot != nullptr ? a.state_slot[b] : -1);
}

// One workgroup per (span slot, sequence): span p0 / 128 + blockIdx.x of
// sequence blockIdx.y, when this call completes it.
template <int D>
__global__ void __launch_bounds__(D) __attribute__((amdgpu_waves_per_eu(5))) hca_compress_kernel(CompressArgs a) {
  __shared__ CompressLds<D> ls;
  const int b = blockIdx.y;
  const int t0 = a.qsl[b];
  const int n = a.qsl[b + 1] - t0;
  if (n <= 0) return;
  const int64_t p0 = a.positions[t0];
  const int64_t j = p0 / kSpan + blockIdx.x;
  if (j * kSpan + kSpan - 1 > p0 + n - 1) return;  // span not completed by this call
  if (j >= a.max_spans) return;
  compress_span<D, false>(a, ls, b, t0, p0, j, a.state_slot != nullptr ? a.state_slot[b] : -1);
}

// Decode-sized HCA write (fewer than 128 new rows per sequence, so at most
// one span per sequence completes: the one holding its first new position)
// in one launch: the first workgroups compress that span when the call
// completes it, the rest run the append grid's blocks and then the index
// rows' blocks on their first 4 waves.  The two touch disjoint memory: the
// compressor reads this call's inputs and state-ring rows of positions
// before the call, the append writes this call's positions (rows, window
// ring, state ring), the index rows only read tables.  Every span such a
// call compresses starts in the state ring (all but its last rows precede
// the call), so the ring path is pipelined here.
//
// Without a workspace: one D-thread workgroup per sequence (compress_span).
template <int D>
__global__ void __launch_bounds__(D) __attribute__((amdgpu_waves_per_eu(4)))
hca_write_small_kernel(CompressArgs c, AppendArgs a, int num_seqs, int main_blocks, int tail_rows,
                       HcaIndexArgs ix, int append_blocks, int index_y) {
  __shared__ CompressLds<D> ls;
  const int block = static_cast<int>(blockIdx.x);
  if (block < num_seqs) {
    const int t0 = c.qsl[block];
    const int n = c.qsl[block + 1] - t0;
    if (n <= 0) return;
    const int64_t p0 = c.positions[t0];
    const int64_t j = p0 / kSpan;
    if (j * kSpan + kSpan - 1 > p0 + n - 1 || j >= c.max_spans) return;  // no span completed by this call
    compress_span<D, true>(c, ls, block, t0, p0, j, c.state_slot != nullptr ? c.state_slot[block] : -1);
    return;
  }
  if (threadIdx.x >= 256) return;  // the append's and index rows' blocks are 4-wave, with no workgroup barrier
  const int ab = block - num_seqs;
  if (ab < append_blocks) {
    hca_append_block<D>(a, ab, main_blocks, tail_rows);
    return;
  }
  const int ib = ab - append_blocks;  // index rows (the step's decode reads them after this launch)
  hca_index_block(ix, ib / index_y, ib % index_y);
}

// With a workspace (a slot per sequence): every block is 4 waves; a span is
// compressed by D / 64 of them (compress_span_part), so the compressor's
// arithmetic spreads over as many CUs.
template <int D>
__global__ void __launch_bounds__(kPartThreads)
hca_write_small_ws_kernel(CompressArgs c, AppendArgs a, int num_seqs, int main_blocks, int tail_rows,
                          HcaIndexArgs ix, int append_blocks, int index_y) {
  __shared__ CompressLds<D> ls;
  constexpr int kParts = D / 64;
  const int block = static_cast<int>(blockIdx.x);
  if (block < kParts * num_seqs) {
    const int seq = block / kParts;
    const int t0 = c.qsl[seq];
    const int n = c.qsl[seq + 1] - t0;
    if (n <= 0) return;
    const int64_t p0 = c.positions[t0];
    const int64_t j = p0 / kSpan;
    if (j * kSpan + kSpan - 1 > p0 + n - 1 || j >= c.max_spans) return;  // no span completed by this call
    const int st = c.state_slot != nullptr ? c.state_slot[seq] : -1;
    compress_span_part<D>(c, ls, seq, block - seq * kParts, t0, p0, j, st);
    return;
  }
  const int ab = block - kParts * num_seqs;
  if (ab < append_blocks) {
    hca_append_block<D>(a, ab, main_blocks, tail_rows);
    return;
  }
  const int ib = ab - append_blocks;  // index rows (the step's decode reads them after this launch)
  hca_index_block(ix, ib / index_y, ib % index_y);
}

}  // namespace ekv

using namespace ekv;

namespace {

// Argument checks and CompressArgs of an HCA compress; 0 or an error status.
int hca_compress_args(CompressArgs& a, const uint16_t* kv_score, int64_t kvs_stride, const int64_t* positions,
                      const int32_t* qsl, int32_t dim, const uint16_t* state, const int32_t* state_slot,
                      int32_t num_state, const float* ape, const float* norm_w, float eps, const float* cos_sin,
                      int32_t max_spans, const int32_t* comp_block_table, int32_t comp_bt_stride, uint8_t* pool,
                      int64_t page_stride, int64_t num_pages, bool bf16_rows = false) {
  EKV_CHECK(dim == 512 || dim == 576, "HCA dim must be 512 or 576");
  EKV_CHECK(kv_score && positions && qsl && ape && norm_w && cos_sin && comp_block_table && pool,
            "null pointer");
  EKV_CHECK(kvs_stride >= 2 * dim && kvs_stride % 4 == 0 && kvs_stride <= (int64_t{1} << 22),
            "kv_score stride must be in [2*dim, 2^22], a multiple of 4");
  EKV_CHECK(page_stride >= kPageTokens * (bf16_rows ? 2 * dim : dim + 4) && page_stride % 16 == 0,
            "bad page_stride");
  EKV_CHECK(aligned16(ape) && aligned16(norm_w) && aligned8(kv_score) && aligned16(pool) &&
                (state == nullptr || aligned8(state)),
            "misaligned buffers");
  a = CompressArgs{kv_score, kvs_stride, positions, qsl, state, state_slot, num_state, ape, norm_w, eps,
                   cos_sin, max_spans, comp_block_table, comp_bt_stride, pool, page_stride, num_pages,
                   nullptr, nullptr, nullptr, bf16_rows ? 1 : 0};
  return 0;
}

// ekv_hca_write workspace holding S spans: arrival counters u32 [S] (zero
// between calls), padded to 256 bytes | softmax results f32 [S, 576] | quad
// sums f32 [S, 144] (a span of width D uses the first D, D / 4 of its row).
// S is the most spans the byte size holds, so the layout depends on the size
// alone and one buffer serves calls of either width.
constexpr int64_t kWsWidth = 576;

int64_t hca_write_ws_bytes(int64_t spans) {
  return ((spans * 4 + 255) / 256) * 256 + spans * (kWsWidth + kWsWidth / 4) * 4;
}

int64_t hca_write_ws_capacity(int64_t bytes) {
  int64_t spans = bytes / (4 + (kWsWidth + kWsWidth / 4) * 4);
  while (spans > 0 && hca_write_ws_bytes(spans) > bytes) --spans;
  return spans;
}

}  // namespace

extern "C" int ekv_hca_compress(const uint16_t* kv_score, int64_t kvs_stride, const int64_t* positions,
                                const int32_t* qsl, int32_t num_seqs, int32_t max_query_len, int32_t dim,
                                const uint16_t* state, const int32_t* state_slot, int32_t num_state,
                                const float* ape, const float* norm_w, float eps, const float* cos_sin,
                                int32_t max_spans, const int32_t* comp_block_table, int32_t comp_bt_stride,
                                uint8_t* pool, int64_t page_stride, int64_t num_pages, void* stream) {
  EKV_CHECK(num_seqs >= 0 && max_query_len >= 0, "sizes must be >= 0");
  if (num_seqs == 0 || max_query_len == 0) return 0;
  CompressArgs a;
  const int rc = hca_compress_args(a, kv_score, kvs_stride, positions, qsl, dim, state, state_slot, num_state, ape,
                                   norm_w, eps, cos_sin, max_spans, comp_block_table, comp_bt_stride, pool,
                                   page_stride, num_pages);
  if (rc) return rc;
  // spans that can complete among max_query_len new positions
  const int spans = max_query_len / kSpan + 1;
  dim3 grid(spans, num_seqs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dim == 512) hipLaunchKernelGGL(hca_compress_kernel<512>, grid, dim3(512), 0, s, a);
  else hipLaunchKernelGGL(hca_compress_kernel<576>, grid, dim3(576), 0, s, a);
  return ekv_launch_status();
}

extern "C" int64_t ekv_hca_write_workspace_size(int32_t num_spans, int32_t dim) {
  return num_spans > 0 && dim > 0 && dim <= kWsWidth ? hca_write_ws_bytes(num_spans) : 0;
}

extern "C" int ekv_hca_decode_indices(const int64_t* positions, const int32_t* req_ids, int32_t num_tokens,
                                      const int32_t* comp_block_table, int32_t comp_bt_stride,
                                      const int32_t* ring_pages, int32_t ring_stride, int32_t ring,
                                      int32_t window, const int32_t* query_start_loc,
                                      const int64_t* slot_mapping, int32_t* out, int64_t out_stride,
                                      int32_t width, int32_t* lengths, void* stream);

namespace {

// ekv_hca_write, and with ix the step's decode index rows in the same launch
// (decode-sized calls) or right after it.
int hca_write_impl(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score, int64_t kvs_stride,
                   int32_t num_tokens, int32_t dim, const int64_t* slot_mapping, const int64_t* positions,
                   const int32_t* token_seq, const int32_t* qsl, int32_t num_seqs, int32_t max_query_len,
                   uint16_t* state, const int32_t* state_slot, int32_t num_state, const float* ape,
                   const float* norm_w, float eps, const float* cos_sin, int32_t max_spans,
                   const int32_t* comp_block_table, int32_t comp_bt_stride, const int32_t* ring_pages,
                   int32_t ring_stride, int32_t ring, uint8_t* pool, int64_t page_stride, int64_t num_pages,
                   void* workspace, int64_t workspace_bytes, const HcaIndexArgs* ix, void* stream,
                   bool bf16_rows = false) {
  EKV_CHECK(num_tokens >= 0 && num_seqs >= 0 && max_query_len >= 0, "sizes must be >= 0");
  if (num_tokens == 0 || num_seqs == 0) return 0;
  CompressArgs c;
  int rc = hca_compress_args(c, kv_score, kvs_stride, positions, qsl, dim, state, state_slot, num_state, ape,
                             norm_w, eps, cos_sin, max_spans, comp_block_table, comp_bt_stride, pool, page_stride,
                             num_pages, bf16_rows);
  if (rc) return rc;
  int64_t ws_spans = 0;
  if (workspace != nullptr) {
    ws_spans = hca_write_ws_capacity(workspace_bytes);
    EKV_CHECK(ws_spans >= num_seqs && aligned16(workspace),
              "workspace too small (ekv_hca_write_workspace_size) or misaligned");
    uint8_t* w = static_cast<uint8_t*>(workspace);
    c.span_count = reinterpret_cast<uint32_t*>(w);
    c.span_x = reinterpret_cast<float*>(w + ((ws_spans * 4 + 255) / 256) * 256);
    c.span_part = c.span_x + ws_spans * kWsWidth;
  }
  AppendArgs ap;
  rc = hca_append_args(ap, latent, latent_stride, kv_score, kvs_stride, num_tokens, dim, slot_mapping, positions,
                       token_seq, qsl, num_seqs, pool, page_stride, num_pages, ring_pages, ring_stride, ring, state,
                       state_slot, num_state, bf16_rows);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (max_query_len < kSpan) {  // decode-sized: compress, append (and index rows) in one launch
    int main_blocks = 0, tail_rows = 0;
    const int64_t compress_blocks = (c.span_count ? int64_t{dim / 64} : int64_t{1}) * num_seqs;
    const int64_t append_blocks = hca_append_grid(ap, dim, num_seqs, true, true, main_blocks, tail_rows);
    const int index_y = ix ? hca_index_blocks_per_row(ix->width) : 1;
    const int64_t index_blocks = ix ? int64_t{num_tokens} * index_y : 0;
    const int64_t blocks = compress_blocks + append_blocks + index_blocks;
    EKV_CHECK(blocks < (int64_t{1} << 31), "too many rows");
    const HcaIndexArgs none{};
    const HcaIndexArgs& ia = ix ? *ix : none;
    const dim3 grid(static_cast<uint32_t>(blocks));
    const int ab = static_cast<int>(append_blocks);
    if (c.span_count != nullptr) {
      if (dim == 512)
        hipLaunchKernelGGL(hca_write_small_ws_kernel<512>, grid, dim3(kPartThreads), 0, s, c, ap, num_seqs,
                           main_blocks, tail_rows, ia, ab, index_y);
      else
        hipLaunchKernelGGL(hca_write_small_ws_kernel<576>, grid, dim3(kPartThreads), 0, s, c, ap, num_seqs,
                           main_blocks, tail_rows, ia, ab, index_y);
    } else if (dim == 512) {
      hipLaunchKernelGGL(hca_write_small_kernel<512>, grid, dim3(512), 0, s, c, ap, num_seqs, main_blocks, tail_rows,
                         ia, ab, index_y);
    } else {
      hipLaunchKernelGGL(hca_write_small_kernel<576>, grid, dim3(576), 0, s, c, ap, num_seqs, main_blocks, tail_rows,
                         ia, ab, index_y);
    }
    return ekv_launch_status();
  }
  const int slots = max_query_len / kSpan + 1;  // spans that can complete per sequence
  if (c.span_count != nullptr && ws_spans >= int64_t{num_seqs} * slots) {
    // a workspace slot per (sequence, span slot): D / 64 one-wave workgroups per span
    const int64_t blocks = int64_t{num_seqs} * slots * (dim / 64);
    EKV_CHECK(blocks < (int64_t{1} << 31), "too many rows");
    const dim3 grid(static_cast<uint32_t>(blocks));
    if (dim == 512) hipLaunchKernelGGL(hca_compress_slab_kernel<512>, grid, dim3(64), 0, s, c, slots);
    else hipLaunchKernelGGL(hca_compress_slab_kernel<576>, grid, dim3(64), 0, s, c, slots);
  } else {
    const dim3 grid(slots, num_seqs);
    if (dim == 512) hipLaunchKernelGGL(hca_compress_kernel<512>, grid, dim3(512), 0, s, c);
    else hipLaunchKernelGGL(hca_compress_kernel<576>, grid, dim3(576), 0, s, c);
  }
  rc = ekv_launch_status();
  if (rc) return rc;
  rc = launch_hca_append(ap, dim, num_seqs, true, true, s);
  if (rc || ix == nullptr) return rc;
  return ekv_hca_decode_indices(ix->positions, ix->req_ids, num_tokens, ix->comp_bt, ix->comp_bt_stride,
                                ix->ring_pages, ix->ring_stride, ix->ring, ix->window, ix->qsl, ix->call_slots,
                                ix->out, ix->out_stride, ix->width, ix->lengths, stream);
}

}  // namespace

extern "C" int ekv_hca_write(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                             int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                             const int64_t* positions, const int32_t* token_seq, const int32_t* qsl,
                             int32_t num_seqs, int32_t max_query_len, uint16_t* state,
                             const int32_t* state_slot, int32_t num_state, const float* ape,
                             const float* norm_w, float eps, const float* cos_sin, int32_t max_spans,
                             const int32_t* comp_block_table, int32_t comp_bt_stride, const int32_t* ring_pages,
                             int32_t ring_stride, int32_t ring, uint8_t* pool, int64_t page_stride,
                             int64_t num_pages, void* workspace, int64_t workspace_bytes, void* stream) {
  return hca_write_impl(latent, latent_stride, kv_score, kvs_stride, num_tokens, dim, slot_mapping, positions,
                        token_seq, qsl, num_seqs, max_query_len, state, state_slot, num_state, ape, norm_w, eps,
                        cos_sin, max_spans, comp_block_table, comp_bt_stride, ring_pages, ring_stride, ring, pool,
                        page_stride, num_pages, workspace, workspace_bytes, nullptr, stream);
}

extern "C" int ekv_hca_write_step(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                                  int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                                  const int64_t* positions, const int32_t* token_seq, const int32_t* qsl,
                                  int32_t num_seqs, int32_t max_query_len, uint16_t* state,
                                  const int32_t* state_slot, int32_t num_state, const float* ape,
                                  const float* norm_w, float eps, const float* cos_sin, int32_t max_spans,
                                  const int32_t* comp_block_table, int32_t comp_bt_stride,
                                  const int32_t* ring_pages, int32_t ring_stride, int32_t ring, uint8_t* pool,
                                  int64_t page_stride, int64_t num_pages, void* workspace, int64_t workspace_bytes,
                                  int32_t window, int32_t* idx_out, int64_t idx_stride, int32_t width,
                                  int32_t* lengths, void* stream) {
  EKV_CHECK(num_tokens >= 0 && num_seqs >= 0, "sizes must be >= 0");
  if (num_tokens == 0 || num_seqs == 0) return 0;  // nothing to write, no index rows
  EKV_CHECK(ring_pages && idx_out && lengths, "null pointer");
  EKV_CHECK(ring >= window && window >= 0 && ring % kPageTokens == 0, "ring must be a multiple of 64 and >= window");
  EKV_CHECK(width >= 0 && idx_stride >= width, "idx_stride must be >= width >= 0");
  const HcaIndexArgs ix{positions, token_seq, comp_block_table, comp_bt_stride, ring_pages, ring_stride, ring,
                        window, qsl, slot_mapping, idx_out, idx_stride, width, lengths};
  return hca_write_impl(latent, latent_stride, kv_score, kvs_stride, num_tokens, dim, slot_mapping, positions,
                        token_seq, qsl, num_seqs, max_query_len, state, state_slot, num_state, ape, norm_w, eps,
                        cos_sin, max_spans, comp_block_table, comp_bt_stride, ring_pages, ring_stride, ring, pool,
                        page_stride, num_pages, workspace, workspace_bytes, &ix, stream);
}

extern "C" int ekv_hca_write_bf16(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                                  int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                                  const int64_t* positions, const int32_t* token_seq, const int32_t* qsl,
                                  int32_t num_seqs, int32_t max_query_len, uint16_t* state,
                                  const int32_t* state_slot, int32_t num_state, const float* ape,
                                  const float* norm_w, float eps, const float* cos_sin, int32_t max_spans,
                                  const int32_t* comp_block_table, int32_t comp_bt_stride,
                                  const int32_t* ring_pages, int32_t ring_stride, int32_t ring, uint16_t* pool,
                                  int64_t page_stride, int64_t num_pages, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  return hca_write_impl(latent, latent_stride, kv_score, kvs_stride, num_tokens, dim, slot_mapping, positions,
                        token_seq, qsl, num_seqs, max_query_len, state, state_slot, num_state, ape, norm_w, eps,
                        cos_sin, max_spans, comp_block_table, comp_bt_stride, ring_pages, ring_stride, ring,
                        reinterpret_cast<uint8_t*>(pool), page_stride, num_pages, workspace, workspace_bytes, nullptr,
                        stream, true);
}

extern "C" int ekv_hca_write_step_bf16(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                                       int64_t kvs_stride, int32_t num_tokens, int32_t dim,
                                       const int64_t* slot_mapping, const int64_t* positions,
                                       const int32_t* token_seq, const int32_t* qsl, int32_t num_seqs,
                                       int32_t max_query_len, uint16_t* state, const int32_t* state_slot,
                                       int32_t num_state, const float* ape, const float* norm_w, float eps,
                                       const float* cos_sin, int32_t max_spans, const int32_t* comp_block_table,
                                       int32_t comp_bt_stride, const int32_t* ring_pages, int32_t ring_stride,
                                       int32_t ring, uint16_t* pool, int64_t page_stride, int64_t num_pages,
                                       void* workspace, int64_t workspace_bytes, int32_t window, int32_t* idx_out,
                                       int64_t idx_stride, int32_t width, int32_t* lengths, void* stream) {
  EKV_CHECK(num_tokens >= 0 && num_seqs >= 0, "sizes must be >= 0");
  if (num_tokens == 0 || num_seqs == 0) return 0;  // nothing to write, no index rows
  EKV_CHECK(ring_pages && idx_out && lengths, "null pointer");
  EKV_CHECK(ring >= window && window >= 0 && ring % kPageTokens == 0, "ring must be a multiple of 64 and >= window");
  EKV_CHECK(width >= 0 && idx_stride >= width, "idx_stride must be >= width >= 0");
  const HcaIndexArgs ix{positions, token_seq, comp_block_table, comp_bt_stride, ring_pages, ring_stride, ring,
                        window, qsl, slot_mapping, idx_out, idx_stride, width, lengths};
  return hca_write_impl(latent, latent_stride, kv_score, kvs_stride, num_tokens, dim, slot_mapping, positions,
                        token_seq, qsl, num_seqs, max_query_len, state, state_slot, num_state, ape, norm_w, eps,
                        cos_sin, max_spans, comp_block_table, comp_bt_stride, ring_pages, ring_stride, ring,
                        reinterpret_cast<uint8_t*>(pool), page_stride, num_pages, workspace, workspace_bytes, &ix,
                        stream, true);
}
