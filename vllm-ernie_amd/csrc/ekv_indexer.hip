// Lightning-indexer scoring and exact top-k.
//
// Exact scores.  Every e4m3fn value is an integer I = value * 2**9 with
// |I| < 2**18, split into three signed base-64 digits (int8).  A head's dot
// product over the 128 dims is the exact int64
//
//   D = sum_{a,b} 64**(a+b) * sum_d qdigit_a[d] * kdigit_b[d]
//
// whose nine digit-pair sums run on v_mfma_i32_16x16x64_i8 (exact int32
// accumulation; partial sums stay below 2**21).  Then
//   dot = fl32(D * 2**-18), p_h = fl32(w_h * max(dot, 0)),
//   heads summed in fp32 in a fixed order (see exact_block),
//   score = fl32(acc * kscale) + 0.
// The CPU oracle evaluates the same formula, so scores -- and the top-k with
// its lowest-index tie-break -- are bit-exact.
//
// Fast top-k (ekv_indexer_filter + ekv_indexer_select): exact scoring costs
// nine int8 MFMAs per fp8 product, so it runs only on candidates.
//   1. filter:  fp8 MFMA (v_mfma_f32_16x16x128_f8f6f4) approximate score a_s
//      of every token, streamed at HBM rate, with an error bound
//      e_s = kscale_s * 448^2 * (2^-8 + 2^-9) * sum_h |w_h|.
//      Writes U_s = a_s + e_s (rounded up to bf16) and a per-row histogram of
//      the 12-bit key prefix of L_s = a_s - e_s; bound_kernel turns the
//      histogram into a key bound: the bin holding the k-th largest L.
//   2. verify: per 2048-token chunk, tokens with key(U_s) >= bound are the
//      candidates (any other token has k tokens whose exact score is strictly
//      larger); they are scored exactly into a per-chunk list.
//   3. select: the chunk lists, concatenated in order, go through an exact
//      radix select; output ascending, -1 padded.
// The filter's error term is eight times the largest fp8-MFMA error measured
// on the device (2^-10.95 of the largest product over 1M random and
// adversarial dot products; |q|, |k| <= 448 by the UE8M0 quantization), and
// 2^-9 covers the fp32 rounding of both head sums (each at most
// 66 * 2^-24 * 128 * 448^2 * sum_h |w_h| ~ 2^-11 * 448^2 * sum_h |w_h|; the
// filter adds each head's term w_h * max(dot_h, 0) with one fused
// multiply-add, the max taken on the bits: a float with its sign bit set
// becomes +0).
//
// MFMA layouts (A = 16 heads of a head block, B = 16 tokens):
//   i8 16x16x64:        lane l: row/col l%16, K bytes [16*(l/16), +16)
//   f8f6f4 16x16x128:   lane l: row/col l%16, K bytes [32*(l/16), +32)
//   C (both):           lane l: rows 4*(l/16)+i, column l%16
#include "ekv_common.h"
#include "ekv_internal.h"
#include "ekv_rows.h"

#include <algorithm>

namespace ekv {

constexpr int kIdxDim = 128;
constexpr int kIdxHeads = 64;
constexpr int kIdxPageBytes = kPageTokens * kIdxDim;  // scales follow the values
constexpr int kHistBits = 12;
constexpr int kHistBins = 1 << kHistBits;
constexpr int kChunk = 2048;  // verify chunk (tokens)

// ---------------------------------------------------------------------------
// Exact scoring helpers
// ---------------------------------------------------------------------------
struct ExactOperands {
  i32x4 qd[4][3][2];  // [head block][digit][K half]
  float wv[4][4];     // this lane's 16 head weights: heads 16hb + 4g + i
};

__device__ __forceinline__ void load_exact_operands(ExactOperands& op, const int8_t* q_digits, const float* w,
                                                    int64_t t, int g, int col) {
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int d = 0; d < 3; ++d)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const int8_t* src = q_digits + ((t * 3 + d) * kIdxHeads + 16 * hb + col) * kIdxDim + 64 * kh + 16 * g;
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        op.qd[hb][d][kh] = i32x4{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z),
                                 static_cast<int>(v.w)};
      }
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) op.wv[hb][i] = w[t * kIdxHeads + 16 * hb + 4 * g + i];
}

__device__ __forceinline__ uint32_t plane_word(uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3, int p) {
  const uint32_t sel = static_cast<uint32_t>(p) | (static_cast<uint32_t>(4 + p) << 8) | 0x0c0c0000u;
  const uint32_t x01 = __builtin_amdgcn_perm(e1, e0, sel);
  const uint32_t x23 = __builtin_amdgcn_perm(e3, e2, sel);
  return x01 | (x23 << 16);
}

// Loads key row s (this lane's 32 bytes: [16g, +16) of each 64-byte half) and
// its scale; zeros when the token has no page.
__device__ __forceinline__ void load_key_i8(const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                            const int32_t* bt, int64_t bt_stride, int64_t s, int g, uint4 kb[2],
                                            float& kscale) {
  kb[0] = make_uint4(0, 0, 0, 0);
  kb[1] = make_uint4(0, 0, 0, 0);
  kscale = 0.0f;
  if (s < 0 || (s >> 6) >= bt_stride) return;
  const int64_t page = bt[s >> 6];
  if (page < 0 || page >= num_pages) return;
  const uint8_t* base = kcache + page * page_stride;
  const int row = static_cast<int>(s & 63);
  kb[0] = *reinterpret_cast<const uint4*>(base + row * kIdxDim + 16 * g);
  kb[1] = *reinterpret_cast<const uint4*>(base + row * kIdxDim + 64 + 16 * g);
  kscale = *reinterpret_cast<const float*>(base + kIdxPageBytes + row * 4);
}

// Exact score of the 16 tokens of a block (token = lane % 16); every lane of
// the column returns the same value.  qd(hb, d, kh) yields this lane's q digit
// operand and wv its 16 head weights.  The head sum order is fixed: per lane
// hb = 0..3, i = 0..3 from +0, then (g0 + g1) + (g2 + g3) across lane groups.
// kStaged keeps each head block's operand reads inside its own schedule
// region (for operands read from LDS: 24 registers live instead of 96).
template <bool kStaged = false, class QDigits>
__device__ __forceinline__ float exact_block_with(QDigits qd, const float (&wv)[4][4], const uint32_t* s_table,
                                                  const uint4 kb[2], float kscale) {
  i32x4 kd[3][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    const uint32_t w4[4] = {kb[kh].x, kb[kh].y, kb[kh].z, kb[kh].w};
    uint32_t e[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) e[j] = s_table[(w4[j >> 2] >> (8 * (j & 3))) & 0xffu];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      kd[d][kh] = i32x4{static_cast<int>(plane_word(e[0], e[1], e[2], e[3], d)),
                        static_cast<int>(plane_word(e[4], e[5], e[6], e[7], d)),
                        static_cast<int>(plane_word(e[8], e[9], e[10], e[11], d)),
                        static_cast<int>(plane_word(e[12], e[13], e[14], e[15], d))};
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) {
    if (kStaged) __builtin_amdgcn_sched_barrier(0);
    i32x4 c[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) c[k] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int da = 0; da < 3; ++da)
#pragma unroll
      for (int db = 0; db < 3; ++db)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
          c[da + db] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd(hb, da, kh), kd[db][kh], c[da + db], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // D = lo + 2^12 c2 + 2^18 hi with lo = c0 + 64 c1, hi = c3 + 64 c4 (each
      // |c| < 2^21, so |lo|, |hi| < 2^27); the two fmas below are exact in
      // double (every partial result is an integer below 2^53), so dot is the
      // single rounding fl32(D * 2^-18).
      const int lo = c[0][i] + (c[1][i] << 6), hi = c[3][i] + (c[4][i] << 6);
      const double Dd = __builtin_fma(__builtin_fma(static_cast<double>(hi), 64.0, static_cast<double>(c[2][i])), 4096.0,
                                      static_cast<double>(lo));
      const float dot = static_cast<float>(Dd * 0x1p-18);
      const float r = fmaxf(dot, 0.0f);
      acc = acc + wv[hb][i] * r;
    }
  }
  const float a01 = acc + __shfl_xor(acc, 16);
  const float tot = a01 + __shfl_xor(a01, 32);
  return tot * kscale + 0.0f;
}

__device__ __forceinline__ float exact_block(const ExactOperands& op, const uint32_t* s_table, const uint4 kb[2],
                                             float kscale) {
  return exact_block_with([&](int hb, int d, int kh) { return op.qd[hb][d][kh]; }, op.wv, s_table, kb, kscale);
}

// ---------------------------------------------------------------------------
// MXFP4 keys (the use_fp4_kv indexer): 64 packed e2m1 bytes per token, then
// the four E8M0 scale bytes of every token of the page.  Exact scores, with
// I = 2 * e2m1 value (|I| <= 12) and sq, sk the scale bytes of block b (32
// dims):
//   D_b = sum_{d in b} Iq[h, d] * Ik[s, d]     (v_mfma_i32_16x16x32_i8, exact)
//   T_b = fl32(D_b * 2^(sq_b + sk_b - 256))    (exact in double, one rounding)
//   dot = ((T_0 + T_1) + T_2) + T_3            (fp32)
// then p_h = fl32(w_h * max(dot, 0)), the fp8 path's head-sum order and
// score = acc + 0 (no per-token factor).
// The filter runs all four blocks in one v_mfma_scale_f32_16x16x128_f8f6f4
// with both operands e2m1 and their E8M0 scales.  Each block sum is exact
// there (at most 32 * 36 in quarter units); adding the four scaled sums is
// aligned to the scales, so its error is bounded by M = sum_b 1152 *
// 2^(sq_b + sk_b - 254), the largest magnitude the scales allow, not by the
// actual block sums (a large-scale block that sums to zero still costs
// precision).  The error term
//   e_s = 1152 * 2^-16 * sum_b 2^(sk_b - 127) * sum_h |w_h| 2^(sq_hb - 127)
//       = 2^-16 * sum_h |w_h| M_h
// covers the MFMA (measured at most 2^-25.2 M on the device), the
// contract's three additions and the two head sums (2 * 18 * 2^-24 of
// sum_h |w_h| |dot_h| <= 2^-18.8 sum_h |w_h| M_h).
// Layouts: i8 16x16x32: lane l: row/col l%16, K bytes [8(l/16), +8) -- lane
// group g takes elements [8g, +8) of block b, the packed bytes
// [16b + 4g, +4) of a row; fp4 16x16x128: lane l: row/col l%16, K values
// [32(l/16), +32), the packed bytes [16g, +16) (block g), with block g's scale
// byte in the lane's scale operand.
// ---------------------------------------------------------------------------
constexpr int kFp4Row = 64;                           // packed bytes per key row
constexpr int kFp4PageBytes = kPageTokens * kFp4Row;  // scales follow the values
constexpr float kFp4BoundFactor = 1152.0f * 0x1p-16f;

struct Fp4Key {
  int64_t kq[4];  // block b: eight int8 values (elements 32b + 8g ...) of the lane's token
  uint32_t ks;    // the token's four scale bytes
};

// This lane's part of key row r of the page at `base` (zeros unless ok; the
// loads themselves are unconditional).
__device__ __forceinline__ void load_key_fp4(const uint8_t* base, int r, int g, bool ok, Fp4Key& key) {
  const uint8_t* row = base + r * kFp4Row + 4 * g;
  uint32_t w[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) w[b] = *reinterpret_cast<const uint32_t*>(row + 16 * b);
  const uint32_t s = *reinterpret_cast<const uint32_t*>(base + kFp4PageBytes + r * 4);
#pragma unroll
  for (int b = 0; b < 4; ++b) key.kq[b] = ok ? fp4x8_to_i8(w[b]) : int64_t{0};
  key.ks = ok ? s : 0u;
}

// q operand of head row (16 hb + col) for block b, as load_key_fp4 lays keys out.
__device__ __forceinline__ int64_t load_q_fp4(const uint8_t* q_values, int64_t t, int hb, int b, int g, int col) {
  const uint8_t* row = q_values + (t * kIdxHeads + 16 * hb + col) * kFp4Row;
  return fp4x8_to_i8(*reinterpret_cast<const uint32_t*>(row + 16 * b + 4 * g));
}

// Exact fp4 scores of the 16 tokens of a block (token = lane % 16); every lane
// of the column returns the same value.  qop(hb, b) yields this lane's q
// operand, qsc(h) the four scale bytes of head h.
template <bool kStaged = false, class QOp, class QSc>
__device__ __forceinline__ float exact_block_fp4(QOp qop, QSc qsc, const float (&wv)[4][4], const Fp4Key& key) {
  const int g = (threadIdx.x & 63) >> 4;
  float acc = 0.0f;
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) {
    if (kStaged) __builtin_amdgcn_sched_barrier(0);
    i32x4 c[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
      c[b] = __builtin_amdgcn_mfma_i32_16x16x32_i8(qop(hb, b), key.kq[b], i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t qs = qsc(16 * hb + 4 * g + i);
      float tb[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int e = static_cast<int>(((qs >> (8 * b)) & 0xffu) + ((key.ks >> (8 * b)) & 0xffu)) - 256;
        tb[b] = static_cast<float>(__builtin_ldexp(static_cast<double>(c[b][i]), e));
      }
      const float dot = ((tb[0] + tb[1]) + tb[2]) + tb[3];
      acc = acc + wv[hb][i] * fmaxf(dot, 0.0f);
    }
  }
  const float a01 = acc + __shfl_xor(acc, 16);
  const float tot = a01 + __shfl_xor(a01, 32);
  return tot + 0.0f;
}

// Exact-path operands of query row t in registers (fp4 keys).
struct Fp4Operands {
  int64_t q[4][4];  // [hb][block]
  float wv[4][4];
};

__device__ __forceinline__ void load_fp4_operands(Fp4Operands& op, const uint8_t* q_values, const float* w, int64_t t,
                                                  int g, int col) {
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int b = 0; b < 4; ++b) op.q[hb][b] = load_q_fp4(q_values, t, hb, b, g, col);
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) op.wv[hb][i] = w[t * kIdxHeads + 16 * hb + 4 * g + i];
}

// ---------------------------------------------------------------------------
// Exact scores of every token s < lengths[t] (ekv_indexer_score).
// ---------------------------------------------------------------------------
struct ScoreArgs {
  const int8_t* q_digits;    // [T, 3, 64, 128]
  const float* w;            // [T, 64] folded head weights
  const uint8_t* kcache;     // [num_pages, page_stride]
  int64_t page_stride;
  int64_t num_pages;
  const int32_t* block_table;  // [B, bt_stride]
  int64_t bt_stride;
  const int32_t* req_ids;    // [T]
  const int32_t* lengths;    // [T]
  float* scores;             // [T, scores_stride]
  int64_t scores_stride;
  int32_t max_len;
  const uint8_t* q_fp4;      // fp4 keys: q values [T, 64, 64] (q_digits unused)
  const int32_t* q_scales;   // fp4 keys: [T, 64], four E8M0 bytes per head
};

constexpr int kScoreIters = 8;                        // 16-token blocks per wave
constexpr int kScoreChunk = 4 * 16 * kScoreIters;     // tokens per workgroup

template <bool kFp4>
__global__ void __launch_bounds__(256) score_exact_kernel(ScoreArgs a) {
  __shared__ uint32_t s_table[256];  // fp8: digit table; fp4: q scale words
  const int tid = threadIdx.x;
  const int t = blockIdx.y;
  if constexpr (kFp4) {
    if (tid < kIdxHeads) s_table[tid] = static_cast<uint32_t>(a.q_scales[static_cast<int64_t>(t) * kIdxHeads + tid]);
  } else {
    s_table[tid] = fp8_digit_pack(static_cast<uint32_t>(tid));
  }
  const int n = min(a.lengths[t], a.max_len);
  __syncthreads();
  const int64_t chunk0 = static_cast<int64_t>(blockIdx.x) * kScoreChunk;
  if (chunk0 >= n) return;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;
  const int32_t* bt = a.block_table + static_cast<int64_t>(a.req_ids[t]) * a.bt_stride;
  if constexpr (kFp4) {
    Fp4Operands op;
    load_fp4_operands(op, a.q_fp4, a.w, t, g, col);
    for (int it = 0; it < kScoreIters; ++it) {
      const int64_t s = chunk0 + (static_cast<int64_t>(wave) * kScoreIters + it) * 16 + col;
      int64_t page = -1;
      if (s < n && (s >> 6) < a.bt_stride) page = bt[s >> 6];
      const bool ok = page >= 0 && page < a.num_pages;
      Fp4Key key;
      load_key_fp4(a.kcache + (ok ? page : 0) * a.page_stride, static_cast<int>(s & 63), g, ok, key);
      const float sc = exact_block_fp4([&](int hb, int b) { return op.q[hb][b]; },
                                       [&](int h) { return s_table[h]; }, op.wv, key);
      if (s < n && g == 0) a.scores[static_cast<int64_t>(t) * a.scores_stride + s] = sc;
    }
  } else {
    ExactOperands op;
    load_exact_operands(op, a.q_digits, a.w, t, g, col);
    for (int it = 0; it < kScoreIters; ++it) {
      const int64_t s = chunk0 + (static_cast<int64_t>(wave) * kScoreIters + it) * 16 + col;
      uint4 kb[2];
      float ks;
      load_key_i8(a.kcache, a.page_stride, a.num_pages, bt, a.bt_stride, s < n ? s : -1, g, kb, ks);
      const float sc = exact_block(op, s_table, kb, ks);
      if (s < n && g == 0) a.scores[static_cast<int64_t>(t) * a.scores_stride + s] = sc;
    }
  }
}

// ---------------------------------------------------------------------------
// Filter: approximate fp8-MFMA scores of every token with an error bound.
// Workgroup = (16 pages of one row); each wave streams 4 pages.
// ---------------------------------------------------------------------------
struct FilterArgs {
  const uint8_t* q_fp8;      // [T, 64, 128]
  const float* w;            // [T, 64]
  const uint8_t* kcache;
  int64_t page_stride;
  int64_t num_pages;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* req_ids;
  const int32_t* lengths;
  int32_t max_len;
  int32_t k;
  uint16_t* upper;           // [T, max_len] U_s rounded up to bf16
  uint32_t* hist;            // [T, kHistBins] counts of L_s key prefixes
  int32_t rows;              // T (filter_kernel: 1-D grid of groups x T workgroups)
  int32_t groups;            // workgroup slots per row, a multiple of 8
  const int32_t* q_scales;   // fp4 keys: [T, 64] E8M0 bytes (q_fp8 is then q values [T, 64, 64])
};


// max(x, 0) on the bits (x is a finite MFMA result): one integer max, where
// fmaxf also quiets a signalling NaN first.
__device__ __forceinline__ float relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// The filter's approximate dot products: 16 heads (A rows, q codes) x 16
// tokens (B columns, key codes) over the 128 dims on the fp8 MFMA, as
// e4m3fn values without scales.  Its error against the exact dot product is
// what the filter's bound e_s covers (ekv_indexer_filter_dots exposes it).
__device__ __forceinline__ f32x4 filter_mfma(const i32x8& q, const i32x8& k) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q, k, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
}

// The fp4 filter's dot products: both operands e2m1 (the first four words of
// each operand) with this lane's block scale byte in bits 0..7 of qs / ks.
__device__ __forceinline__ f32x4 filter_mfma_fp4(const i32x8& q, uint32_t qs, const i32x8& k, uint32_t ks) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(q, k, f32x4{0.f, 0.f, 0.f, 0.f}, 4, 4, 0,
                                                          static_cast<int>(qs), 0, static_cast<int>(ks));
}

// out[s][h] = the fp4 filter's MFMA dot product of q row h (q values [64, 64],
// q scales [64] words) and key row s (k values [N, 64], k scales [N] words).
__global__ void __launch_bounds__(64) filter_dots_fp4_kernel(const uint8_t* q, const int32_t* qs, const uint8_t* k,
                                                             const int32_t* ks, float* out) {
  const int lane = threadIdx.x, g = lane >> 4, col = lane & 15;
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * 16;
  auto load4 = [](const uint8_t* p) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    return i32x8{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w), 0, 0, 0, 0};
  };
  const i32x8 kv = load4(k + (s0 + col) * kFp4Row + 16 * g);
  const uint32_t kb = (static_cast<uint32_t>(ks[s0 + col]) >> (8 * g)) & 0xffu;
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) {
    const uint32_t qb = (static_cast<uint32_t>(qs[16 * hb + col]) >> (8 * g)) & 0xffu;
    const f32x4 cc = filter_mfma_fp4(load4(q + (16 * hb + col) * kFp4Row + 16 * g), qb, kv, kb);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(s0 + col) * kIdxHeads + 16 * hb + 4 * g + i] = cc[i];
  }
}

// out[s][h] = the filter's MFMA dot product of q row h and key row s (one
// wave per 16 keys; operands laid out as filter_stream loads them).
__global__ void __launch_bounds__(64) filter_dots_kernel(const uint8_t* q, const uint8_t* k, float* out) {
  const int lane = threadIdx.x, g = lane >> 4, col = lane & 15;
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * 16;
  auto load8 = [](const uint8_t* p) {
    const uint4 v0 = reinterpret_cast<const uint4*>(p)[0], v1 = reinterpret_cast<const uint4*>(p)[1];
    return i32x8{static_cast<int>(v0.x), static_cast<int>(v0.y), static_cast<int>(v0.z), static_cast<int>(v0.w),
                 static_cast<int>(v1.x), static_cast<int>(v1.y), static_cast<int>(v1.z), static_cast<int>(v1.w)};
  };
  const i32x8 kv = load8(k + (s0 + col) * kIdxDim + 32 * g);
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) {
    const f32x4 cc = filter_mfma(load8(q + (16 * hb + col) * kIdxDim + 32 * g), kv);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(s0 + col) * kIdxHeads + 16 * hb + 4 * g + i] = cc[i];
  }
}

// Block-wide exclusive prefix sum of an int; writes the block total.
template <int kThreads>
__device__ __forceinline__ int block_scan_excl(int v, int* s_wave, int& total) {
  constexpr int kWaves = kThreads / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = s_wave[w];
    before += (w < wave) ? c : 0;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return before + x - v;
}

// Bin b of an nb-bin histogram (nb <= 2 * kThreads) with
// (count above b) < remaining <= (count above b) + hist[b]; `above` gets the
// count above b.
template <int kThreads>
__device__ __forceinline__ int find_bin(const uint32_t* hist, int nb, int remaining, int* s_wave, int* s_res,
                                        int& above) {
  const int tid = threadIdx.x;
  const int r0 = 2 * tid, r1 = 2 * tid + 1;  // reversed order: bin = nb-1-r
  const int c0 = (r0 < nb) ? static_cast<int>(hist[nb - 1 - r0]) : 0;
  const int c1 = (r1 < nb) ? static_cast<int>(hist[nb - 1 - r1]) : 0;
  int total;
  const int excl = block_scan_excl<kThreads>(c0 + c1, s_wave, total);
  if (r0 < nb && excl < remaining && remaining <= excl + c0) { s_res[0] = nb - 1 - r0; s_res[1] = excl; }
  if (r1 < nb && excl + c0 < remaining && remaining <= excl + c0 + c1) {
    s_res[0] = nb - 1 - r1;
    s_res[1] = excl + c0;
  }
  __syncthreads();
  const int bin = s_res[0];
  above = s_res[1];
  __syncthreads();
  return bin;
}

// Pages of each wave: every row's 64-token pages are split into contiguous
// ranges of the same length, one per wave (4 waves per workgroup), so
// workgroup x of a row owns pages [4x, 4x + 4) * per_wave; per_wave is set by
// the batch's longest row over `groups` workgroups, so a longer row uses
// proportionally more workgroups and every wave streams about as many pages.
__host__ __device__ inline int filter_per_wave(int n, int groups) {
  const int npages = (n + kPageTokens - 1) / kPageTokens;
  return (npages + 4 * groups - 1) / (4 * groups);
}

// Filter operands of row t for this lane: the q rows in f8f6f4 A layout (fp8:
// 32 codes; fp4: 16 packed bytes of block g, and qsc[hb] = that block's scale
// byte of head 16hb + col), the 16 head weights wv[hb][i] = w[16hb + 4g + i]
// and the error-bound factors: fp8 eb[0] = 448^2 (2^-8 + 2^-9) sum_h |w_h|
// (times a token's kscale); fp4 eb[b] = 1152 * 2^-16 * sum_h |w_h|
// 2^(sq_hb - 127) (times 2^(sk_b - 127), summed over b).
struct FilterOps {
  i32x8 qa[4];
  uint32_t qsc[4];
  float wv[4][4];
  float eb[4];
};

// fp8 keys: the operands from one row's q codes q8[h * 128 + d] and folded
// weights w[h] (global memory, or the fused prologue's copy in LDS).
__device__ __forceinline__ void filter_operands_fp8(const uint8_t* q8, const float* w, int g, int col, FilterOps& op) {
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) {
    const uint4* src = reinterpret_cast<const uint4*>(q8 + (16 * hb + col) * kIdxDim + 32 * g);
    const uint4 v0 = src[0], v1 = src[1];
    op.qa[hb] = i32x8{static_cast<int>(v0.x), static_cast<int>(v0.y), static_cast<int>(v0.z), static_cast<int>(v0.w),
                      static_cast<int>(v1.x), static_cast<int>(v1.y), static_cast<int>(v1.z), static_cast<int>(v1.w)};
    op.qsc[hb] = 0u;
  }
  float wabs = 0.0f;
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float wi = w[16 * hb + 4 * g + i];
      op.wv[hb][i] = wi;
      wabs += fabsf(wi);
    }
  float ws = (col == 0) ? wabs : 0.0f;  // lanes 0, 16, 32, 48 hold all 64 heads between them
  for (int off = 32; off > 0; off >>= 1) ws += __shfl_xor(ws, off);
  op.eb[0] = ws * (448.0f * 448.0f * (0x1p-8f + 0x1p-9f));
  op.eb[1] = op.eb[2] = op.eb[3] = 0.0f;
}

template <bool kFp4>
__device__ __forceinline__ void load_filter_operands(const FilterArgs& a, int t, int g, int col, FilterOps& op) {
  const int64_t th = static_cast<int64_t>(t) * kIdxHeads;
  if constexpr (!kFp4) {
    filter_operands_fp8(a.q_fp8 + th * kIdxDim, a.w + th, g, col, op);
    return;
  }
#pragma unroll
  for (int hb = 0; hb < 4; ++hb) {
    const uint4 v = *reinterpret_cast<const uint4*>(a.q_fp8 + (th + 16 * hb + col) * kFp4Row + 16 * g);
    op.qa[hb] = i32x8{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w),
                      0, 0, 0, 0};
    op.qsc[hb] = (static_cast<uint32_t>(a.q_scales[th + 16 * hb + col]) >> (8 * g)) & 0xffu;
  }
  float wabs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float wi = a.w[th + 16 * hb + 4 * g + i];
      op.wv[hb][i] = wi;
      const uint32_t qs = static_cast<uint32_t>(a.q_scales[th + 16 * hb + 4 * g + i]);
#pragma unroll
      for (int b = 0; b < 4; ++b) wabs[b] += fabsf(wi) * e8m0_value((qs >> (8 * b)) & 0xffu);
    }
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    float ws = (col == 0) ? wabs[b] : 0.0f;  // lanes 0, 16, 32, 48 hold all 64 heads between them
    for (int off = 32; off > 0; off >>= 1) ws += __shfl_xor(ws, off);
    op.eb[b] = ws * kFp4BoundFactor;
  }
}

// The pages of a row a filter streams (its request `req`, the row of the
// block table, read by the caller before the row's length is known, so the
// two loads overlap): block-table entry of logical page
// lp (-1 outside [0, p_end), the table or the cache; unmapped pages load
// page 0, always present, and score 0), and one page's loads: this lane's 32
// bytes (fp4: 16) of each of the 4 blocks of 16 token rows, and the scale
// (fp4: four scale bytes) of row `lane` (one coalesced 256-byte load per
// page).  Loads are unconditional so the compiler keeps them in flight.
template <bool kFp4>
struct PageSource {
  const FilterArgs& a;
  const int32_t* bt;
  int p_end;
  __device__ PageSource(const FilterArgs& args, int32_t req, int end)
      : a(args), bt(args.block_table + static_cast<int64_t>(req) * args.bt_stride), p_end(end) {}
  __device__ int64_t page_of(int lp) const {
    const int64_t p = (lp < p_end && lp < a.bt_stride) ? static_cast<int64_t>(bt[lp]) : -1;
    return (p >= 0 && p < a.num_pages) ? p : -1;
  }
  __device__ void load(int64_t page, uint4 (&kb)[4][2], uint32_t& ks) const {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, col = lane & 15;
    const uint8_t* pbase = a.kcache + (page >= 0 ? page : 0) * a.page_stride;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int row = 16 * b + col;
      if constexpr (kFp4) {
        kb[b][0] = *reinterpret_cast<const uint4*>(pbase + row * kFp4Row + 16 * g);
        kb[b][1] = make_uint4(0, 0, 0, 0);
      } else {
        const uint4* src = reinterpret_cast<const uint4*>(pbase + row * kIdxDim + 32 * g);
        kb[b][0] = src[0];
        kb[b][1] = src[1];
      }
    }
    ks = *reinterpret_cast<const uint32_t*>(pbase + (kFp4 ? kFp4PageBytes : kIdxPageBytes) + lane * 4);
  }
};

// A wave's first page, loaded before the stream starts (by the caller, so
// its memory latency overlaps the caller's set-up).
struct FirstPage {
  uint4 kb[4][2];
  uint32_t ks;
  int64_t page;
};

// Streams logical pages of row t: `first`, then the pages next() returns (an
// increasing sequence; the stream ends at the first page >= p_end).  The next
// page's rows are in flight and the block-table entry of the one after that
// already read while a page is scored, so start-up latency is paid once per
// wave.  Per page, lane l gets the approximate score sc and error e of token
// 64 lp + l (sc = e = 0 on an unmapped page, whose exact scores are 0) and
// calls emit(lp, page, sc, e) with page = the block-table entry, or -1 when the
// page is unmapped; the lower bound sc - e of every token s < n goes into the
// LDS histogram.  With `pre`, page `first` has been loaded already (its
// rows and scale word in pre).
template <bool kFp4, class Next, class Emit>
__device__ __forceinline__ void filter_stream(const FilterArgs& a, int32_t req, int n, int first, int p_end, Next next,
                                              uint32_t* s_hist, const FilterOps& op, Emit emit,
                                              FirstPage* pre = nullptr) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, col = lane & 15;
  const PageSource<kFp4> src(a, req, p_end);
  auto page_of = [&](int lp) -> int64_t { return src.page_of(lp); };
  auto load_page = [&](int64_t page, uint4 (&kb)[4][2], uint32_t& ks) { src.load(page, kb, ks); };
  // One page scored: its 64 tokens' approximate scores and bounds into the
  // histogram and emit.
  auto score_page = [&](const uint4 (&kb)[4][2], uint32_t row_scale, int64_t page, int lp) {
    float mine = 0.0f;  // after the 4 blocks: approximate head sum of token `lane` of the page
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const i32x8 kv = i32x8{static_cast<int>(kb[b][0].x), static_cast<int>(kb[b][0].y), static_cast<int>(kb[b][0].z),
                             static_cast<int>(kb[b][0].w), static_cast<int>(kb[b][1].x), static_cast<int>(kb[b][1].y),
                             static_cast<int>(kb[b][1].z), static_cast<int>(kb[b][1].w)};
      // fp4: block g's scale byte of token 16b + col (page row 16b + col)
      const uint32_t kscb =
          kFp4 ? (static_cast<uint32_t>(__shfl(static_cast<int>(row_scale), 16 * b + col)) >> (8 * g)) & 0xffu : 0u;
      float acc = 0.0f;
#pragma unroll
      for (int hb = 0; hb < 4; ++hb) {
        const f32x4 cc = kFp4 ? filter_mfma_fp4(op.qa[hb], op.qsc[hb], kv, kscb) : filter_mfma(op.qa[hb], kv);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(op.wv[hb][i], relu_bits(cc[i]), acc);
      }
      acc += __shfl_xor(acc, 16);
      acc += __shfl_xor(acc, 32);
      if (g == b) mine = acc;  // block b's token col is page row 16b + col = this lane
    }
    const int64_t s = static_cast<int64_t>(lp) * kPageTokens + lane;
    float sc, e;
    if constexpr (kFp4) {
      float eb = 0.0f;
#pragma unroll
      for (int b = 0; b < 4; ++b) eb += op.eb[b] * e8m0_value((row_scale >> (8 * b)) & 0xffu);
      sc = page >= 0 ? mine : 0.0f;
      e = page >= 0 ? eb : 0.0f;
    } else {
      const float page_scale = page >= 0 ? __uint_as_float(row_scale) : 0.0f;
      sc = mine * page_scale;
      e = page_scale * op.eb[0];
    }
    if (s < n) atomicAdd(&s_hist[score_key((sc - e) + 0.0f) >> (32 - kHistBits)], 1u);
    emit(lp, page, sc, e);
  };
  // Two page buffers taken in turn (the next page loads into one while the
  // other is scored), so no page is copied between registers.
  uint4 buf_a[4][2], buf_b[4][2];
  uint32_t ks_a, ks_b;
  int lp = first;
  int lp1 = next();
  int64_t cur_page;
  if (pre != nullptr) {
    cur_page = pre->page;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      buf_a[b][0] = pre->kb[b][0];
      buf_a[b][1] = pre->kb[b][1];
    }
    ks_a = pre->ks;
  } else {
    cur_page = page_of(lp);
    load_page(cur_page, buf_a, ks_a);
  }
  int64_t page1 = page_of(lp1);
  for (;;) {
    if (lp >= p_end) break;
    {
      const int64_t page = cur_page;
      load_page(page1, buf_b, ks_b);  // in flight while this page is scored
      cur_page = page1;
      const int lp2 = next();
      page1 = page_of(lp2);
      score_page(buf_a, ks_a, page, lp);
      lp = lp1;
      lp1 = lp2;
    }
    if (lp >= p_end) break;
    {
      const int64_t page = cur_page;
      load_page(page1, buf_a, ks_a);
      cur_page = page1;
      const int lp2 = next();
      page1 = page_of(lp2);
      score_page(buf_b, ks_b, page, lp);
      lp = lp1;
      lp1 = lp2;
    }
  }
}

// 12-bit key prefix of the upper bound sc + e rounded up to bf16: a token is a
// candidate when this prefix reaches the bound bin.
__device__ __forceinline__ uint16_t upper_prefix(float sc, float e) {
  return static_cast<uint16_t>(score_key(bf16_to_f32(bf16_round_up(sc + e)) + 0.0f) >> (32 - kHistBits));
}

// Workgroup = (group x of row t), waves streaming the contiguous page ranges
// above.  Upper bounds are staged in LDS and written kFilterStage pages at a
// time: a store between two page loads would make the wait for the later load
// also wait for the store (vector memory counts retire in order).
constexpr int kFilterStage = 32;  // pages of upper bounds staged per wave

template <bool kFp4>
__global__ void __launch_bounds__(256) filter_kernel(FilterArgs a) {
  __shared__ uint32_t s_hist[kHistBins];
  __shared__ __align__(16) uint16_t s_up[4][kFilterStage * kPageTokens];
  __shared__ int s_maxn;
  const int tid = threadIdx.x;
  // Workgroup b runs on XCD b % 8 (round-robin dispatch).  Slot b / 8 of an
  // XCD takes segment x = 8 (slot / T) + (b % 8 + seq) % 8 of row t = slot % T
  // (seq its request): segments are spread over the XCDs, and the rows of one
  // segment of a sequence run back to back on one XCD, so its draft-token rows
  // read the same pages there at about the same time and share them through
  // its L2.  The rotation by sequence spreads the last, partly active groups
  // of segments of rows of equal length over the XCDs instead of piling them
  // on the first ones.
  const int b = static_cast<int>(blockIdx.x);
  const int slot = b >> 3;
  const int t = slot % a.rows;
  const int32_t req = a.req_ids[t];
  const int x = 8 * (slot / a.rows) + (((b & 7) + req) & 7);
  if (x >= a.groups) return;
  if (tid == 0) s_maxn = 0;
  __syncthreads();
  int mx = 0;
  for (int i = tid; i < a.rows; i += 256) mx = max(mx, min(a.lengths[i], a.max_len));
  for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
  if ((tid & 63) == 0) atomicMax(&s_maxn, mx);
  __syncthreads();
  const int n = min(a.lengths[t], a.max_len);
  const int npages = (n + kPageTokens - 1) / kPageTokens;
  const int per_wave = filter_per_wave(s_maxn, a.groups);
  if (4 * x * per_wave >= npages || n <= a.k) return;  // rows with n <= k need no filtering
  for (int i = tid; i < kHistBins; i += 256) s_hist[i] = 0;

  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;
  FilterOps op;
  load_filter_operands<kFp4>(a, t, g, col, op);
  __syncthreads();

  const int wr = __builtin_amdgcn_readfirstlane(4 * x + wave);  // wave of the row
  const int p_begin = min(wr * per_wave, npages), p_end = min(p_begin + per_wave, npages);
  uint16_t* up_row = a.upper + static_cast<int64_t>(t) * a.max_len;
  uint16_t* stage = s_up[wave];
  // Upper bounds of pages [first, first + count) of the stage to global
  // (coalesced 16-byte stores; element-wise at the end of the row).
  auto flush = [&](int first, int count) {
    const int64_t base = static_cast<int64_t>(first) * kPageTokens;
    const int elems = min(count * kPageTokens, n - static_cast<int>(base));
    const bool vec = (reinterpret_cast<uintptr_t>(up_row + base) & 15) == 0;
    for (int e = 8 * lane; e < elems; e += 8 * 64) {
      if (vec && e + 8 <= elems) {
        *reinterpret_cast<uint4*>(up_row + base + e) = *reinterpret_cast<const uint4*>(stage + e);
      } else {
        for (int j = e; j < min(e + 8, elems); ++j) up_row[base + j] = stage[j];
      }
    }
  };
  int staged = 0, stage_first = p_begin;
  int seq = p_begin;
  filter_stream<kFp4>(a, req, n, p_begin, p_end, [&] { return ++seq; }, s_hist, op,
                      [&](int lp, int64_t, float sc, float e) {
    stage[staged * kPageTokens + lane] = bf16_round_up(sc + e);
    if (++staged == kFilterStage) {  // wave-uniform
      __builtin_amdgcn_wave_barrier();
      flush(stage_first, staged);
      __builtin_amdgcn_wave_barrier();
      staged = 0;
      stage_first = lp + 1;
    }
  });
  if (staged > 0) {
    __builtin_amdgcn_wave_barrier();
    flush(stage_first, staged);
  }
  __syncthreads();
  uint32_t* gh = a.hist + static_cast<int64_t>(t) * kHistBins;
  for (int i = tid; i < kHistBins; i += 256) {
    const uint32_t v = s_hist[i];
    if (v) atomicAdd(&gh[i], v);
  }
}

// Candidate key bound of each row: the 12-bit bin holding the k-th largest
// lower bound (one 256-thread workgroup per row, after the filter).
__global__ void __launch_bounds__(256) bound_kernel(const uint32_t* hist, const int32_t* lengths, int32_t max_len,
                                                    int32_t k, uint32_t* kbound) {
  __shared__ int s_wave[4];
  __shared__ int s_res[2];
  const int tid = threadIdx.x, t = blockIdx.x;
  const int n = min(lengths[t], max_len);
  if (n <= k) return;  // unused: every token is selected
  const uint32_t* gh = hist + static_cast<int64_t>(t) * kHistBins;
  // 4096 bins, 16 per thread, scanned from the top bin down
  const int r0 = 16 * tid;
  int c[16];
  int sum = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    c[j] = static_cast<int>(gh[kHistBins - 1 - (r0 + j)]);
    sum += c[j];
  }
  int total;
  int excl = block_scan_excl<256>(sum, s_wave, total);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if (excl < k && k <= excl + c[j]) s_res[0] = kHistBins - 1 - (r0 + j);
    excl += c[j];
  }
  __syncthreads();
  if (tid == 0) kbound[t] = static_cast<uint32_t>(s_res[0]) << (32 - kHistBits);
}

__global__ void zero_u32_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

// ---------------------------------------------------------------------------
// Verify: candidates of a 2048-token chunk, scored exactly into the chunk's
// slice of the list buffers ([t][chunk0 ...]), count per chunk.
// ---------------------------------------------------------------------------
struct VerifyArgs {
  const int8_t* q_digits;
  const float* w;
  const uint8_t* kcache;
  int64_t page_stride;
  int64_t num_pages;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* req_ids;
  const int32_t* lengths;
  int32_t max_len;
  int32_t k;
  const uint16_t* upper;     // [T, max_len] bf16 upper bounds
  const uint32_t* kbound;    // [T]
  float* cand_score;         // [T, max_len] (chunk slices)
  int32_t* cand_idx;         // [T, max_len]
  int32_t* cand_count;       // [T, chunks]
  int32_t chunks;
  const uint8_t* q_fp4;      // fp4 keys: q values [T, 64, 64] (q_digits unused)
  const int32_t* q_scales;   // fp4 keys: [T, 64]
};

constexpr int kVerifyChunks = 4;  // chunks per verify workgroup
constexpr int kVerifyPages = kVerifyChunks * kChunk / kPageTokens;

template <bool kFp4>
__global__ void __launch_bounds__(256) verify_kernel(VerifyArgs a) {
  __shared__ uint32_t s_table[256];  // fp8: digit table; fp4: q scale words
  __shared__ int16_t s_list[kVerifyChunks * kChunk];  // candidate token offsets in the group, ascending
  __shared__ int16_t s_meta[kVerifyChunks * kChunk];  // chunk (bits 11..12) and position in its chunk list
  __shared__ int32_t s_pages[kVerifyPages];           // block-table entries of the group's pages
  __shared__ int s_wave[4];
  const int tid = threadIdx.x;
  const int t = blockIdx.y;
  if constexpr (kFp4) {
    if (tid < kIdxHeads) s_table[tid] = static_cast<uint32_t>(a.q_scales[static_cast<int64_t>(t) * kIdxHeads + tid]);
  } else {
    s_table[tid] = fp8_digit_pack(static_cast<uint32_t>(tid));
  }
  const int n = min(a.lengths[t], a.max_len);
  const int64_t row = static_cast<int64_t>(t) * a.max_len;
  const int c_begin = blockIdx.x * kVerifyChunks;
  int32_t* counts = a.cand_count + static_cast<int64_t>(t) * a.chunks;
  if (c_begin * kChunk >= n) {  // every chunk past the row's end: empty lists
    if (tid < kVerifyChunks && c_begin + tid < a.chunks) counts[c_begin + tid] = 0;
    return;
  }
  if (n <= a.k) {  // every token is selected: list them, no scores needed
    for (int c = c_begin; c < min(c_begin + kVerifyChunks, a.chunks); ++c) {
      const int chunk0 = c * kChunk;
      const int len = max(0, min(kChunk, n - chunk0));
      for (int i = tid; i < len; i += 256) a.cand_idx[row + chunk0 + i] = chunk0 + i;
      if (tid == 0) counts[c] = len;
    }
    return;
  }
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;
  // The q operands and the block-table entries of the group's pages are
  // independent of the candidate scan: in flight first.
  const int tok0 = c_begin * kChunk;  // first token of the group
  const int32_t* bt = a.block_table + static_cast<int64_t>(a.req_ids[t]) * a.bt_stride;
  if (tid < kVerifyPages) {
    const int64_t blk = (tok0 >> 6) + tid;
    s_pages[tid] = (blk < a.bt_stride) ? bt[blk] : -1;
  }
  // fp8: digit operands; fp4: packed-value operands (the other is unused)
  ExactOperands op;
  Fp4Operands op4;
  if constexpr (kFp4) {
    load_fp4_operands(op4, a.q_fp4, a.w, t, g, col);
  } else {
    load_exact_operands(op, a.q_digits, a.w, t, g, col);
  }
  // Candidates of each chunk (ascending), appended to one list.  The upper
  // bounds of all the workgroup's chunks are loaded before any is tested.
  const uint32_t kbound = a.kbound[t];
  constexpr int kPer = kChunk / 256;
  const int start = tid * kPer;
  uint4 ub[kVerifyChunks];
#pragma unroll
  for (int cc = 0; cc < kVerifyChunks; ++cc) {
    const int chunk0 = (c_begin + cc) * kChunk;
    const bool full = (row & 7) == 0 && chunk0 + start + kPer <= n;  // aligned and in bounds
    ub[cc] = full ? *reinterpret_cast<const uint4*>(a.upper + row + chunk0 + start) : make_uint4(0, 0, 0, 0);
    if (!full && chunk0 + start < n) {  // ragged tail of the row
      uint16_t tmp[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) tmp[j] = (chunk0 + start + j < n) ? a.upper[row + chunk0 + start + j] : 0;
      ub[cc] = *reinterpret_cast<const uint4*>(tmp);
    }
  }
  int total = 0;
#pragma unroll
  for (int cc = 0; cc < kVerifyChunks; ++cc) {
    const int c = c_begin + cc;
    const int chunk0 = c * kChunk;
    const int len = (c < a.chunks) ? max(0, min(kChunk, n - chunk0)) : 0;
    const uint32_t uw[4] = {ub[cc].x, ub[cc].y, ub[cc].z, ub[cc].w};
    uint32_t flags = 0;
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const uint16_t bits = static_cast<uint16_t>((uw[j >> 1] >> (16 * (j & 1))) & 0xffffu);
      if (start + j < len && score_key(bf16_to_f32(bits) + 0.0f) >= kbound) {
        flags |= 1u << j;
        ++cnt;
      }
    }
    int ctot;
    const int ex = block_scan_excl<256>(cnt, s_wave, ctot);
    int pos = total + ex, slot = ex;
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (flags & (1u << j)) {
        s_list[pos] = static_cast<int16_t>(chunk0 + start + j - tok0);
        s_meta[pos] = static_cast<int16_t>((cc << 11) | slot);
        ++pos;
        ++slot;
      }
    if (tid == 0 && c < a.chunks) counts[c] = ctot;
    total += ctot;
  }
  __syncthreads();
  if (total == 0) return;

  // Wave w scores blocks w, w+4, ... in batches of kVerifyBatch: the key rows
  // of a whole batch are loaded together (pages come from LDS).
  constexpr int kVerifyBatch = 4;
  for (int bb = wave * 16; bb < total; bb += 64 * kVerifyBatch) {
    int tok[kVerifyBatch];
    int64_t page[kVerifyBatch];
#pragma unroll
    for (int j = 0; j < kVerifyBatch; ++j) {
      const int li = bb + 64 * j + col;
      tok[j] = (li < total) ? s_list[li] : -1;  // offset in the group
      page[j] = (tok[j] >= 0) ? static_cast<int64_t>(s_pages[tok[j] >> 6]) : -1;
    }
    uint4 kb[kVerifyBatch][2];
    float ks[kVerifyBatch];
    Fp4Key k4[kFp4 ? kVerifyBatch : 1];
#pragma unroll
    for (int j = 0; j < kVerifyBatch; ++j) {
      const bool ok = page[j] >= 0 && page[j] < a.num_pages;
      const uint8_t* base = a.kcache + (ok ? page[j] : 0) * a.page_stride;
      const int r = static_cast<int>(tok[j] & 63);
      if constexpr (kFp4) {
        load_key_fp4(base, r, g, ok, k4[j]);
      } else {
        const uint4 k0 = *reinterpret_cast<const uint4*>(base + r * kIdxDim + 16 * g);
        const uint4 k1 = *reinterpret_cast<const uint4*>(base + r * kIdxDim + 64 + 16 * g);
        const float sc = *reinterpret_cast<const float*>(base + kIdxPageBytes + r * 4);
        kb[j][0] = ok ? k0 : make_uint4(0, 0, 0, 0);
        kb[j][1] = ok ? k1 : make_uint4(0, 0, 0, 0);
        ks[j] = ok ? sc : 0.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < kVerifyBatch; ++j) {
      const int b0 = bb + 64 * j;
      if (b0 >= total) break;
      float sc;
      if constexpr (kFp4) {
        sc = exact_block_fp4([&](int hb, int b) { return op4.q[hb][b]; }, [&](int h) { return s_table[h]; }, op4.wv,
                             k4[j]);
      } else {
        sc = exact_block(op, s_table, kb[j], ks[j]);
      }
      const int li = b0 + col;
      if (li < total && g == 0) {
        const int meta = s_meta[li];
        const int64_t dst = row + static_cast<int64_t>(c_begin + (meta >> 11)) * kChunk + (meta & 2047);
        a.cand_score[dst] = sc;
        a.cand_idx[dst] = tok0 + s_list[li];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Filter + verify in one launch.  Every workgroup of the grid is resident at
// once (the host sizes the grid from the occupancy), so the upper bounds stay
// in LDS: each workgroup streams its contiguous page range, adds its
// lower-bound histogram to the row's, and the last workgroup of the row to
// arrive turns the complete histogram into the bound and publishes it.  Each
// workgroup then lists its own candidates in token order and scores them
// exactly into its segment's slice.
// Within a workgroup the waves take pages one at a time from an LDS counter:
// the hardware issues the oldest waves first, so a static split would leave
// the youngest waves finishing last.
// The wait for the bound is bounded: a workgroup that gives up takes bin 0,
// which makes every token of its segment a candidate -- slower, still exact.
//
// In-launch select (FusedArgs::sel_out set): the row's workgroups then also
// agree on the exact top-k threshold and each writes its own selected tokens,
// at offset (greater keys in earlier segments) + min(tied keys in earlier
// segments, ties to take): segments are in token order, so the lowest
// indices take the ties.
//   * Exchange: each workgroup writes its candidate list (token, exact score)
//     and count, arrives, and once the whole row has arrived reads the
//     counts.  At least k tokens have a lower bound L in the bound bin b* or
//     above, so the k-th largest exact key is >= lo = b* << 20.
//   * Local select (the row's candidates fit a workgroup's LDS, 2 kList
//     keys): every workgroup loads all of the row's keys and finds the
//     threshold with histogram passes in LDS -- first [lo, lo + 2^22) in 4096
//     bins of 2^10 keys (keys above in one more counter); a threshold bin
//     whose keys are all needed ends the search, else the next pass splits
//     its low 10 bits; if the window misses the threshold, passes of 12, 12
//     and 8 bits over the whole key range follow (radix select).  The keys of
//     the earlier segments give its offsets.
//   * Otherwise the same passes run as rounds over the workgroups, each
//     closed by the last to arrive, which publishes the decision the others
//     wait for, and a records round exchanges each workgroup's (greater,
//     tied) counts.
// Every wait is bounded.  A workgroup that gives up marks the row; each
// workgroup has written its candidate list before the exchange, and the last
// to depart from a marked row selects over those lists alone (exact, slower)
// and counts it in timeouts[2].
// Outputs, lists and counters of this path are written with agent-scope
// stores and read back with agent-scope loads, so they are coherent across
// the XCDs' L2s within the launch.
// ---------------------------------------------------------------------------
// Per-row control block of the fused kernel, kCounterRow words per row at
// fixed offsets at the front of the workspace:
//   [0, kHistSlot)              histogram A: kHistBins bins, then [kHistBins]
//                               keys above the bins, [kHistBins + 1] keys counted
//   [kHistSlot, 2 kHistSlot)    histogram B (the rounds alternate A and B;
//                               the bound uses A)
//   kArriveWord                 arrivals (bits 0..15, cumulative over the
//                               rounds) and departures (bits 16..31)
//   kFailWord                   set when a wait of the row gave up
//   kDecWords + 8 r             decision of round r (r = 0: the bound word,
//                               (bin << 20) | 1 once published; r = 1, the
//                               exchange, has none)
//   kRecWords + 2 x             workgroup x's (greater, tied) counts
// All of it is zero when a call starts and the call leaves it zero: a round's
// last arriver zeroes its histogram after reading it, the last workgroup to
// depart clears the arrival, fail and decision words and the records (and,
// for a marked row, both histograms).  So the fused path needs no clearing
// launch, only a workspace that was zero-filled once.
constexpr int kHistSlot = kHistBins + 2;
constexpr int kArriveWord = 2 * kHistSlot;
constexpr int kFailWord = kArriveWord + 1;
constexpr int kDecWords = kArriveWord + 4;
constexpr int kSelRounds = 6;  // the bound, the exchange and at most four histogram rounds
constexpr int kRecWords = kDecWords + 8 * kSelRounds;
constexpr int kSelMaxGroups = 256;  // workgroups per row the in-launch select takes
constexpr int kCounterRow = kRecWords + 2 * kSelMaxGroups;
constexpr int kCounterRows = 1024;  // rows the fused path takes (at most 3 x CUs)
constexpr int kHistRereads = 64;    // reads of a row histogram that does not yet sum to its tokens
constexpr int64_t kCounterBytes = 256 + int64_t{kCounterRows} * kCounterRow * 4;

// The DSA decode prologue (ekv_dsa_decode_prologue) folded into the fused
// launch, for decode rows (the new tokens lie in their rows' windows, so no
// row scores them): every workgroup prepares and quantizes its row's indexer
// q into LDS as indexer_q_quant does, and takes the row's key count as
// max(position + 1 - window, 0); the row's first workgroup to arrive at the
// bound (workgroup 0 of a row with nothing to score) appends the new token's
// indexer K row and latent row (two waves) and writes the q codes, the
// folded weights and the digit planes out as the prologue would, while the
// bound is computed; workgroup 0 writes the count.
struct FusedPrologue {
  const uint16_t* q;         // [T, 64, 128] bf16 (the raw projection when cos_sin is set)
  int64_t q_tok_stride, q_head_stride;
  const void* w;             // [T, w_stride] bf16 or fp32 head weights
  int32_t w_is_bf16;
  int64_t w_stride;
  const float* cos_sin;      // [cs_rows, 64] (RoPE and Hadamard of q first), or null
  int32_t cs_rows;
  int32_t* lengths;          // [T] out: max(position + 1 - window, 0)
  uint8_t* q_fp8_out;        // [T, 64, 128] out (or null)
  float* w_out;              // [T, 64] out (or null)
  int8_t* q_digits_out;      // [T, 3, 64, 128] out (or null)
  AppendArgs k_rows;         // the indexer K rows (D = 128; the prep fields with cos_sin)
  AppendArgs latent;         // the latent rows
  int32_t latent_dim;        // 512 or 576
};

// Row t's q rows as loaded (16 lanes per head, kThreads / 16 heads a pass)
// and the head weights (lane 0 of each head).
template <int kThreads>
struct FusedQRows {
  static constexpr int kPasses = (kIdxHeads * 16 + kThreads - 1) / kThreads;
  uint4 raw[kPasses];
  uint32_t wbits[kPasses];  // the weight as loaded (bf16 or fp32 bits), converted when used
  RopeLane rope;            // (the same position for every head)
};

template <int kThreads>
__device__ __forceinline__ void fused_q_load(const FusedPrologue& p, int64_t t, int64_t pos, FusedQRows<kThreads>& r) {
  const int ln = threadIdx.x & 15;
  r.rope = rope_lane((p.cos_sin != nullptr && pos >= 0 && pos < p.cs_rows) ? p.cos_sin + pos * 64 : nullptr, ln);
#pragma unroll
  for (int ps = 0; ps < FusedQRows<kThreads>::kPasses; ++ps) {
    const int h = ps * (kThreads / 16) + static_cast<int>(threadIdx.x >> 4);
    r.raw[ps] = make_uint4(0, 0, 0, 0);
    r.wbits[ps] = 0u;
    if (h < kIdxHeads) {
      r.raw[ps] = *reinterpret_cast<const uint4*>(p.q + t * p.q_tok_stride + h * p.q_head_stride + 8 * ln);
      if (ln == 0)
        r.wbits[ps] = p.w_is_bf16 ? static_cast<uint32_t>(static_cast<const uint16_t*>(p.w)[t * p.w_stride + h])
                                  : static_cast<const uint32_t*>(p.w)[t * p.w_stride + h];
    }
  }
}

// indexer_q_quant's arithmetic on row t (position pos): codes to
// s_q8[h * 128 + d], folded weights to s_w[h].
template <int kThreads>
__device__ __forceinline__ void fused_q_quant(const FusedPrologue& p, const FusedQRows<kThreads>& r, uint8_t* s_q8,
                                              float* s_w) {
  const int ln = threadIdx.x & 15;
#pragma unroll
  for (int ps = 0; ps < FusedQRows<kThreads>::kPasses; ++ps) {
    const int h = ps * (kThreads / 16) + static_cast<int>(threadIdx.x >> 4);
    if (h >= kIdxHeads) continue;  // whole 16-lane groups
    float v[8];
    unpack_bf16x8(r.raw[ps], v);
    if (p.cos_sin != nullptr) {
      row_rope_neox64_lane(v, r.rope, ln);
      row_hadamard(v, ln);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = wave_max_xor(amax, 16);
    const int e = ue8m0_exponent(amax);
    const float inv = exp2i(-e);
    const uint32_t b0 = f32x2_to_fp8(v[0] * inv, v[1] * inv);
    const uint32_t b1 = f32x2_to_fp8(v[2] * inv, v[3] * inv);
    const uint32_t b2 = f32x2_to_fp8(v[4] * inv, v[5] * inv);
    const uint32_t b3 = f32x2_to_fp8(v[6] * inv, v[7] * inv);
    *reinterpret_cast<uint2*>(s_q8 + h * kIdxDim + 8 * ln) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
    if (ln == 0) {
      const float wt = p.w_is_bf16 ? bf16_to_f32(static_cast<uint16_t>(r.wbits[ps])) : __uint_as_float(r.wbits[ps]);
      s_w[h] = (wt * exp2i(e)) * 0x1.6a09e6p-7f;  // fl32(128**-0.5 * 64**-0.5)
    }
  }
}

// Digit d of 16 fp8 codes (byte i of the result: digit d of code i), with
// pack(code) = fp8_digit_pack(code) or its table.
template <class Pack>
__device__ __forceinline__ i32x4 digit_word(const uint4& codes, int d, Pack pack) {
  const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
  int out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t r = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) r |= ((pack((w[i] >> (8 * b)) & 0xffu) >> (8 * d)) & 0xffu) << (8 * b);
    out[i] = static_cast<int>(r);
  }
  return i32x4{out[0], out[1], out[2], out[3]};
}

// The prologue's q outputs of row t from the LDS copy: the codes, the folded
// weights and the digit planes [t][digit][h][128] (a null output skipped).
template <int kThreads, class Pack>
__device__ __forceinline__ void fused_store_q(const FusedPrologue& p, int64_t t, const uint8_t* s_q8, const float* s_w,
                                              Pack pack) {
  const int tid = threadIdx.x;
  constexpr int kChunks = kIdxHeads * kIdxDim / 16;  // 16-byte chunks of codes
  for (int c = tid; c < kChunks; c += kThreads) {
    const uint4 v = *reinterpret_cast<const uint4*>(s_q8 + 16 * c);
    if (p.q_fp8_out != nullptr) *reinterpret_cast<uint4*>(p.q_fp8_out + t * (kIdxHeads * kIdxDim) + 16 * c) = v;
    if (p.q_digits_out != nullptr) {
      const int h = c / (kIdxDim / 16), d0 = 16 * (c % (kIdxDim / 16));
#pragma unroll
      for (int d = 0; d < 3; ++d)
        *reinterpret_cast<i32x4*>(p.q_digits_out + ((t * 3 + d) * kIdxHeads + h) * kIdxDim + d0) =
            digit_word(v, d, pack);
    }
  }
  if (p.w_out != nullptr && tid < kIdxHeads) p.w_out[t * kIdxHeads + tid] = s_w[tid];
}

// The new token's rows of query row t, as the prologue appends them: wave
// kWaves - 1 the indexer K row (16 lanes; the k_norm, RoPE and Hadamard prep
// when k_rows.cos_sin is set), wave kWaves - 2 the latent row.
template <int kWaves>
__device__ __forceinline__ void fused_appends(const FusedPrologue& p, int64_t t) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave == kWaves - 1) {
    const AppendArgs& a = p.k_rows;
    const int ln = lane & 15;  // (the four 16-lane groups compute the row, the first stores it)
    uint4 raw[1];
    load_bf16_row<128, 16>(a.rows + t * a.row_stride, ln, raw);
    const int64_t slot = a.slot_mapping[t];
    if (a.cos_sin != nullptr) {
      float v[8];
      unpack_bf16x8(raw[0], v);
      const int64_t pos = a.positions[t];
      row_layer_norm(v, a.ln_w, a.ln_b, a.eps, ln);
      row_rope_neox64(v, (pos >= 0 && pos < a.cs_rows) ? a.cos_sin + pos * 64 : nullptr, ln);
      row_hadamard(v, ln);
      raw[0] = pack_bf16x8(v);
    }
    if (lane < 16) store_row<128, 16>(a, slot, ln, raw);
  } else if (wave == kWaves - 2) {
    const AppendArgs& a = p.latent;
    if (p.latent_dim == 576) {
      uint4 raw[Fp8Row<576, 64>::kPerLane];
      load_bf16_row<576, 64>(a.rows + t * a.row_stride, lane, raw);
      store_row<576, 64>(a, a.slot_mapping[t], lane, raw);
    } else {
      uint4 raw[Fp8Row<512, 64>::kPerLane];
      load_bf16_row<512, 64>(a.rows + t * a.row_stride, lane, raw);
      store_row<512, 64>(a, a.slot_mapping[t], lane, raw);
    }
  }
}

// The prologue's outputs and appends of row t: after the stream (digits
// through the LDS digit table), or alone in a row with nothing to score.
template <int kThreads, int kWaves>
__device__ __forceinline__ void fused_outputs(const FusedPrologue& p, int64_t t, const uint8_t* s_q8,
                                              const float* s_w, const uint32_t* s_table) {
  fused_store_q<kThreads>(p, t, s_q8, s_w, [=](uint32_t code) { return s_table[code]; });
  fused_appends<kWaves>(p, t);
}

template <int kThreads, int kWaves>
__device__ __forceinline__ void fused_prologue_only(const FusedPrologue& p, int64_t t, int64_t pos, uint8_t* s_q8,
                                                    float* s_w) {
  FusedQRows<kThreads> qr;
  fused_q_load<kThreads>(p, t, pos, qr);
  fused_q_quant<kThreads>(p, qr, s_q8, s_w);
  __syncthreads();
  fused_store_q<kThreads>(p, t, s_q8, s_w, [](uint32_t code) { return fp8_digit_pack(code); });
  fused_appends<kWaves>(p, t);
}

struct FusedArgs {
  FilterArgs f;              // f.upper and f.hist are not used
  const int8_t* q_digits;    // [T, 3, 64, 128]
  uint32_t* counters;        // [kCounterRows, kCounterRow]
  uint32_t* timeouts;        // [0] bound waits that gave up, [1] histograms that never summed,
                             // [2] rows whose select ran alone after a wait gave up
                             // (diagnostic, cumulative)
  float* cand_score;         // [T, max_len] segment slices
  int32_t* cand_idx;
  int32_t* cand_count;       // [T, groups]
  int32_t groups;
  int32_t stage_pages;       // LDS capacity in pages (>= pages per workgroup of every row)
  int32_t spin_limit;        // polls of a wait before it gives up
  // In-launch select (null: the candidate lists are left for topk_select_kernel)
  int32_t* sel_out;          // [T, sel_stride] top-k, ascending, -1 padded
  int64_t sel_stride;
  int32_t* merged;           // optional [T, merged_stride] rows of merge_swa_topk (see SelectArgs)
  int64_t merged_stride;
  int32_t merged_width;
  const int64_t* positions;
  int32_t window;
  int32_t merged_slots;      // merged entries as cache slots through the block table
  // The folded prologue, read by filter_verify_kernel<W, false, true> only
  // (fp8 keys, in-launch select with merged rows): q, the weights and the
  // key counts come from `pro`, not from f.q_fp8, f.w, q_digits and
  // f.lengths.
  FusedPrologue pro;
};

__device__ __forceinline__ uint32_t ld_agent(const void* p) {
  return __hip_atomic_load(static_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(void* p, uint32_t v) {
  __hip_atomic_store(static_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS histogram increment: the lanes sharing a bin with the first remaining
// lane add with one atomic, twice; the others one atomic per lane.  Runs of
// equal keys (ties) then cost one or two atomics per wave instead of one per
// lane on the same address.
__device__ __forceinline__ void hist_add_ties(uint32_t* hist, int bin) {
  const int lane = threadIdx.x & 63;
  uint64_t act = __ballot(bin >= 0);
  // two rounds: the lanes sharing the first remaining lane's bin add with
  // one atomic (a tie group, most of a wave in tie-heavy rows, is taken in
  // one of them); the rest add one each
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (act == 0) return;
    const int leader = static_cast<int>(__builtin_ctzll(act));
    const int lb = __builtin_amdgcn_readlane(bin, leader);
    const uint64_t same = __ballot(bin == lb) & act;
    if (lane == leader) atomicAdd(&hist[lb], static_cast<uint32_t>(__popcll(same)));
    act &= ~same;
  }
  if ((act >> lane) & 1u) atomicAdd(&hist[bin], 1u);
}

// Pages of each workgroup's segment: workgroup x of a row owns logical pages
// [x, x + 1) * fused_group_pages.
__host__ __device__ inline int fused_group_pages(int n, int groups) {
  const int npages = (n + kPageTokens - 1) / kPageTokens;
  return (npages + groups - 1) / groups;
}

constexpr int kFusedQdBytes = 4 * 3 * 2 * 64 * 16;  // q digit operands [hb][digit][K half][lane]
constexpr int kFusedSpinLimit = 1 << 14;            // default FusedArgs::spin_limit
static_assert(kHistSlot * 4 <= kFusedQdBytes, "a select round's LDS histogram shares the q operands' LDS");

template <int kWaves>
struct FusedLayout {
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kList = 8 * kThreads;  // candidates scored per pass (>= one compaction round)
  // q operands / histogram | table | list | list scores | misc
  static constexpr int kFixed = kFusedQdBytes + 256 * 4 + 2 * kList * 4 + 32 * 4;
  static constexpr int bytes(int stage_pages) { return kFixed + stage_pages * (4 + 2 * kPageTokens); }
};

// The bin of an nbins-bin histogram (read(b) = count of bin b, `above` keys
// past the bins) holding the k-th largest key: (keys above bin fb) < k <=
// (keys above fb) + h.  fb = -1 when the bins and `above` cannot hold it.
template <int kThreads, class Read>
__device__ __forceinline__ void find_threshold_bin(Read read, int nbins, int above, int k, int* s_misc, int& fb,
                                                   int& above_f, int& h) {
  constexpr int kPer = (kHistBins + kThreads - 1) / kThreads;  // bins per thread, from the top down
  const int rb0 = kPer * static_cast<int>(threadIdx.x);
  int hc[kPer];
  int sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    hc[j] = (rb0 + j < nbins) ? read(nbins - 1 - (rb0 + j)) : 0;
    sum += hc[j];
  }
  if (threadIdx.x == 0) s_misc[28] = -1;
  int total;
  int e = above + block_scan_excl<kThreads>(sum, s_misc, total);  // keys above this thread's first bin
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (rb0 + j < nbins && e < k && k <= e + hc[j]) {
      s_misc[28] = nbins - 1 - (rb0 + j);
      s_misc[29] = e;
      s_misc[30] = hc[j];
    }
    e += hc[j];
  }
  __syncthreads();
  fb = s_misc[28];
  above_f = s_misc[29];
  h = s_misc[30];
  __syncthreads();
}

// What a histogram pass over keys >= lo (bins of 2^shift keys) decides, from
// its threshold bin fb (above_f keys above it, h in it):
//   1: another pass: p = (lo, shift, nbins, keys >= lo) -- the bin's low
//      bits split 12 at a time, or, when the first pass's window missed
//      (fb < 0), 12 bits of the whole key range;
//   2: final: p = (thr_lo, thr_hi, ties to take): keys >= thr_hi are taken,
//      then `need` keys of [thr_lo, thr_hi) -- the bin's lower edge when all
//      its keys are needed, else its single key;
//   3: no decision (a pass after the first whose window misses).
__device__ inline int select_decision(bool first, uint32_t lo, int shift, int k, int fb, int above_f, int h,
                                      uint32_t (&p)[5]) {
  p[0] = p[1] = p[2] = p[3] = p[4] = 0u;
  if (fb < 0) {
    if (!first) return 3;
    p[1] = 20u;
    p[2] = static_cast<uint32_t>(kHistBins);
    p[3] = 0xffffffffu;
    return 1;
  }
  const int nd = k - above_f;
  const uint32_t base = lo + (static_cast<uint32_t>(fb) << shift);
  if (nd == h) {
    p[0] = p[1] = base;
    return 2;
  }
  if (shift == 0) {
    p[0] = base;
    p[1] = base + 1u;
    p[2] = static_cast<uint32_t>(nd);
    return 2;
  }
  const int next = shift > kHistBits ? shift - kHistBits : 0;  // split the bin's low bits, 12 at a time
  p[0] = base;
  p[1] = static_cast<uint32_t>(next);
  p[2] = 1u << (shift - next);
  p[3] = static_cast<uint32_t>(above_f + h);
  return 1;
}

// The in-launch select's outputs of row t: the top-k row and the optional
// merged row, whose entry for token i is i or, with merged_slots, its cache
// slot through the block table (-1 when unmapped).  Built where it is used,
// so none of it stays live across the page stream.
struct SelRow {
  int32_t* out;
  int32_t* merged;
  int64_t seq, m_topk, width, window;
  const int32_t* bt;  // null unless merged_slots
  int64_t bt_stride, num_pages;
  __device__ __forceinline__ SelRow(const FusedArgs& a, int t)
      : out(a.sel_out + static_cast<int64_t>(t) * a.sel_stride),
        merged(a.merged ? a.merged + static_cast<int64_t>(t) * a.merged_stride : nullptr),
        seq(0), m_topk(0), width(a.merged_width), window(a.window), bt(nullptr), bt_stride(a.f.bt_stride),
        num_pages(a.f.num_pages) {
    if (merged) {
      seq = a.positions[t] + 1;
      m_topk = min(min(max(seq - window, int64_t{0}), static_cast<int64_t>(a.f.k)), width);
      if (a.merged_slots) bt = a.f.block_table + static_cast<int64_t>(a.f.req_ids[t]) * a.f.bt_stride;
    }
  }
  __device__ __forceinline__ uint32_t entry(int64_t i) const {
    if (bt == nullptr || i < 0) return static_cast<uint32_t>(i);
    if ((i >> 6) >= bt_stride) return 0xffffffffu;
    const int64_t p = bt[i >> 6];
    return (p >= 0 && p < num_pages) ? static_cast<uint32_t>(p * kPageTokens + (i & 63)) : 0xffffffffu;
  }
  // output entry pos = token tok (or -1); the merged entry from the block table
  __device__ __forceinline__ void emit(int64_t pos, int64_t tok) const {
    st_agent(out + pos, static_cast<uint32_t>(tok));
    if (merged && pos < m_topk) st_agent(merged + pos, entry(tok));
  }
  // the same with the token's page known (-1: unmapped)
  __device__ __forceinline__ void emit_paged(int64_t pos, int64_t tok, int64_t page) const {
    st_agent(out + pos, static_cast<uint32_t>(tok));
    if (merged && pos < m_topk)
      st_agent(merged + pos, bt == nullptr ? static_cast<uint32_t>(tok)
                                           : (page >= 0 ? static_cast<uint32_t>(page * kPageTokens + (tok & 63))
                                                        : 0xffffffffu));
  }
  // entries [m_topk, width) of the merged row: the window, then -1
  __device__ __forceinline__ void window_part(int tid, int nthreads) const {
    if (!merged) return;
    const int64_t w = min(seq, window);
    for (int64_t c = m_topk + tid; c < width; c += nthreads)
      st_agent(merged + c, (c < m_topk + w) ? entry(seq - w + (c - m_topk)) : 0xffffffffu);
  }
};

// fp4 keys: the q operands of the exact path, [hb][block][lane] 8-byte words.
constexpr int kFusedQ4Words = 4 * 4 * 64;
static_assert(kFusedQ4Words * 8 <= kFusedQdBytes, "fp4 q operands share the digit operands' LDS");

template <int kWaves, bool kFp4, bool kPro = false>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(3))) filter_verify_kernel(FusedArgs a) {
  using Lay = FusedLayout<kWaves>;
  constexpr int kThreads = Lay::kThreads;
  extern __shared__ __align__(16) uint8_t fused_smem[];
  uint32_t* s_hist = reinterpret_cast<uint32_t*>(fused_smem);     // phase 1
  const uint4* s_qd = reinterpret_cast<const uint4*>(fused_smem);  // phases 2-3 (same bytes)
  const uint2* s_q4 = reinterpret_cast<const uint2*>(fused_smem);  // fp4: phases 2-3 (same bytes)
  uint32_t* s_table = reinterpret_cast<uint32_t*>(fused_smem + kFusedQdBytes);  // fp4: q scale words
  int32_t* s_list = reinterpret_cast<int32_t*>(s_table + 256);
  float* s_score = reinterpret_cast<float*>(s_list + Lay::kList);  // exact scores of the list
  int* s_misc = reinterpret_cast<int*>(s_score + Lay::kList);  // [0..15] scans, [16] last, [17] bin, [18] next page
  int32_t* s_pages = reinterpret_cast<int32_t*>(s_misc + 32);
  uint16_t* s_pref = reinterpret_cast<uint16_t*>(s_pages + a.stage_pages);

  const int tid = threadIdx.x;
  const int t = blockIdx.y, x = blockIdx.x;
  const FilterArgs& f = a.f;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;
  // The folded prologue's q codes and weights (8 KB + 256 B) sit in the list's
  // LDS until the list is built.
  uint8_t* const s_q8 = reinterpret_cast<uint8_t*>(s_list);
  float* const s_qw = reinterpret_cast<float*>(s_q8 + kIdxHeads * kIdxDim);
  static_assert(kIdxHeads * (kIdxDim + 4) <= 2 * Lay::kList * 4, "the prologue's q fits the list's LDS");
  static_assert(!(kPro && kFp4), "the folded prologue takes fp8 keys");
  constexpr bool pro = kPro;
  const int32_t req = f.req_ids[t];  // (requested with the row's length or position)
  FilterOps op;
  int64_t pos = 0, wl = 0;
  int n;
  if (pro) {
    pos = a.positions[t];
    wl = max(pos + 1 - static_cast<int64_t>(a.window), int64_t{0});
    n = static_cast<int>(min(wl, static_cast<int64_t>(f.max_len)));
  } else {
    load_filter_operands<kFp4>(f, t, g, col, op);  // (issued with the row length's load)
    n = max(0, min(f.lengths[t], f.max_len));
  }
  const int npages = (n + kPageTokens - 1) / kPageTokens;
  const int per_group = fused_group_pages(n, a.groups);
  const int wg_p0 = x * per_group, wg_p1 = min(wg_p0 + per_group, npages);
  const int seg0 = wg_p0 * kPageTokens;  // first token of this workgroup's segment
  const int seg_len = min(per_group * kPageTokens, n - seg0);
  const int64_t out0 = static_cast<int64_t>(t) * f.max_len + seg0;
  int32_t* count = a.cand_count + static_cast<int64_t>(t) * a.groups + x;

  const bool sel = a.sel_out != nullptr;
  if (sel && x == 0) {
    // the window part of the merged row, and the -1 fill past n when every
    // token is selected (also for rows without tokens)
    const SelRow so(a, t);
    so.window_part(tid, kThreads);
    if (n <= f.k)
      for (int i = n + tid; i < f.k; i += kThreads) so.emit(i, -1);
  }
  if (pro && x == 0 && tid == 0 && a.pro.lengths != nullptr) a.pro.lengths[t] = static_cast<int32_t>(wl);
  // (the first workgroup of a row with nothing to score still writes the
  // prologue's outputs and appends)
  if (seg_len <= 0) {  // no pages in this segment
    if (pro && x == 0) fused_prologue_only<kThreads, kWaves>(a.pro, t, pos, s_q8, s_qw);
    if (tid == 0) *count = 0;
    return;
  }
  if (n <= f.k) {  // every token is selected: list them, no scores needed
    if (sel) {
      const SelRow so(a, t);
      for (int i = tid; i < seg_len; i += kThreads) so.emit(seg0 + i, seg0 + i);
    } else {
      for (int i = tid; i < seg_len; i += kThreads) a.cand_idx[out0 + i] = seg0 + i;
    }
    if (pro && x == 0) fused_prologue_only<kThreads, kWaves>(a.pro, t, pos, s_q8, s_qw);
    if (tid == 0) *count = seg_len;
    return;
  }
  // (the folded prologue's q rows, weights and RoPE entries are requested
  // with the block-table entry, and quantized while the first pages load)
  FusedQRows<kThreads> qr;
  if (pro) fused_q_load<kThreads>(a.pro, t, pos, qr);
  // each wave's first page is requested before the LDS set-up, so its
  // memory latency overlaps it and the q operands' (requested first)
  FirstPage first_page;
  {
    const PageSource<kFp4> src(f, req, wg_p1);
    first_page.page = src.page_of(wg_p0 + wave);
    src.load(first_page.page, first_page.kb, first_page.ks);
  }
  if (pro) fused_q_quant<kThreads>(a.pro, qr, s_q8, s_qw);
  for (int i = tid; i < kHistBins; i += kThreads) s_hist[i] = 0;
  if constexpr (kFp4) {
    if (tid < kIdxHeads) s_table[tid] = static_cast<uint32_t>(f.q_scales[static_cast<int64_t>(t) * kIdxHeads + tid]);
  } else {
    if (tid < 256) s_table[tid] = fp8_digit_pack(static_cast<uint32_t>(tid));
  }
  if (tid == 0) s_misc[18] = wg_p0 + kWaves;  // wave w starts at page wg_p0 + w
  __syncthreads();
  if (pro) filter_operands_fp8(s_q8, s_qw, g, col, op);

  // Phase 1: stream the pages; upper-bound prefixes and page entries to LDS.
  auto grab = [&]() -> int {
    int v = 0;
    if (lane == 0) v = atomicAdd(&s_misc[18], 1);
    return __builtin_amdgcn_readfirstlane(v);
  };
  filter_stream<kFp4>(f, req, n, wg_p0 + wave, wg_p1, grab, s_hist, op,
                      [&](int lp, int64_t page, float sc, float e) {
                        s_pref[(lp - wg_p0) * kPageTokens + lane] = upper_prefix(sc, e);
                        if (lane == 0) s_pages[lp - wg_p0] = static_cast<int32_t>(page);
                      },
                      &first_page);
  __syncthreads();
  uint32_t* const rowc = a.counters + static_cast<int64_t>(t) * kCounterRow;
  uint32_t* const gh = rowc;  // histogram A
  uint32_t* const arrive = rowc + kArriveWord;
  uint32_t* const kword = rowc + kDecWords;
  for (int i = tid; i < kHistBins; i += kThreads) {
    const uint32_t v = s_hist[i];
    if (v) atomicAdd(&gh[i], v);
  }
  // q exact operands, loaded now and stored into the histogram's LDS once
  // every lane is past it (fp8: digit planes; fp4: the 2 * e2m1 values,
  // [hb][block][lane]).
  constexpr int kQdPer = (kFusedQdBytes / 16) / kThreads;
  static_assert(kQdPer * kThreads * 16 == kFusedQdBytes, "q digit staging must divide evenly");
  constexpr int kQ4Per = (kFusedQ4Words + kThreads - 1) / kThreads;
  // (native vectors: kept in registers)
  i32x4 qd_regs[kFp4 ? 1 : kQdPer];
  i32x2 q4_regs[kFp4 ? kQ4Per : 1];
  if constexpr (kFp4) {
#pragma unroll
    for (int j = 0; j < kQ4Per; ++j) {
      const int idx = tid + kThreads * j;  // entry e = hb * 4 + b, lane ln
      const int e = idx >> 6, ln = idx & 63;
      int64_t v = 0;
      if (idx < kFusedQ4Words) v = load_q_fp4(f.q_fp8, t, e >> 2, e & 3, ln >> 4, ln & 15);
      q4_regs[j] = i32x2{static_cast<int>(v), static_cast<int>(static_cast<uint64_t>(v) >> 32)};
    }
  } else {
#pragma unroll
    for (int j = 0; j < kQdPer; ++j) {
      const int idx = tid + kThreads * j;  // entry e = (hb * 3 + d) * 2 + kh, lane ln
      const int e = idx >> 6, ln = idx & 63;
      const int hb = e / 6, d = (e / 2) % 3, kh = e & 1;
      const int lg = ln >> 4, lc = ln & 15;
      if (pro)  // digit d of the 16 codes, through the digit table
        qd_regs[j] = digit_word(*reinterpret_cast<const uint4*>(s_q8 + (16 * hb + lc) * kIdxDim + 64 * kh + 16 * lg), d,
                                [&](uint32_t code) { return s_table[code]; });
      else
        qd_regs[j] = *reinterpret_cast<const i32x4*>(a.q_digits + ((static_cast<int64_t>(t) * 3 + d) * kIdxHeads +
                                                                   16 * hb + lc) * kIdxDim + 64 * kh + 16 * lg);
    }
  }
  // Every histogram atomic of the workgroup has completed before it arrives.
  // No cache maintenance is needed: device-scope atomics and the agent-scope
  // loads and stores below are coherent across the L2s, and a histogram read
  // before some adds were visible could only lower the bound (more
  // candidates, still exact).
  handoff_wait();
  __syncthreads();
  // (every lane is past the histogram: the q operands take its LDS now, so
  // they are not held in registers across the wait below)
  if constexpr (kFp4) {
    i32x2* s_q4_w = reinterpret_cast<i32x2*>(fused_smem);
#pragma unroll
    for (int j = 0; j < kQ4Per; ++j)
      if (tid + kThreads * j < kFusedQ4Words) s_q4_w[tid + kThreads * j] = q4_regs[j];
  } else {
    i32x4* s_qd_w = reinterpret_cast<i32x4*>(fused_smem);
#pragma unroll
    for (int j = 0; j < kQdPer; ++j) s_qd_w[tid + kThreads * j] = qd_regs[j];
  }

  // Phase 2: arrive; the last workgroup of the row publishes the bound.
  // Every workgroup reads the row histogram as it arrives (the last one to
  // arrive then has it without a second round trip; the others ignore it).
  constexpr int kBinsPer = (kHistBins + kThreads - 1) / kThreads;  // scanned from the top bin down
  const int r0 = kBinsPer * tid;
  int c[kBinsPer];
  auto read_hist = [&]() -> int {
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kBinsPer; ++j) {
      c[j] = (r0 + j < kHistBins) ? static_cast<int>(__hip_atomic_load(gh + (kHistBins - 1 - (r0 + j)),
                                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                                  : 0;
      sum += c[j];
    }
    return sum;
  };
  int first_sum = read_hist();
  const int groups_row = (npages + per_group - 1) / per_group;
  if (tid == 0) {
    const uint32_t before = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_misc[16] = ((before & 0xffffu) + 1u == static_cast<uint32_t>(groups_row)) ? 1 : 0;
    s_misc[17] = 0;
    s_misc[19] = 0;  // a wait of this workgroup gave up
    s_misc[26] = ((before & 0xffffu) == 0u) ? 1 : 0;  // the row's first arrival
  }
  __syncthreads();
  // The folded prologue's outputs and appends: by the row's first workgroup
  // to arrive, while it waits for the bound (after publishing it, in a row of
  // one workgroup).
  const bool pro_out = pro && s_misc[26] != 0;
  if (pro_out && !s_misc[16]) fused_outputs<kThreads, kWaves>(a.pro, t, s_q8, s_qw, s_table);
  if (s_misc[16]) {
    int excl = 0, total = 0;
    // The row histogram counts each of the row's n tokens once.  Every
    // workgroup's adds completed before it arrived, so the bins sum to n;
    // the check makes the bound (and the clearing below) rely on that sum,
    // not on the ordering: the bins are read again until they sum to n (the
    // read made on arrival may predate the other workgroups' arrivals), and
    // a histogram that never does gives bin 0 (every token a candidate).
    for (int attempt = 0;; ++attempt) {
      const int sum = attempt == 0 ? first_sum : read_hist();
      excl = block_scan_excl<kThreads>(sum, s_misc, total);
      if (total == n || attempt == kHistRereads) break;
      __builtin_amdgcn_s_sleep(8);
    }
    if (total == n) {
#pragma unroll
      for (int j = 0; j < kBinsPer; ++j) {
        if (excl < f.k && f.k <= excl + c[j]) s_misc[17] = kHistBins - 1 - (r0 + j);
        excl += c[j];
      }
    } else if (tid == 0) {
      atomicAdd(a.timeouts + 1, 1u);  // bin 0 (s_misc[17] stays 0)
    }
    __syncthreads();
    if (tid == 0)
      __hip_atomic_store(kword, (static_cast<uint32_t>(s_misc[17]) << (32 - kHistBits)) | 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    // then leave the row histogram zero for the next call (every workgroup
    // of the row has arrived, so nothing in this call reads it again, and
    // the stores complete before the kernel does)
#pragma unroll
    for (int j = 0; j < kBinsPer; ++j)
      if (r0 + j < kHistBins)
        __hip_atomic_store(gh + (kHistBins - 1 - (r0 + j)), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if (tid == 0) {
    uint32_t v = 0;
    for (int spins = 0; spins < a.spin_limit; ++spins) {
      v = __hip_atomic_load(kword, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (v != 0) break;
      __builtin_amdgcn_s_sleep(4);
    }
    if (v == 0) {  // bin 0: every token is a candidate
      atomicAdd(a.timeouts, 1u);
      s_misc[19] = 1;
    }
    s_misc[17] = static_cast<int>(v >> (32 - kHistBits));
  }
  if (pro_out && s_misc[16]) fused_outputs<kThreads, kWaves>(a.pro, t, s_q8, s_qw, s_table);
  // depart: the last workgroup of the row to hold the bound clears the
  // bound and arrival words (the last arriver departs after publishing).
  // With the in-launch select the workgroups depart after the select.
  if (tid == 0 && !sel) {
    handoff_wait();
    const uint32_t before = __hip_atomic_fetch_add(arrive, 1u << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((before >> 16) + 1u == static_cast<uint32_t>(groups_row)) {
      __hip_atomic_store(kword, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  const uint32_t bin = static_cast<uint32_t>(s_misc[17]);
  const bool bound_gave_up = s_misc[19] != 0;

  // Phase 3: candidates of the segment in order, scored Lay::kList at a time.
  auto score_list = [&](int cnt, int base) {
    __syncthreads();
    // Passes of kBatch blocks per wave; the next pass's key rows are loaded
    // (into the other buffer) while a pass is scored.
    constexpr int kBatch = 2;
    constexpr int kStride = 16 * kWaves * kBatch;
    struct Keys {
      int tok[kBatch];
      bool ok[kBatch];
      uint4 kb[kBatch][2];
      float ks[kBatch];
      Fp4Key k4[kFp4 ? kBatch : 1];
    };
    auto load = [&](int bb, Keys& p) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int li = bb + 16 * kWaves * j + col;
        p.tok[j] = (li < cnt) ? s_list[li] : -1;  // offset in the segment
        const int64_t page = (p.tok[j] >= 0) ? static_cast<int64_t>(s_pages[p.tok[j] >> 6]) : -1;
        const bool ok = page >= 0;  // mapped pages only (checked when streamed)
        p.ok[j] = ok;
        const uint8_t* base_p = f.kcache + (ok ? page : 0) * f.page_stride;
        const int r = p.tok[j] & 63;
        if constexpr (kFp4) {
          load_key_fp4(base_p, r, g, ok, p.k4[j]);
        } else {
          // used as loaded (a missing entry reads a row of page 0 and its
          // score is zeroed after): values selected on `ok` here would let
          // the compiler put the loads under a branch
          p.kb[j][0] = *reinterpret_cast<const uint4*>(base_p + r * kIdxDim + 16 * g);
          p.kb[j][1] = *reinterpret_cast<const uint4*>(base_p + r * kIdxDim + 64 + 16 * g);
          p.ks[j] = *reinterpret_cast<const float*>(base_p + kIdxPageBytes + r * 4);
        }
      }
    };
    auto run = [&](int bb, const Keys& p) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int b0 = bb + 16 * kWaves * j;
        if (b0 >= cnt) break;
        float sc;
        if constexpr (kFp4) {
          sc = exact_block_fp4<true>(
              [&](int hb, int b) {
                const uint2 v = s_q4[(hb * 4 + b) * 64 + lane];
                return static_cast<int64_t>((static_cast<uint64_t>(v.y) << 32) | v.x);
              },
              [&](int h) { return s_table[h]; }, op.wv, p.k4[j]);
        } else {
          sc = exact_block_with<true>(
              [&](int hb, int d, int kh) {
                const uint4 v = s_qd[((hb * 3 + d) * 2 + kh) * 64 + lane];
                return i32x4{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
              },
              op.wv, s_table, p.kb[j], p.ks[j]);
          sc = p.ok[j] ? sc : 0.0f;  // an unmapped page's tokens score 0
        }
        const int li = b0 + col;
        if (li < cnt && g == 0) s_score[li] = sc;
      }
    };
    // (the loads are unconditional -- past the list they read a row of page
    // 0 and give zeros -- and the scores go to LDS, so only loads are in
    // flight and the waits for one buffer leave the other's loads going)
    Keys ka, kb2;
    int bb = wave * 16;
    load(bb, ka);
    __builtin_amdgcn_sched_barrier(0);
    for (;;) {
      if (bb >= cnt) break;
      load(bb + kStride, kb2);
      __builtin_amdgcn_sched_barrier(0);
      run(bb, ka);
      bb += kStride;
      if (bb >= cnt) break;
      load(bb + kStride, ka);
      __builtin_amdgcn_sched_barrier(0);
      run(bb, kb2);
      bb += kStride;
    }
    __syncthreads();
    for (int i = tid; i < cnt; i += kThreads) {
      st_agent(a.cand_score + out0 + base + i, __float_as_uint(s_score[i]));
      st_agent(a.cand_idx + out0 + base + i, static_cast<uint32_t>(seg0 + s_list[i]));
    }
    // the list's LDS may be refilled after this; the stores need not have
    // completed (a barrier with a fence would wait for them)
    __builtin_amdgcn_s_barrier();
  };
  // One scan over the whole segment (kOnePass groups of 8 tokens per thread)
  // when it is short enough and its candidates fit the list.
  constexpr int kOnePass = 3;
  int out_n = 0, lds_n = 0;  // candidates listed; the last lds_n of them are still in LDS
  bool listed = false;
  if (seg_len <= 8 * kOnePass * kThreads) {
    const int o0 = 8 * kOnePass * tid;
    uint32_t flags = 0;
    int cnt = 0;
#pragma unroll
    for (int v4 = 0; v4 < kOnePass; ++v4) {
      const int o = o0 + 8 * v4;
      if (o < seg_len) {
        const uint4 v = *reinterpret_cast<const uint4*>(s_pref + o);
        const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t pref = (wds[j >> 1] >> (16 * (j & 1))) & 0xffffu;
          if (o + j < seg_len && pref >= bin) {
            flags |= 1u << (8 * v4 + j);
            ++cnt;
          }
        }
      }
    }
    int tot;
    int pos = block_scan_excl<kThreads>(cnt, s_misc, tot);
    if (tot <= Lay::kList) {  // uniform
#pragma unroll
      for (int b = 0; b < 8 * kOnePass; ++b)
        if (flags & (1u << b)) s_list[pos++] = o0 + b;
      if (tot > 0) score_list(tot, 0);
      out_n = lds_n = tot;
      listed = true;
    }
  }
  if (!listed) {
    int list_n = 0;
    for (int r0 = 0; r0 < seg_len; r0 += 8 * kThreads) {
      const int o0 = r0 + 8 * tid;
      uint32_t flags = 0;
      int cnt = 0;
      if (o0 < seg_len) {
        const uint4 v = *reinterpret_cast<const uint4*>(s_pref + o0);
        const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t pref = (wds[j >> 1] >> (16 * (j & 1))) & 0xffffu;
          if (o0 + j < seg_len && pref >= bin) {
            flags |= 1u << j;
            ++cnt;
          }
        }
      }
      int rtot;
      const int ex = block_scan_excl<kThreads>(cnt, s_misc, rtot);
      if (list_n + rtot > Lay::kList) {  // uniform
        score_list(list_n, out_n);
        out_n += list_n;
        lds_n = list_n;
        list_n = 0;
      }
      int pos = list_n + ex;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (flags & (1u << j)) s_list[pos++] = o0 + j;
      list_n += rtot;
    }
    if (list_n > 0) {
      score_list(list_n, out_n);
      out_n += list_n;
      lds_n = list_n;
    }
  }
  if (tid == 0) st_agent(count, static_cast<uint32_t>(out_n));
  if (!sel) return;

  // ---- In-launch select (see the comment above FusedArgs) ----
  const int G = groups_row;
  const int lds_base = out_n - lds_n;
  uint32_t* const s_lh = reinterpret_cast<uint32_t*>(fused_smem);  // pass histogram (q operands are done)
  int* const s_off = reinterpret_cast<int*>(s_table);              // [G] offsets of the row's lists
  int* const s_dec = s_misc + 20;  // [20..25] a round's decision; s_misc[26..31] scratch
  uint32_t* const failw = rowc + kFailWord;
  auto key_at = [&](int i) -> uint32_t {  // exact score key of entry i of this workgroup's list
    const float sc = (i >= lds_base) ? s_score[i - lds_base] : __uint_as_float(ld_agent(a.cand_score + out0 + i));
    return score_key(sc + 0.0f);
  };
  auto tok_at = [&](int i) -> int64_t {  // its token
    return (i >= lds_base) ? static_cast<int64_t>(seg0 + s_list[i - lds_base])
                           : static_cast<int64_t>(static_cast<int32_t>(ld_agent(a.cand_idx + out0 + i)));
  };
  bool failed = bound_gave_up;

  // Exchange: once every workgroup of the row has written its list and count
  // (agent-scope stores, completed before it arrives), each reads the counts.
  handoff_wait();
  __syncthreads();
  if (tid == 0) {
    bool all_in = false;
    if (!failed) {
      const uint32_t target = 2u * static_cast<uint32_t>(G);
      const uint32_t before = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      all_in = (before & 0xffffu) + 1u >= target;
      for (int spins = 0; !all_in && spins < a.spin_limit; ++spins) {
        __builtin_amdgcn_s_sleep(4);
        all_in = (ld_agent(arrive) & 0xffffu) >= target;
        if (!all_in && ld_agent(failw) != 0) break;
      }
    }
    s_misc[16] = all_in ? 1 : 0;
    s_misc[17] = 0;
  }
  __syncthreads();
  failed = s_misc[16] == 0;
  int n_row = 0, max_list = 0;
  if (!failed) {
    const int cy = (tid < G) ? static_cast<int>(ld_agent(a.cand_count + static_cast<int64_t>(t) * a.groups + tid)) : 0;
    if (tid == 0) s_misc[27] = 0;
    const int ex = block_scan_excl<kThreads>(cy, s_misc, n_row);
    if (tid < G) s_off[tid] = ex;
    if (tid == x && cy != out_n) s_misc[17] = 1;  // (a count that is not this call's)
    int cm = cy;
    for (int off = 32; off > 0; off >>= 1) cm = max(cm, __shfl_xor(cm, off));
    if ((tid & 63) == 0 && cm > 0) atomicMax(s_misc + 27, cm);
    __syncthreads();
    failed = s_misc[17] != 0;
    max_list = s_misc[27];
  }

  const SelRow so(a, t);  // (its loads in flight during the select)

  // Local select: with the row's candidates fitting LDS beside this
  // workgroup's list, every workgroup loads all their keys (in list order, so
  // segment by segment) and finds the threshold itself, histogram passes over
  // LDS; its offsets count the keys of the segments before its own.  No
  // further exchange.
  // (the keys go after this workgroup's list tokens, over its scores; the
  // choice is the same in every workgroup of the row: from the counts, every
  // list in LDS and the longest beside all the keys)
  const bool local = !failed && max_list <= Lay::kList && max_list + n_row <= 2 * Lay::kList;
  uint32_t* const s_key = reinterpret_cast<uint32_t*>(s_list + out_n);  // [n_row]
  uint32_t thr_lo = 0, thr_hi = 0;  // selected: keys >= thr_hi, then ties in [thr_lo, thr_hi)
  int need = 0, gt_before = 0, eq_before = 0, my0 = 0;
  const int64_t row0 = static_cast<int64_t>(t) * f.max_len;
  const int64_t seg_tokens = static_cast<int64_t>(per_group) * kPageTokens;
  if (local) {
    my0 = s_off[x];
    __syncthreads();  // the scores' LDS becomes the keys
    constexpr int kKeys = 8;  // loads in flight per thread
    uint32_t kmax = 0u;       // the row's largest key
    if (tid == 0) s_misc[26] = 0;
    // the lists' offsets in scalar registers when the row has at most
    // kRegLists workgroups (past G: no key is that far)
    constexpr int kRegLists = 8;
    int offr[kRegLists];
#pragma unroll
    for (int i = 0; i < kRegLists; ++i) offr[i] = __builtin_amdgcn_readfirstlane(i < G ? s_off[i] : INT_MAX);
    for (int p0 = 0; p0 < n_row; p0 += kKeys * kThreads) {
      float v[kKeys];
#pragma unroll
      for (int j = 0; j < kKeys; ++j) {
        const int p = p0 + tid + j * kThreads;
        v[j] = 0.0f;
        if (p < n_row) {
          // the last list with its offset <= p (empty lists are skipped)
          int y = 0, off = offr[0];
          if (G <= kRegLists) {
#pragma unroll
            for (int i = 1; i < kRegLists; ++i)
              if (offr[i] <= p) {
                y = i;
                off = offr[i];
              }
          } else {
            int hi = G - 1;
            while (y < hi) {
              const int mid = (y + hi + 1) >> 1;
              if (s_off[mid] <= p) y = mid;
              else hi = mid - 1;
            }
            off = s_off[y];
          }
          v[j] = __uint_as_float(ld_agent(a.cand_score + row0 + y * seg_tokens + (p - off)));
        }
      }
#pragma unroll
      for (int j = 0; j < kKeys; ++j) {
        const int p = p0 + tid + j * kThreads;
        if (p < n_row) {
          const uint32_t key = score_key(v[j] + 0.0f);
          s_key[p] = key;
          kmax = max(kmax, key);
        }
      }
    }
    for (int off = 32; off > 0; off >>= 1) kmax = max(kmax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmax), off)));
    if ((tid & 63) == 0) atomicMax(reinterpret_cast<uint32_t*>(s_misc + 26), kmax);
    __syncthreads();
    kmax = static_cast<uint32_t>(s_misc[26]);
    uint32_t lo = bin << (32 - kHistBits);  // the k-th largest exact key is >= lo
    // first pass: [lo, lo + 2^22) in bins of 2^10 keys, or wider bins when
    // the keys reach beyond that (so the pass always holds the threshold)
    int shift = 10, nbins = kHistBins;
    if (kmax >= lo) {
      const uint32_t span = (kmax - lo) >> 10;
      if (span >= static_cast<uint32_t>(kHistBins)) shift = 10 + (32 - __clz(static_cast<int>(span))) - kHistBits;
    }
    for (bool first = true;; first = false) {
      for (int i = tid; i <= kHistBins; i += kThreads) s_lh[i] = 0;
      __syncthreads();
      for (int p0 = 0; p0 < n_row; p0 += kThreads) {
        const int p = p0 + tid;
        int b = -1;
        if (p < n_row) {
          const uint32_t key = s_key[p];
          if (key >= lo) {
            const uint32_t d = (key - lo) >> shift;
            b = (d >= static_cast<uint32_t>(nbins)) ? kHistBins : static_cast<int>(d);
          }
        }
        hist_add_ties(s_lh, b);
      }
      __syncthreads();
      int fb, above_f, h;
      find_threshold_bin<kThreads>([&](int bb) { return static_cast<int>(s_lh[bb]); }, nbins,
                                   static_cast<int>(s_lh[kHistBins]), f.k, s_misc, fb, above_f, h);
      uint32_t pd[5];
      const int kind = select_decision(first, lo, shift, f.k, fb, above_f, h, pd);
      if (kind == 2) {
        thr_lo = pd[0];
        thr_hi = pd[1];
        need = static_cast<int>(pd[2]);
        break;
      }
      if (kind != 1) {  // (cannot happen: the keys are the row's candidates, all exact)
        failed = true;
        break;
      }
      lo = pd[0];
      shift = static_cast<int>(pd[1]);
      nbins = static_cast<int>(pd[2]);
    }
    int gtc = 0, eqc = 0;
    for (int p = tid; p < my0; p += kThreads) {
      const uint32_t key = s_key[p];
      gtc += key >= thr_hi;
      eqc += (key >= thr_lo) && (key < thr_hi);
    }
    (void)block_scan_excl<kThreads>(gtc, s_misc, gt_before);
    (void)block_scan_excl<kThreads>(eqc, s_misc, eq_before);
  }

  // Rows with more candidates than LDS holds: rounds over the workgroups,
  // each closed by its last arriver, which publishes the decision.
  int rnd = 2;  // round 0 was the bound, round 1 the exchange
  if (!failed && !local) {
    uint32_t lo = bin << (32 - kHistBits);
    int shift = 10, nbins = kHistBins;
    int expect = -1;  // keys >= lo in the row, when known
    int gt_total = 0, eq_total = 0;
    constexpr int kPer = (kHistBins + kThreads - 1) / kThreads;  // bins per thread, scanned from the top down
    while (!failed) {
      uint32_t* const hr = rowc + (rnd & 1) * kHistSlot;
      uint32_t* const dec = rowc + kDecWords + 8 * rnd;
      for (int i = tid; i <= kHistBins; i += kThreads) s_lh[i] = 0;
      __syncthreads();
      int mine = 0;
      for (int i0 = 0; i0 < out_n; i0 += kThreads) {
        const int i = i0 + tid;
        int b = -1;
        if (i < out_n) {
          const uint32_t key = key_at(i);
          if (key >= lo) {
            const uint32_t d = (key - lo) >> shift;
            b = (d >= static_cast<uint32_t>(nbins)) ? kHistBins : static_cast<int>(d);  // kHistBins: above
            ++mine;
          }
        }
        hist_add_ties(s_lh, b);
      }
      int counted;
      (void)block_scan_excl<kThreads>(mine, s_misc, counted);  // (its barriers also complete s_lh)
      for (int i = tid; i <= kHistBins; i += kThreads) {
        const uint32_t v = s_lh[i];
        if (v) atomicAdd(hr + i, v);
      }
      if (tid == 0 && counted) atomicAdd(hr + kHistBins + 1, static_cast<uint32_t>(counted));
      handoff_wait();
      __syncthreads();
      if (tid == 0) {
        const uint32_t before = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_misc[16] = ((before & 0xffffu) + 1u == static_cast<uint32_t>((rnd + 1) * G)) ? 1 : 0;
      }
      __syncthreads();
      if (s_misc[16]) {
        // Last to arrive: every workgroup's adds completed before it arrived.
        // The bins and the above counter must sum to the keys counted (and to
        // the keys the previous decision expects at or above lo).
        bool ok = false;
        int above = 0;
        for (int attempt = 0;; ++attempt) {
          if (tid == 0) {
            s_misc[26] = static_cast<int>(ld_agent(hr + kHistBins));
            s_misc[27] = static_cast<int>(ld_agent(hr + kHistBins + 1));
          }
          const int rb0 = kPer * tid;
          int sum = 0;
#pragma unroll
          for (int j = 0; j < kPer; ++j)
            sum += (rb0 + j < nbins) ? static_cast<int>(ld_agent(hr + (nbins - 1 - (rb0 + j)))) : 0;
          int total;
          (void)block_scan_excl<kThreads>(sum, s_misc, total);
          above = s_misc[26];
          ok = (total + above == s_misc[27]) && (expect < 0 || s_misc[27] == expect);
          __syncthreads();  // before s_misc[26..27] are written again
          if (ok || attempt == kHistRereads) break;
          __builtin_amdgcn_s_sleep(8);
        }
        int fb = -1, above_f = 0, h = 0;
        if (ok)
          find_threshold_bin<kThreads>([&](int bb) { return static_cast<int>(ld_agent(hr + bb)); }, nbins, above,
                                       f.k, s_misc, fb, above_f, h);
        if (tid == 0) {
          uint32_t pd[5] = {0u, 0u, 0u, 0u, 0u};
          int kind = 3;
          if (!ok) atomicAdd(a.timeouts + 1, 1u);
          else kind = select_decision(rnd == 2, lo, shift, f.k, fb, above_f, h, pd);
          if (kind == 2) {  // the final decision carries the row's totals of greater and tied keys
            pd[3] = static_cast<uint32_t>(pd[0] == pd[1] ? f.k : above_f);
            pd[4] = static_cast<uint32_t>(pd[0] == pd[1] ? 0 : h);
          }
          s_dec[0] = kind;
#pragma unroll
          for (int w = 0; w < 5; ++w) {
            s_dec[1 + w] = static_cast<int>(pd[w]);
            st_agent(dec + 1 + w, pd[w]);
          }
          handoff_wait();  // the payload before the word that announces it
          st_agent(dec, static_cast<uint32_t>(kind));
        }
        // leave the histogram zero (everyone has arrived; nobody reads it again)
        for (int i = tid; i < nbins; i += kThreads) st_agent(hr + i, 0u);
        if (tid == 0) {
          st_agent(hr + kHistBins, 0u);
          st_agent(hr + kHistBins + 1, 0u);
        }
      } else if (tid == 0) {
        uint32_t v = 0;
        for (int spins = 0; spins < a.spin_limit; ++spins) {
          v = ld_agent(dec);
          if (v != 0 || ld_agent(failw) != 0) break;
          __builtin_amdgcn_s_sleep(4);
        }
        s_dec[0] = (v != 0) ? static_cast<int>(v) : 3;
        if (v != 0)
#pragma unroll
          for (int w = 0; w < 5; ++w) s_dec[1 + w] = static_cast<int>(ld_agent(dec + 1 + w));
      }
      __syncthreads();
      const int kind = s_dec[0];
      if (kind == 2) {
        thr_lo = static_cast<uint32_t>(s_dec[1]);
        thr_hi = static_cast<uint32_t>(s_dec[2]);
        need = s_dec[3];
        gt_total = s_dec[4];
        eq_total = s_dec[5];
      } else if (kind == 1) {
        lo = static_cast<uint32_t>(s_dec[1]);
        shift = s_dec[2];
        nbins = s_dec[3];
        expect = s_dec[4];
      } else {
        failed = true;
      }
      __syncthreads();  // s_dec and s_misc are reused
      if (kind != 1) break;
      if (++rnd >= kSelRounds) failed = true;  // (at most four histogram rounds are ever decided)
    }

    // Records round: this workgroup's (greater, tied) counts; its offsets
    // are the sums over the row's earlier workgroups.
    uint32_t* const rec = rowc + kRecWords;
    if (!failed) {
      int gt = 0, eq = 0;
      for (int i = tid; i < out_n; i += kThreads) {
        const uint32_t key = key_at(i);
        gt += key >= thr_hi;
        eq += (key >= thr_lo) && (key < thr_hi);
      }
      int gt_x, eq_x;
      (void)block_scan_excl<kThreads>(gt, s_misc, gt_x);
      (void)block_scan_excl<kThreads>(eq, s_misc, eq_x);
      if (tid == 0) {
        st_agent(rec + 2 * x, static_cast<uint32_t>(gt_x));
        st_agent(rec + 2 * x + 1, static_cast<uint32_t>(eq_x));
        handoff_wait();
        const uint32_t target = static_cast<uint32_t>((rnd + 2) * G);
        const uint32_t before = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool all_in = (before & 0xffffu) + 1u >= target;
        for (int spins = 0; !all_in && spins < a.spin_limit; ++spins) {
          __builtin_amdgcn_s_sleep(4);
          all_in = (ld_agent(arrive) & 0xffffu) >= target;
          if (!all_in && ld_agent(failw) != 0) break;
        }
        s_misc[16] = all_in ? 1 : 0;
      }
      __syncthreads();
      if (!s_misc[16]) failed = true;
      for (int attempt = 0; !failed; ++attempt) {
        int gy = 0, ey = 0;
        if (tid < G) {
          gy = static_cast<int>(ld_agent(rec + 2 * tid));
          ey = static_cast<int>(ld_agent(rec + 2 * tid + 1));
        }
        int gsum, esum;
        const int gex = block_scan_excl<kThreads>(gy, s_misc, gsum);
        const int eex = block_scan_excl<kThreads>(ey, s_misc, esum);
        if (tid == x) {
          s_misc[28] = gex;
          s_misc[29] = eex;
        }
        __syncthreads();
        gt_before = s_misc[28];
        eq_before = s_misc[29];
        __syncthreads();
        if (gsum == gt_total && esum == eq_total) break;
        if (attempt == kHistRereads) failed = true;
        __builtin_amdgcn_s_sleep(8);
      }
    }
  }

  // Ordered output of this segment's selected tokens: a selected key's
  // position is (greater keys before it) + min(tied keys before it, need).
  if (!failed) {
    auto okey = [&](int i) -> uint32_t { return local ? s_key[my0 + i] : key_at(i); };
    auto otok = [&](int i) -> int64_t { return local ? static_cast<int64_t>(seg0 + s_list[i]) : tok_at(i); };
    auto emit = [&](int pos, int64_t tok) { so.emit_paged(pos, tok, s_pages[(tok - seg0) >> 6]); };
    int gt_base = gt_before, eq_base = eq_before;
    for (int i0 = 0; i0 < out_n; i0 += kThreads * 8) {
      const int start = i0 + tid * 8;
      uint32_t gtm = 0, eqm = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (start + j < out_n) {
          const uint32_t key = okey(start + j);
          if (key >= thr_hi) gtm |= 1u << j;
          else if (key >= thr_lo) eqm |= 1u << j;
        }
      }
      int packed_total;
      const int packed = block_scan_excl<kThreads>(__popc(gtm) | (__popc(eqm) << 16), s_misc, packed_total);
      int gb = gt_base + (packed & 0xffff), eb = eq_base + (packed >> 16);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (gtm & (1u << j)) {
          const int pos = gb + min(eb, need);
          if (pos < f.k) emit(pos, otok(start + j));
          ++gb;
        } else if (eqm & (1u << j)) {
          if (eb < need && gb + eb < f.k) emit(gb + eb, otok(start + j));
          ++eb;
        }
      }
      gt_base += packed_total & 0xffff;
      eq_base += packed_total >> 16;
    }
  }

  // Depart.  The last workgroup of the row to depart clears the row's words
  // and, if any wait of the row gave up, selects over the row's lists alone.
  handoff_wait();
  __syncthreads();
  if (tid == 0) {
    if (failed) {
      st_agent(failw, 1u);
      handoff_wait();
    }
    const uint32_t before = __hip_atomic_fetch_add(arrive, 1u << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_misc[16] = ((before >> 16) + 1u == static_cast<uint32_t>(G)) ? 1 : 0;
    s_misc[17] = (s_misc[16] && ld_agent(failw) != 0) ? 1 : 0;
  }
  __syncthreads();
  if (!s_misc[16]) return;
  if (s_misc[17]) {
    if (tid == 0) atomicAdd(a.timeouts + 2, 1u);
    // Every workgroup wrote its list and count before it departed.  Radix
    // select (4 passes of 8 bits) over the lists, then the ordered output.
    int* const s_cnt = s_off;
    for (int y = tid; y < G; y += kThreads)
      s_cnt[y] = static_cast<int>(ld_agent(a.cand_count + static_cast<int64_t>(t) * a.groups + y));
    __syncthreads();
    int ncand = 0;
    for (int y = 0; y < G; ++y) ncand += s_cnt[y];
    auto gkey = [&](int y, int i) -> uint32_t {
      return score_key(__uint_as_float(ld_agent(a.cand_score + row0 + y * seg_tokens + i)) + 0.0f);
    };
    uint32_t prefix = 0u, mask = 0u;
    int remaining = f.k;
    const bool all = ncand <= f.k;
    if (!all) {
      for (int sh = 24; sh >= 0; sh -= 8) {
        for (int b = tid; b < 256; b += kThreads) s_lh[b] = 0;
        __syncthreads();
        for (int y = 0; y < G; ++y)
          for (int i = tid; i < s_cnt[y]; i += kThreads) {
            const uint32_t key = gkey(y, i);
            if ((key & mask) == prefix) atomicAdd(&s_lh[(key >> sh) & 255u], 1u);
          }
        __syncthreads();
        int above;
        const int b = find_bin<kThreads>(s_lh, 256, remaining, s_misc, s_misc + 28, above);
        remaining -= above;
        prefix |= static_cast<uint32_t>(b) << sh;
        mask |= 255u << sh;
      }
    }
    int gt_base = 0, eq_base = 0;
    for (int y = 0; y < G; ++y)
      for (int i0 = 0; i0 < s_cnt[y]; i0 += kThreads * 4) {
        const int start = i0 + tid * 4;
        uint32_t gtm = 0, eqm = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (start + j < s_cnt[y]) {
            if (all) {
              gtm |= 1u << j;
            } else {
              const uint32_t key = gkey(y, start + j);
              if (key > prefix) gtm |= 1u << j;
              else if (key == prefix) eqm |= 1u << j;
            }
          }
        }
        int packed_total;
        const int packed = block_scan_excl<kThreads>(__popc(gtm) | (__popc(eqm) << 16), s_misc, packed_total);
        int gb = gt_base + (packed & 0xffff), eb = eq_base + (packed >> 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bool g_ = gtm & (1u << j), e_ = eqm & (1u << j);
          if (!g_ && !e_) continue;
          const int64_t tok = static_cast<int32_t>(ld_agent(a.cand_idx + row0 + y * seg_tokens + start + j));
          if (g_) {
            const int pos = gb + min(eb, remaining);
            if (pos < f.k) so.emit(pos, tok);
            ++gb;
          } else {
            if (eb < remaining && gb + eb < f.k) so.emit(gb + eb, tok);
            ++eb;
          }
        }
        gt_base += packed_total & 0xffff;
        eq_base += packed_total >> 16;
      }
    for (int i = gt_base + min(eq_base, all ? 0 : remaining) + tid; i < f.k; i += kThreads) so.emit(i, -1);
    // both histograms may hold adds of rounds that were never closed
    for (int i = tid; i < 2 * kHistSlot; i += kThreads) st_agent(rowc + i, 0u);
  }
  for (int i = tid; i < 8 * kSelRounds; i += kThreads) st_agent(rowc + kDecWords + i, 0u);
  for (int i = tid; i < 2 * G; i += kThreads) st_agent(rowc + kRecWords + i, 0u);
  if (tid == 0) {
    st_agent(failw, 0u);
    st_agent(arrive, 0u);
  }
}

// ---------------------------------------------------------------------------
// Exact select: top-k by (score desc, index asc), written ascending, -1 padded.
// Sources: an implicit range of scores, or per-chunk candidate lists that are
// concatenated (in chunk order) into LDS, or -- when they do not fit -- into a
// contiguous global staging row.
// ---------------------------------------------------------------------------
constexpr int kSelThreads = 1024;
constexpr int kSelLds = 16384;
constexpr int kSelPerThread = 8;

struct SelectArgs {
  const float* scores;       // implicit mode: [T, scores_stride]
  int64_t scores_stride;
  const int32_t* lengths;    // implicit mode: [T]
  const float* cand_score;   // chunk mode: [T, max_len]
  const int32_t* cand_idx;
  const int32_t* cand_count; // [T, chunks]
  int32_t chunks;
  float* stage_score;        // chunk mode spill: [T, max_len]
  int32_t* stage_idx;
  int32_t* out;              // [T, out_stride]
  int64_t out_stride;
  int32_t k;
  int32_t max_len;
  int32_t seg_groups;        // chunk mode: 0 = lists of kChunk-token chunks, else of
                             // filter_verify_kernel segments (`seg_groups` per row)
  // Optional merged output (merge_swa_topk of the result): [T, merged_stride]
  // rows of merged_width = [top-k[:n] | seq-w .. seq-1 | -1 ...] with
  // seq = positions[t] + 1, n = min(max(seq - window, 0), k), w = min(seq, window).
  int32_t* merged;
  int64_t merged_stride;
  int32_t merged_width;
  const int64_t* positions;
  int32_t window;
  // With slot_bt non-null the merged entries are cache slots:
  // slot_bt[req[t]][i >> 6] * 64 + (i & 63), -1 when unmapped.
  const int32_t* slot_bt;
  int64_t slot_bt_stride;
  const int32_t* slot_req;
  int64_t num_pages;
};

constexpr int kSelMaxChunks = 4096;  // up to 8M-token rows

struct SelectSmem {
  uint32_t key[kSelLds];
  int32_t idx[kSelLds];
  uint32_t hist[2048];
  int off[kSelMaxChunks + 1];
  int wave[kSelThreads / 64];
  uint32_t wmin[kSelThreads / 64], wmax[kSelThreads / 64];  // per-wave key range
  int res[2];
  int cnt;
  uint32_t pmin, pmax;  // range of the current pass's keys
};

__global__ void __launch_bounds__(kSelThreads) topk_select_kernel(SelectArgs a) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  SelectSmem& sm = *reinterpret_cast<SelectSmem*>(smem_raw);
  uint32_t* s_hist = sm.hist;
  uint32_t* s_key = sm.key;
  int32_t* s_idx = sm.idx;
  int* s_wave = sm.wave;
  int* s_res = sm.res;
  const int tid = threadIdx.x;
  const int t = blockIdx.x;
  const int k = a.k;
  int32_t* out = a.out + static_cast<int64_t>(t) * a.out_stride;
  int32_t* merged = a.merged ? a.merged + static_cast<int64_t>(t) * a.merged_stride : nullptr;
  int64_t seq = 0, m_topk = 0;  // merged: sequence length, top-k entries taken
  const int32_t* mbt = nullptr;
  if (merged) {
    seq = a.positions[t] + 1;
    m_topk = min(min(max(seq - a.window, static_cast<int64_t>(0)), static_cast<int64_t>(k)),
                 static_cast<int64_t>(a.merged_width));
    if (a.slot_bt) mbt = a.slot_bt + static_cast<int64_t>(a.slot_req[t]) * a.slot_bt_stride;
  }
  // Slot conversion reads the row's first kSelBtPages block-table entries
  // from LDS (loaded now, stored over the histogram once the passes are done).
  constexpr int kSelBtPages = 2048;
  const int64_t bt_lds = mbt ? min(a.slot_bt_stride, static_cast<int64_t>(kSelBtPages)) : 0;
  int32_t btv[kSelBtPages / kSelThreads];
#pragma unroll
  for (int j = 0; j < kSelBtPages / kSelThreads; ++j) {
    const int pg = tid + kSelThreads * j;
    btv[j] = (pg < bt_lds) ? mbt[pg] : -1;
  }
  auto to_merged = [&](int64_t i) -> int32_t {  // token index -> merged entry
    if (i < 0 || mbt == nullptr) return static_cast<int32_t>(i);
    if ((i >> 6) >= a.slot_bt_stride) return -1;
    const int64_t page = ((i >> 6) < bt_lds) ? static_cast<int64_t>(static_cast<int32_t>(s_hist[i >> 6])) : mbt[i >> 6];
    return (page >= 0 && page < a.num_pages) ? static_cast<int32_t>(page * kPageTokens + (i & 63)) : -1;
  };
  auto emit = [&](int pos, int32_t v) {
    out[pos] = v;
    if (merged && pos < m_topk) merged[pos] = to_merged(v);
  };

  // gather the elements; lo / hi track the range of the keys put in LDS
  uint32_t lo = 0xffffffffu, hi = 0u;
  int n;
  const float* gsc = nullptr;     // global scores (implicit mode or spilled lists)
  const int32_t* gidx = nullptr;  // global indices (spilled lists); null = implicit
  bool in_lds;
  if (a.cand_count == nullptr) {
    n = max(0, min(a.lengths[t], a.max_len));
    gsc = a.scores + static_cast<int64_t>(t) * a.scores_stride;
    in_lds = n <= kSelLds;
    if (in_lds)
      for (int i = tid; i < n; i += kSelThreads) {
        const uint32_t key = score_key(gsc[i] + 0.0f);  // -0 ties with +0
        s_key[i] = key;
        s_idx[i] = i;
        lo = min(lo, key);
        hi = max(hi, key);
      }
  } else {
    const int32_t* cnt = a.cand_count + static_cast<int64_t>(t) * a.chunks;
    // exclusive offsets of the chunk lists
    int base = 0;
    for (int c0 = 0; c0 < a.chunks; c0 += kSelThreads) {
      const int c = c0 + tid;
      const int v = (c < a.chunks) ? cnt[c] : 0;
      int total;
      const int ex = block_scan_excl<kSelThreads>(v, s_wave, total);
      if (c < a.chunks) sm.off[c] = base + ex;
      base += total;
    }
    n = base;
    if (tid == 0) sm.off[a.chunks] = n;
    __syncthreads();
    in_lds = n <= kSelLds;
    const int64_t row = static_cast<int64_t>(t) * a.max_len;
    const int64_t seg = a.seg_groups > 0
                            ? kPageTokens * fused_group_pages(max(0, min(a.lengths[t], a.max_len)), a.seg_groups)
                            : kChunk;  // tokens per list slice
    float* st_sc = a.stage_score + row;
    int32_t* st_ix = a.stage_idx + row;
    // Position p of the concatenation lies in list c = the last with
    // off[c] <= p (binary search; empty lists are skipped by construction).
    // Every thread copies kGather positions per round, loads issued together.
    auto list_of = [&](int p) -> int {
      int lo = 0, hi = a.chunks - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sm.off[mid] <= p) lo = mid;
        else hi = mid - 1;
      }
      return lo;
    };
    constexpr int kGather = 4;
    for (int p0 = 0; p0 < n; p0 += kGather * kSelThreads) {
      float sv[kGather];
      int32_t iv[kGather];
#pragma unroll
      for (int q = 0; q < kGather; ++q) {
        const int p = p0 + q * kSelThreads + tid;
        sv[q] = 0.0f;
        iv[q] = 0;
        if (p < n) {
          const int c = list_of(p);
          const int64_t src = row + c * seg + (p - sm.off[c]);
          sv[q] = a.cand_score[src];
          iv[q] = a.cand_idx[src];
        }
      }
#pragma unroll
      for (int q = 0; q < kGather; ++q) {
        const int p = p0 + q * kSelThreads + tid;
        if (p >= n) continue;
        if (in_lds) {
          const uint32_t key = score_key(sv[q] + 0.0f);
          s_key[p] = key;
          s_idx[p] = iv[q];
          lo = min(lo, key);
          hi = max(hi, key);
        } else {
          st_sc[p] = sv[q];
          st_ix[p] = iv[q];
        }
      }
    }
    if (!in_lds) {
      __threadfence_block();
      gsc = st_sc;
      gidx = st_ix;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    lo = min(lo, static_cast<uint32_t>(__shfl_xor(static_cast<int>(lo), off)));
    hi = max(hi, static_cast<uint32_t>(__shfl_xor(static_cast<int>(hi), off)));
  }
  if ((tid & 63) == 0) {
    sm.wmin[tid >> 6] = lo;
    sm.wmax[tid >> 6] = hi;
  }
  __syncthreads();
  auto key_at = [&](int i) -> uint32_t { return in_lds ? s_key[i] : score_key(gsc[i] + 0.0f); };
  auto idx_at = [&](int i) -> int32_t { return in_lds ? s_idx[i] : (gidx ? gidx[i] : i); };

  uint32_t kstar = 0;
  int need = n;
  if (n > k) {
    // Bits every key shares need no pass: with the keys in LDS their range
    // is known, so the first pass splits the bits just below the common
    // prefix (where the candidates, all near the threshold, differ).
    uint32_t kmin = 0u, kmax = 0xffffffffu;
    if (in_lds) {
      kmin = 0xffffffffu;
      kmax = 0u;
#pragma unroll
      for (int w = 0; w < kSelThreads / 64; ++w) {
        kmin = min(kmin, sm.wmin[w]);
        kmax = max(kmax, sm.wmax[w]);
      }
    }
    const int common = (kmin == kmax) ? 32 : __clz(static_cast<int>(kmin ^ kmax));
    uint32_t mask = common == 0 ? 0u : (common == 32 ? 0xffffffffu : 0xffffffffu << (32 - common));
    uint32_t prefix = kmin & mask;
    int remaining = k;
    int top = 32 - common;  // bits [0, top) are still open
    bool first = true;      // the first pass's key range is [kmin, kmax]
    while (top > 0) {
      const int width = min(11, top);
      const int sh = top - width;
      const int nb = 1 << width;
      for (int b = tid; b < 2048; b += kSelThreads) s_hist[b] = 0;
      if (tid == 0) {
        sm.pmin = 0xffffffffu;
        sm.pmax = 0u;
      }
      __syncthreads();
      uint32_t plo = 0xffffffffu, phi = 0u;  // range of the keys under the prefix
      for (int i0 = 0; i0 < n; i0 += kSelThreads * kSelPerThread) {
#pragma unroll
        for (int j = 0; j < kSelPerThread; ++j) {
          const int i = i0 + j * kSelThreads + tid;
          int bin = -1;
          if (i < n) {
            const uint32_t key = key_at(i);
            if ((key & mask) == prefix) {
              bin = static_cast<int>((key >> sh) & static_cast<uint32_t>(nb - 1));
              plo = min(plo, key);
              phi = max(phi, key);
            }
          }
          hist_add_ties(s_hist, bin);
        }
      }
      if (!first) {
        for (int off = 32; off > 0; off >>= 1) {
          plo = min(plo, static_cast<uint32_t>(__shfl_xor(static_cast<int>(plo), off)));
          phi = max(phi, static_cast<uint32_t>(__shfl_xor(static_cast<int>(phi), off)));
        }
        if ((tid & 63) == 0) {
          atomicMin(&sm.pmin, plo);
          atomicMax(&sm.pmax, phi);
        }
      }
      __syncthreads();
      if (!first && sm.pmin == sm.pmax) {  // every key left is the same: it is the threshold
        prefix = sm.pmin;
        break;
      }
      first = false;
      int above;
      const int bin = find_bin<kSelThreads>(s_hist, nb, remaining, s_wave, s_res, above);
      remaining -= above;
      prefix |= static_cast<uint32_t>(bin) << sh;
      mask |= static_cast<uint32_t>(nb - 1) << sh;
      top = sh;
      if (top == 0) break;
      const int m = static_cast<int>(s_hist[bin]);  // keys sharing the threshold's prefix
      __syncthreads();                              // before s_hist is reused
      if (m <= kSelThreads) {
        // Few keys share the prefix: rank them directly.  The threshold is
        // the key with (count above) < remaining <= (count above) + (count
        // equal).  The keys are collected with one LDS atomic per wave.
        if (tid == 0) sm.cnt = 0;
        __syncthreads();
        uint32_t* s_small = s_hist;  // 2048 entries, 16-byte aligned
        const int lane = tid & 63;
        for (int i0 = 0; i0 < n; i0 += kSelThreads * kSelPerThread) {
#pragma unroll
          for (int j = 0; j < kSelPerThread; ++j) {
            const int i = i0 + j * kSelThreads + tid;
            uint32_t key = 0;
            bool hit = false;
            if (i < n) {
              key = key_at(i);
              hit = (key & mask) == prefix;
            }
            const uint64_t bal = __ballot(hit);
            if (bal != 0) {  // wave-uniform
              const int leader = static_cast<int>(__builtin_ctzll(bal));
              int base = 0;
              if (lane == leader) base = atomicAdd(&sm.cnt, static_cast<int>(__popcll(bal)));
              base = __shfl(base, leader);
              if (hit) s_small[base + static_cast<int>(__popcll(bal & ((uint64_t{1} << lane) - 1)))] = key;
            }
          }
        }
        __syncthreads();
        if (tid < m) {
          const uint32_t mine = s_small[tid];
          int gt = 0, eq = 0;
          auto rank4 = [&](uint4 v) {
            gt += (v.x > mine) + (v.y > mine) + (v.z > mine) + (v.w > mine);
            eq += (v.x == mine) + (v.y == mine) + (v.z == mine) + (v.w == mine);
          };
          int j = 0;
#pragma unroll 4
          for (; j + 8 <= m; j += 8) {  // broadcast reads, two 16-byte loads per step
            rank4(*reinterpret_cast<const uint4*>(s_small + j));
            rank4(*reinterpret_cast<const uint4*>(s_small + j + 4));
          }
          for (; j < m; ++j) {
            const uint32_t o = s_small[j];
            gt += o > mine;
            eq += o == mine;
          }
          if (gt < remaining && remaining <= gt + eq) {  // every such thread holds the same key
            s_res[0] = static_cast<int>(mine);
            s_res[1] = remaining - gt;
          }
        }
        __syncthreads();
        prefix = static_cast<uint32_t>(s_res[0]);
        remaining = s_res[1];
        break;
      }
    }
    kstar = prefix;
    need = remaining;  // threshold-valued elements to take, lowest index first
  }

  if (mbt) {  // every pass is done with s_hist (each ended with a barrier)
#pragma unroll
    for (int j = 0; j < kSelBtPages / kSelThreads; ++j) s_hist[tid + kSelThreads * j] = static_cast<uint32_t>(btv[j]);
    __syncthreads();
  }
  // Ordered compaction: thread owns kSelPerThread consecutive elements.  An
  // element's output position is (greater keys before it) + min(threshold
  // keys before it, need); both counts come from one scan, packed as
  // gt | eq << 16 (each below 2^14 per round).
  int gt_base = 0, eq_base = 0;
  for (int i0 = 0; i0 < n; i0 += kSelThreads * kSelPerThread) {
    const int start = i0 + tid * kSelPerThread;
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < kSelPerThread; ++j) {
      const int i = start + j;
      if (i < n) {
        if (n <= k) {
          gt |= 1u << j;
        } else {
          const uint32_t key = key_at(i);
          if (key > kstar) gt |= 1u << j;
          else if (key == kstar) eq |= 1u << j;
        }
      }
    }
    int packed_total;
    const int packed = block_scan_excl<kSelThreads>(__popc(gt) | (__popc(eq) << 16), s_wave, packed_total);
    int gt_before = gt_base + (packed & 0xffff), eq_before = eq_base + (packed >> 16);
#pragma unroll
    for (int j = 0; j < kSelPerThread; ++j) {
      if (gt & (1u << j)) {
        const int pos = gt_before + min(eq_before, need);
        if (pos < k) emit(pos, idx_at(start + j));
        ++gt_before;
      } else if (eq & (1u << j)) {
        if (eq_before < need) {
          const int pos = gt_before + eq_before;
          if (pos < k) emit(pos, idx_at(start + j));
        }
        ++eq_before;
      }
    }
    gt_base += packed_total & 0xffff;
    eq_base += packed_total >> 16;
  }
  for (int i = gt_base + min(eq_base, need) + tid; i < k; i += kSelThreads) emit(i, -1);
  if (merged) {
    const int64_t w = min(seq, static_cast<int64_t>(a.window));
    for (int64_t c = m_topk + tid; c < a.merged_width; c += kSelThreads)
      merged[c] = (c < m_topk + w) ? to_merged(seq - w + (c - m_topk)) : -1;
  }
}

}  // namespace ekv

using namespace ekv;

namespace {

void launch_select(const SelectArgs& a, int32_t rows, hipStream_t s) {
  const int smem = static_cast<int>(sizeof(SelectSmem));
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(topk_select_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                      smem);
  hipLaunchKernelGGL(topk_select_kernel, dim3(rows), dim3(kSelThreads), smem, s, a);
}

int num_chunks(int32_t max_len) { return max_len > 0 ? (max_len + kChunk - 1) / kChunk : 1; }

// Workgroups the filter targets in all: about three per CU, each wave
// streaming many pages.
constexpr int64_t kFilterTargetGroups = 768;
constexpr int64_t kFilterMaxWavePages = 64;

// Count slots [T, groups] of either path: chunks per row, or segments (at most
// ceil(kFilterTargetGroups / T) per row).
int64_t count_slots(int64_t T, int32_t max_len) { return T * num_chunks(max_len) + T + kFilterTargetGroups; }

// workspace: timeouts u32 [4] (cumulative), padded to 256 B | fused-path
//            counters u32 [kCounterRows, kCounterRow] (kept zero between
//            calls) | upper u16 [T,L] (4 B per entry reserved) |
//            cand_score f32 [T,L] | cand_idx i32 [T,L] | stage_score f32 [T,L] |
//            stage_idx i32 [T,L] | hist u32 [T,4096] | arrive u32 [T] |
//            kbound u32 [T] (the unfused path's, cleared per call) |
//            counts i32 [count_slots]
// The front (timeouts and counters) sits at the same offsets for every
// (T, L), so one zero-filled allocation serves calls of any shape.
struct TopkWorkspace {
  uint32_t* counters;
  uint16_t* upper;
  float* cand_score;
  int32_t* cand_idx;
  float* stage_score;
  int32_t* stage_idx;
  uint32_t* hist;
  uint32_t* arrive;
  uint32_t* kbound;
  uint32_t* timeouts;
  int32_t* counts;
};

TopkWorkspace carve(void* workspace, int64_t T, int64_t L) {
  TopkWorkspace w;
  uint8_t* base = static_cast<uint8_t*>(workspace);
  w.timeouts = reinterpret_cast<uint32_t*>(base);
  w.counters = reinterpret_cast<uint32_t*>(base + 256);
  w.upper = reinterpret_cast<uint16_t*>(base + kCounterBytes);
  w.cand_score = reinterpret_cast<float*>(base + kCounterBytes + T * L * 4);
  w.cand_idx = reinterpret_cast<int32_t*>(w.cand_score + T * L);
  w.stage_score = reinterpret_cast<float*>(w.cand_idx + T * L);
  w.stage_idx = reinterpret_cast<int32_t*>(w.stage_score + T * L);
  w.hist = reinterpret_cast<uint32_t*>(w.stage_idx + T * L);
  w.arrive = w.hist + T * kHistBins;
  w.kbound = w.arrive + T;
  w.counts = reinterpret_cast<int32_t*>(w.kbound + T);
  return w;
}

// How the filter runs for (T, max_len) on the current device.  Fused: one
// 12-wave workgroup per CU when the rows allow, else 4-wave workgroups (about
// three per CU), if the grid fits on the device at once and its LDS staging
// fits a CU.  Otherwise the filter / bound / verify kernels.  Both stages of
// a top-k call make the same plan.
struct FilterPlan {
  bool fused;
  int waves;        // fused: waves per workgroup (12 or 4)
  int groups;       // workgroups per row
  int stage_pages;  // fused: LDS pages per workgroup
  int smem;         // fused: dynamic LDS bytes
};

constexpr int kLdsPerCu = 160 * 1024;

// Workgroups of `kernel` (threads, smem) resident per CU; cached per thread.
int occupancy(const void* kernel, int threads, int smem) {
  struct Entry {
    const void* kernel;
    int smem, occ;
  };
  static thread_local Entry cache[4] = {};
  static thread_local int next = 0;
  for (const Entry& e : cache)
    if (e.kernel == kernel && e.smem == smem) return e.occ;
  int occ = 0;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, smem) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, smem) != hipSuccess)
    occ = 0;
  cache[next] = Entry{kernel, smem, occ};
  next = (next + 1) & 3;
  return occ;
}

template <int kWaves, bool kFp4>
bool plan_fused(int64_t T, int32_t max_len, int64_t pages, int cus, int64_t target_groups, FilterPlan& p) {
  if (T > kCounterRows) return false;
  const void* kernel = reinterpret_cast<const void*>(filter_verify_kernel<kWaves, kFp4>);
  int64_t groups = std::max<int64_t>(1, std::min<int64_t>((pages + kWaves - 1) / kWaves, (target_groups + T - 1) / T));
  for (int attempt = 0; attempt < 4 && groups >= 1; ++attempt) {
    const int per_group = fused_group_pages(max_len, static_cast<int>(groups));
    const int stage = std::max(4, (per_group + 3) & ~3);
    const int smem = FusedLayout<kWaves>::bytes(stage);
    if (smem > kLdsPerCu) return false;
    const int64_t capacity = static_cast<int64_t>(occupancy(kernel, 64 * kWaves, smem)) * cus;
    if (T * groups <= capacity && T * groups <= count_slots(T, max_len)) {
      p = FilterPlan{true, kWaves, static_cast<int>(groups), stage, smem};
      return true;
    }
    groups = capacity / T;
  }
  return false;
}

template <bool kFp4>
FilterPlan plan_filter(int64_t T, int32_t max_len) {
  const int64_t pages = (static_cast<int64_t>(max_len) + kPageTokens - 1) / kPageTokens;
  FilterPlan p{false, 4, 1, 0, 0};
  // unfused: about kFilterTargetGroups workgroups over T equal rows, and at
  // least enough that a max_len row takes at most kFilterMaxWavePages pages
  // per wave (rows of mixed lengths use slots in proportion to their pages);
  // a multiple of 8 (the segments are spread over the 8 XCDs)
  const int64_t g = std::max<int64_t>((kFilterTargetGroups + T - 1) / T, (pages + 4 * kFilterMaxWavePages - 1) /
                                                                             (4 * kFilterMaxWavePages));
  p.groups = static_cast<int>((std::max<int64_t>(1, std::min<int64_t>((pages + 3) / 4, g)) + 7) & ~int64_t{7});
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return p;
  if (T <= cus && plan_fused<12, kFp4>(T, max_len, pages, cus, cus, p)) return p;
  if (plan_fused<4, kFp4>(T, max_len, pages, cus, kFilterTargetGroups, p)) return p;
  return p;
}

}  // namespace

extern "C" int64_t ekv_indexer_topk_workspace_size(int32_t num_tokens, int32_t max_len) {
  if (num_tokens <= 0) return 0;
  const int64_t T = num_tokens, L = max_len > 0 ? max_len : 1;
  return kCounterBytes + T * L * 20 + T * kHistBins * 4 + T * 8 + count_slots(T, max_len) * 4 + 256;
}

extern "C" int ekv_indexer_score(const int8_t* q_digits, const float* w, const uint8_t* kcache,
                                 int64_t page_stride, int64_t num_pages, const int32_t* block_table,
                                 int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
                                 int32_t num_tokens, int32_t max_len, float* scores, int64_t scores_stride,
                                 void* stream) {
  EKV_CHECK(num_tokens >= 0 && max_len >= 0, "sizes must be >= 0");
  if (num_tokens == 0 || max_len == 0) return 0;
  EKV_CHECK(q_digits && w && kcache && block_table && req_ids && lengths && scores, "null pointer");
  EKV_CHECK(page_stride >= kPageTokens * (kIdxDim + 4) && page_stride % 16 == 0, "bad page_stride");
  EKV_CHECK(scores_stride >= max_len, "scores_stride must be >= max_len");
  EKV_CHECK(aligned16(q_digits) && aligned16(kcache), "misaligned buffers");
  ScoreArgs a{q_digits, w, kcache, page_stride, num_pages, block_table, bt_stride, req_ids, lengths,
              scores, scores_stride, max_len, nullptr, nullptr};
  dim3 grid((max_len + kScoreChunk - 1) / kScoreChunk, num_tokens);
  hipLaunchKernelGGL(score_exact_kernel<false>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_score_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                                     const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                     const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                     const int32_t* lengths, int32_t num_tokens, int32_t max_len, float* scores,
                                     int64_t scores_stride, void* stream) {
  EKV_CHECK(num_tokens >= 0 && max_len >= 0, "sizes must be >= 0");
  if (num_tokens == 0 || max_len == 0) return 0;
  EKV_CHECK(q_values && q_scales && w && kcache && block_table && req_ids && lengths && scores, "null pointer");
  EKV_CHECK(page_stride >= kPageTokens * (kFp4Row + 4) && page_stride % 16 == 0, "bad page_stride");
  EKV_CHECK(scores_stride >= max_len, "scores_stride must be >= max_len");
  EKV_CHECK(aligned16(q_values) && aligned16(kcache), "misaligned buffers");
  ScoreArgs a{nullptr, w, kcache, page_stride, num_pages, block_table, bt_stride, req_ids, lengths,
              scores, scores_stride, max_len, q_values, q_scales};
  dim3 grid((max_len + kScoreChunk - 1) / kScoreChunk, num_tokens);
  hipLaunchKernelGGL(score_exact_kernel<true>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_filter_dots(const uint8_t* q_codes, const uint8_t* k_codes, int32_t num_keys,
                                       float* out, void* stream) {
  EKV_CHECK(num_keys >= 0 && num_keys % 16 == 0, "num_keys must be a multiple of 16");
  if (num_keys == 0) return 0;
  EKV_CHECK(q_codes && k_codes && out, "null pointer");
  EKV_CHECK(aligned16(q_codes) && aligned16(k_codes), "misaligned buffers");
  hipLaunchKernelGGL(filter_dots_kernel, dim3(num_keys / 16), dim3(64), 0, static_cast<hipStream_t>(stream), q_codes,
                     k_codes, out);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_filter_dots_fp4(const uint8_t* q_values, const int32_t* q_scales, const uint8_t* k_values,
                                           const int32_t* k_scales, int32_t num_keys, float* out, void* stream) {
  EKV_CHECK(num_keys >= 0 && num_keys % 16 == 0, "num_keys must be a multiple of 16");
  if (num_keys == 0) return 0;
  EKV_CHECK(q_values && q_scales && k_values && k_scales && out, "null pointer");
  EKV_CHECK(aligned16(q_values) && aligned16(k_values), "misaligned buffers");
  hipLaunchKernelGGL(filter_dots_fp4_kernel, dim3(num_keys / 16), dim3(64), 0, static_cast<hipStream_t>(stream),
                     q_values, q_scales, k_values, k_scales, out);
  return ekv_launch_status();
}

extern "C" int ekv_topk_select(const float* scores, int64_t scores_stride, const int32_t* lengths,
                               int32_t num_tokens, int32_t max_len, int32_t* out, int64_t out_stride,
                               int32_t k, void* stream) {
  EKV_CHECK(num_tokens >= 0 && k > 0, "bad sizes");
  if (num_tokens == 0) return 0;
  EKV_CHECK(scores && lengths && out, "null pointer");
  EKV_CHECK(out_stride >= k, "out_stride must be >= k");
  EKV_CHECK(max_len >= 0 && scores_stride >= max_len, "scores_stride must be >= max_len");
  SelectArgs s{scores, scores_stride, lengths, nullptr, nullptr, nullptr, 0, nullptr, nullptr, out, out_stride, k,
               max_len, 0, nullptr, 0, 0, nullptr, 0, nullptr, 0, nullptr, 0};
  launch_select(s, num_tokens, static_cast<hipStream_t>(stream));
  return ekv_launch_status();
}

namespace {

// Outputs of a top-k call that selects: top-k rows and the optional merged rows.
struct SelOutputs {
  int32_t* topk_out;
  int64_t out_stride;
  int32_t* merged;
  int64_t merged_stride;
  int32_t merged_width;
  const int64_t* positions;
  int32_t window;
  int32_t merged_slots;
};

// Polls of a fused-kernel wait before it gives up (ekv_indexer_set_spin_limit).
int g_spin_limit = kFusedSpinLimit;

int check_topk_args(const void* q, const float* w, const uint8_t* kcache, int64_t page_stride,
                    const int32_t* block_table, const int32_t* req_ids, const int32_t* lengths, int32_t num_tokens,
                    int32_t max_len, int32_t k, void* workspace, int64_t workspace_bytes, bool fp4) {
  EKV_CHECK(num_tokens >= 0 && max_len >= 0 && k > 0, "bad sizes");
  if (num_tokens == 0) return 0;  // an empty batch: no buffer is read or written
  EKV_CHECK(q && w && kcache && block_table && req_ids && lengths, "null pointer");
  EKV_CHECK(page_stride >= kPageTokens * ((fp4 ? kFp4Row : kIdxDim) + 4) && page_stride % 16 == 0, "bad page_stride");
  EKV_CHECK(aligned16(q) && aligned16(kcache), "misaligned buffers");
  const int64_t need = ekv_indexer_topk_workspace_size(num_tokens, max_len);
  EKV_CHECK(workspace != nullptr || need == 0, "workspace is null");
  if (workspace_bytes < need) {
    set_error("workspace too small (see ekv_indexer_topk_workspace_size)");
    return kWorkspaceTooSmall;
  }
  return 0;
}

// Query-side operands of one top-k call: fp8 keys take q codes, their digit
// planes and the folded weights; fp4 keys take q values, q scale words and
// the weights.
struct TopkQuery {
  const uint8_t* q;         // fp8: codes [T, 64, 128]; fp4: packed values [T, 64, 64]
  const int8_t* q_digits;   // fp8 only
  const int32_t* q_scales;  // fp4 only
  const float* w;
};

// Stage 1: MFMA filter.  Fused plan: filter, bound and exact scoring of the
// candidates in one launch.  Otherwise: upper bounds, lower-bound histogram
// and key bound; the candidates are scored in stage 2.  With `so` the fused
// plan also selects (when a row's workgroups fit the control block) and
// *selected says whether it did.
template <bool kFp4>
int run_filter(const TopkQuery& q, const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
               const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
               int32_t num_tokens, int32_t max_len, int32_t k, void* workspace, int64_t workspace_bytes,
               void* stream, const SelOutputs* so = nullptr, bool* selected = nullptr) {
  if (selected) *selected = false;
  int rc = check_topk_args(q.q, q.w, kcache, page_stride, block_table, req_ids, lengths, num_tokens, max_len, k,
                           workspace, workspace_bytes, kFp4);
  if (rc || num_tokens == 0) return rc;
  if constexpr (kFp4) {
    EKV_CHECK(q.q_scales != nullptr, "q_scales must be a [T, 64] int32");
  } else {
    EKV_CHECK(q.q_digits != nullptr && aligned16(q.q_digits), "q_digits must be a 16-byte aligned [T, 3, 64, 128]");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t T = num_tokens, L = max_len > 0 ? max_len : 1;
  TopkWorkspace ws = carve(workspace, T, L);
  const FilterPlan plan = plan_filter<kFp4>(T, max_len);
  FilterArgs f{q.q, q.w, kcache, page_stride, num_pages, block_table, bt_stride, req_ids, lengths,
               max_len, k, ws.upper, ws.hist, num_tokens, plan.groups, q.q_scales};
  if (plan.fused) {
    // the fused kernel's counters are zero on entry and left zero
    const bool in_launch = so != nullptr && plan.groups <= kSelMaxGroups;
    FusedArgs fa{f, q.q_digits, ws.counters, ws.timeouts, ws.cand_score, ws.cand_idx, ws.counts,
                 plan.groups, plan.stage_pages, g_spin_limit,
                 in_launch ? so->topk_out : nullptr, in_launch ? so->out_stride : 0,
                 in_launch ? so->merged : nullptr, in_launch ? so->merged_stride : 0,
                 in_launch ? so->merged_width : 0, in_launch ? so->positions : nullptr,
                 in_launch ? so->window : 0, in_launch ? so->merged_slots : 0};
    if (selected) *selected = in_launch;
    const dim3 grid(static_cast<unsigned>(plan.groups), num_tokens);
    if (plan.waves == 12)
      hipLaunchKernelGGL((filter_verify_kernel<12, kFp4>), grid, dim3(64 * 12), plan.smem, s, fa);
    else
      hipLaunchKernelGGL((filter_verify_kernel<4, kFp4>), grid, dim3(64 * 4), plan.smem, s, fa);
  } else if (max_len > 0) {
    const int64_t nz = T * kHistBins + 2 * T;  // this call's hist, arrive, kbound
    const int64_t zero_blocks = (nz + 255) / 256;
    hipLaunchKernelGGL(zero_u32_kernel, dim3(static_cast<unsigned>(zero_blocks < 1024 ? zero_blocks : 1024)),
                       dim3(256), 0, s, ws.hist, nz);
    hipLaunchKernelGGL(filter_kernel<kFp4>, dim3(static_cast<unsigned>(plan.groups * T)), dim3(256), 0, s, f);
    hipLaunchKernelGGL(bound_kernel, dim3(num_tokens), dim3(256), 0, s, ws.hist, lengths, max_len, k, ws.kbound);
  }
  return ekv_launch_status();
}

// Stage 2: (unfused plan) exact scores of the candidates of each chunk; then
// the exact select over the candidate lists.
template <bool kFp4>
int run_select(const TopkQuery& q, const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
               const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
               int32_t num_tokens, int32_t max_len, int32_t* topk_out, int64_t out_stride, int32_t k,
               void* workspace, int64_t workspace_bytes, int32_t* merged_out, int64_t merged_stride,
               int32_t merged_width, const int64_t* positions, int32_t window, int32_t merged_slots, void* stream) {
  int rc = check_topk_args(kFp4 ? static_cast<const void*>(q.q) : static_cast<const void*>(q.q_digits), q.w, kcache,
                           page_stride, block_table, req_ids, lengths, num_tokens, max_len, k, workspace,
                           workspace_bytes, kFp4);
  if (rc || num_tokens == 0) return rc;
  if constexpr (kFp4) EKV_CHECK(q.q_scales != nullptr, "q_scales must be a [T, 64] int32");
  EKV_CHECK(topk_out != nullptr && out_stride >= k, "topk_out must be [T, >= k]");
  EKV_CHECK(merged_out == nullptr || (positions != nullptr && window >= 0 && merged_width >= 0 &&
                                      merged_stride >= merged_width),
            "merged_out needs positions, window >= 0 and merged_stride >= merged_width");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t T = num_tokens, L = max_len > 0 ? max_len : 1;
  const int chunks = num_chunks(max_len);
  EKV_CHECK(chunks <= kSelMaxChunks, "max_len too large for the select stage");
  TopkWorkspace ws = carve(workspace, T, L);
  const FilterPlan plan = plan_filter<kFp4>(T, max_len);
  if (!plan.fused) {
    VerifyArgs v{q.q_digits, q.w, kcache, page_stride, num_pages, block_table, bt_stride, req_ids, lengths,
                 max_len, k, ws.upper, ws.kbound, ws.cand_score, ws.cand_idx, ws.counts, chunks,
                 kFp4 ? q.q : nullptr, q.q_scales};
    hipLaunchKernelGGL(verify_kernel<kFp4>, dim3((chunks + kVerifyChunks - 1) / kVerifyChunks, num_tokens),
                       dim3(256), 0, s, v);
  }
  SelectArgs sel{nullptr, 0, lengths, ws.cand_score, ws.cand_idx, ws.counts, plan.fused ? plan.groups : chunks,
                 ws.stage_score, ws.stage_idx, topk_out, out_stride, k, static_cast<int32_t>(L),
                 plan.fused ? plan.groups : 0, merged_out, merged_stride, merged_width, positions, window,
                 merged_slots ? block_table : nullptr, bt_stride, req_ids, num_pages};
  launch_select(sel, num_tokens, s);
  return ekv_launch_status();
}

// Both stages in one call: with the fused plan the filter launch also
// selects (and merges), otherwise stage 2 runs after it.
template <bool kFp4>
int run_topk(const TopkQuery& q, const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
             const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
             int32_t num_tokens, int32_t max_len, int32_t* topk_out, int64_t out_stride, int32_t k, void* workspace,
             int64_t workspace_bytes, int32_t* merged_out, int64_t merged_stride, int32_t merged_width,
             const int64_t* positions, int32_t window, int32_t merged_slots, void* stream) {
  EKV_CHECK(num_tokens >= 0 && max_len >= 0 && k > 0, "bad sizes");
  if (num_tokens == 0) return 0;  // an empty batch: no buffer is read or written
  EKV_CHECK(topk_out != nullptr && out_stride >= k, "topk_out must be [T, >= k]");
  EKV_CHECK(merged_out == nullptr || (positions != nullptr && window >= 0 && merged_width >= 0 &&
                                      merged_stride >= merged_width),
            "merged_out needs positions, window >= 0 and merged_stride >= merged_width");
  const SelOutputs so{topk_out, out_stride, merged_out, merged_stride, merged_width, positions, window,
                      merged_slots ? 1 : 0};
  bool selected = false;
  int rc = run_filter<kFp4>(q, kcache, page_stride, num_pages, block_table, bt_stride, req_ids, lengths, num_tokens,
                            max_len, k, workspace, workspace_bytes, stream, &so, &selected);
  if (rc || selected) return rc;
  return run_select<kFp4>(q, kcache, page_stride, num_pages, block_table, bt_stride, req_ids, lengths, num_tokens,
                          max_len, topk_out, out_stride, k, workspace, workspace_bytes, merged_out, merged_stride,
                          merged_width, positions, window, merged_slots, stream);
}

}  // namespace

extern "C" int64_t ekv_indexer_topk_counter_bytes(void) { return kCounterBytes; }

extern "C" int32_t ekv_indexer_set_spin_limit(int32_t polls) {
  const int32_t prev = g_spin_limit;
  g_spin_limit = polls < 0 ? kFusedSpinLimit : polls;
  return prev;
}

extern "C" int ekv_indexer_filter(const uint8_t* q_fp8, const int8_t* q_digits, const float* w,
                                  const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                  const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                  const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t k,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  return run_filter<false>(TopkQuery{q_fp8, q_digits, nullptr, w}, kcache, page_stride, num_pages, block_table,
                           bt_stride, req_ids, lengths, num_tokens, max_len, k, workspace, workspace_bytes, stream);
}

extern "C" int ekv_indexer_select(const int8_t* q_digits, const float* w, const uint8_t* kcache, int64_t page_stride,
                                  int64_t num_pages, const int32_t* block_table, int64_t bt_stride,
                                  const int32_t* req_ids, const int32_t* lengths, int32_t num_tokens,
                                  int32_t max_len, int32_t* topk_out, int64_t out_stride, int32_t k,
                                  void* workspace, int64_t workspace_bytes, int32_t* merged_out,
                                  int64_t merged_stride, int32_t merged_width, const int64_t* positions,
                                  int32_t window, int32_t merged_slots, void* stream) {
  return run_select<false>(TopkQuery{nullptr, q_digits, nullptr, w}, kcache, page_stride, num_pages, block_table,
                           bt_stride, req_ids, lengths, num_tokens, max_len, topk_out, out_stride, k, workspace,
                           workspace_bytes, merged_out, merged_stride, merged_width, positions, window,
                           merged_slots, stream);
}

extern "C" int ekv_indexer_topk(const uint8_t* q_fp8, const int8_t* q_digits, const float* w,
                                const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t* topk_out,
                                int64_t out_stride, int32_t k, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  return run_topk<false>(TopkQuery{q_fp8, q_digits, nullptr, w}, kcache, page_stride, num_pages, block_table,
                         bt_stride, req_ids, lengths, num_tokens, max_len, topk_out, out_stride, k, workspace,
                         workspace_bytes, nullptr, 0, 0, nullptr, 0, 0, stream);
}

extern "C" int ekv_indexer_topk_merged(const uint8_t* q_fp8, const int8_t* q_digits, const float* w,
                                       const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                       const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                       const int32_t* lengths, int32_t num_tokens, int32_t max_len,
                                       int32_t* topk_out, int64_t out_stride, int32_t k, void* workspace,
                                       int64_t workspace_bytes, int32_t* merged_out, int64_t merged_stride,
                                       int32_t merged_width, const int64_t* positions, int32_t window,
                                       int32_t merged_slots, void* stream) {
  return run_topk<false>(TopkQuery{q_fp8, q_digits, nullptr, w}, kcache, page_stride, num_pages, block_table,
                         bt_stride, req_ids, lengths, num_tokens, max_len, topk_out, out_stride, k, workspace,
                         workspace_bytes, merged_out, merged_stride, merged_width, positions, window, merged_slots,
                         stream);
}

// ---------------------------------------------------------------------------
// The DSA decode prologue and the merged top-k in one call: one launch of
// the fused kernel with the prologue folded in (FusedPrologue) when the plan
// selects in that launch, else ekv_dsa_decode_prologue then
// ekv_indexer_topk_merged.  The outputs are those of the two calls.
// ---------------------------------------------------------------------------
extern "C" int ekv_dsa_decode_prologue(const uint16_t* k, int64_t k_stride, uint8_t* kcache, int64_t k_page_stride,
                                       int64_t k_num_pages, const uint16_t* latent, int64_t latent_stride,
                                       int32_t dim, uint8_t* cache, int64_t page_stride, int64_t num_pages,
                                       const int64_t* slot_mapping, int32_t num_tokens, const uint16_t* q,
                                       int64_t q_tok_stride, int64_t q_head_stride, const void* weights,
                                       int32_t weights_is_bf16, int64_t w_stride, int32_t heads, uint8_t* q_fp8,
                                       float* w_out, int8_t* q_digits, const int64_t* positions, int32_t window,
                                       int32_t* lengths, const float* ln_w, const float* ln_b, float eps,
                                       const float* cos_sin, int32_t cos_sin_rows, void* stream);

namespace {

// The prologue's checks of one appended row set (ekv_append.hip).
int check_rows(const uint16_t* rows, int64_t row_stride, int32_t dim, const int64_t* slot_mapping,
               const uint8_t* cache, int64_t page_stride) {
  EKV_CHECK(rows && slot_mapping && cache, "null pointer");
  EKV_CHECK(row_stride >= dim && row_stride % 8 == 0, "row_stride must be >= dim and a multiple of 8");
  EKV_CHECK(page_stride >= kPageTokens * (dim + 4) && page_stride % 16 == 0,
            "page_stride must hold 64 rows + 64 scales and be a multiple of 16");
  EKV_CHECK(aligned16(rows) && aligned16(cache), "rows and cache must be 16-byte aligned");
  return 0;
}

// The plan of a folded call over T rows of at most max_len keys: the fused
// plan that selects in its launch, with the folded kernel as resident as the
// plan needs (plan.fused false: the two calls run).
FilterPlan folded_plan(int64_t T, int32_t max_len) {
  FilterPlan plan = plan_filter<false>(T, max_len);
  if (!plan.fused || plan.groups > kSelMaxGroups) {
    plan.fused = false;
    return plan;
  }
  const void* kernel = plan.waves == 12 ? reinterpret_cast<const void*>(filter_verify_kernel<12, false, true>)
                                        : reinterpret_cast<const void*>(filter_verify_kernel<4, false, true>);
  int dev = 0, cus = 0;
  plan.fused = hipGetDevice(&dev) == hipSuccess &&
               hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
               T * plan.groups <= static_cast<int64_t>(occupancy(kernel, 64 * plan.waves, plan.smem)) * cus;
  return plan;
}

AppendArgs rows_args(const uint16_t* rows, int64_t row_stride, int32_t num_tokens, const int64_t* slot_mapping,
                     uint8_t* cache, int64_t page_stride, int64_t num_pages) {
  AppendArgs a{};
  a.rows = rows; a.row_stride = row_stride; a.num_tokens = num_tokens; a.slot_mapping = slot_mapping;
  a.cache = cache; a.page_stride = page_stride; a.num_pages = num_pages;
  return a;
}

}  // namespace

extern "C" int32_t ekv_dsa_decode_prologue_folds(int32_t num_tokens, int32_t max_len) {
  return (num_tokens > 0 && max_len >= 0 && folded_plan(num_tokens, max_len).fused) ? 1 : 0;
}

extern "C" int ekv_dsa_decode_prologue_topk_merged(
    const uint16_t* k, int64_t k_stride, uint8_t* kcache, int64_t k_page_stride, int64_t k_num_pages,
    const uint16_t* latent, int64_t latent_stride, int32_t dim, uint8_t* cache, int64_t page_stride,
    int64_t num_pages, const int64_t* slot_mapping, int32_t num_tokens, const uint16_t* q, int64_t q_tok_stride,
    int64_t q_head_stride, const void* weights, int32_t weights_is_bf16, int64_t w_stride, int32_t heads,
    uint8_t* q_fp8, float* w_out, int8_t* q_digits, const int64_t* positions, int32_t window,
    int32_t max_new_rows, int32_t* lengths, const float* ln_w, const float* ln_b, float eps, const float* cos_sin,
    int32_t cos_sin_rows, const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids, int32_t max_len,
    int32_t* topk_out, int64_t out_stride, int32_t k_top, void* workspace, int64_t workspace_bytes,
    int32_t* merged_out, int64_t merged_stride, int32_t merged_width, int32_t merged_slots, void* stream) {
  EKV_CHECK(num_tokens >= 0 && window >= 0 && max_len >= 0 && k_top > 0, "bad sizes");
  if (num_tokens == 0) return 0;
  const int64_t T = num_tokens;
  FilterPlan plan{false, 4, 1, 0, 0};
  // folded only when no row can score a key this call appends: every
  // sequence's new rows (its last positions) number at most `window`
  if (heads == kIdxHeads && max_new_rows >= 1 && max_new_rows <= window && merged_out != nullptr)
    plan = folded_plan(T, max_len);
  if (!plan.fused) {
    const int rc = ekv_dsa_decode_prologue(k, k_stride, kcache, k_page_stride, k_num_pages, latent, latent_stride,
                                           dim, cache, page_stride, num_pages, slot_mapping, num_tokens, q,
                                           q_tok_stride, q_head_stride, weights, weights_is_bf16, w_stride, heads,
                                           q_fp8, w_out, q_digits, positions, window, lengths, ln_w, ln_b, eps,
                                           cos_sin, cos_sin_rows, stream);
    if (rc) return rc;
    return ekv_indexer_topk_merged(q_fp8, q_digits, w_out, kcache, k_page_stride, k_num_pages, block_table,
                                   bt_stride, req_ids, lengths, num_tokens, max_len, topk_out, out_stride, k_top,
                                   workspace, workspace_bytes, merged_out, merged_stride, merged_width, positions,
                                   window, merged_slots, stream);
  }
  // the checks the two calls make
  EKV_CHECK(cos_sin == nullptr || (ln_w && ln_b && cos_sin_rows >= 0 && aligned16(ln_w) && aligned16(ln_b) &&
                                   aligned16(cos_sin)),
            "the indexer prep needs 16-byte aligned ln_w, ln_b and cos_sin");
  EKV_CHECK(dim == 512 || dim == 576, "latent dim must be 512 or 576");
  int rc = check_rows(k, k_stride, 128, slot_mapping, kcache, k_page_stride);
  if (rc) return rc;
  rc = check_rows(latent, latent_stride, dim, slot_mapping, cache, page_stride);
  if (rc) return rc;
  EKV_CHECK(q && weights && q_fp8 && w_out, "null pointer");
  EKV_CHECK(q_head_stride % 8 == 0 && q_tok_stride % 8 == 0, "strides must be multiples of 8");
  EKV_CHECK(aligned16(q), "misaligned buffers");
  EKV_CHECK(positions && lengths, "null pointer");
  EKV_CHECK(topk_out != nullptr && out_stride >= k_top, "topk_out must be [T, >= k]");
  EKV_CHECK(merged_width >= 0 && merged_stride >= merged_width,
            "merged_out needs positions, window >= 0 and merged_stride >= merged_width");
  rc = check_topk_args(q_fp8, w_out, kcache, k_page_stride, block_table, req_ids, lengths, num_tokens, max_len,
                       k_top, workspace, workspace_bytes, false);
  if (rc) return rc;
  EKV_CHECK(q_digits != nullptr && aligned16(q_digits), "q_digits must be a 16-byte aligned [T, 3, 64, 128]");

  const int64_t L = max_len > 0 ? max_len : 1;
  TopkWorkspace ws = carve(workspace, T, L);
  FilterArgs f{q_fp8, w_out, kcache, k_page_stride, k_num_pages, block_table, bt_stride, req_ids, lengths,
               max_len, k_top, ws.upper, ws.hist, num_tokens, plan.groups, nullptr};
  FusedArgs fa{f, q_digits, ws.counters, ws.timeouts, ws.cand_score, ws.cand_idx, ws.counts, plan.groups,
               plan.stage_pages, g_spin_limit, topk_out, out_stride, merged_out, merged_stride, merged_width,
               positions, window, merged_slots ? 1 : 0};
  FusedPrologue& pro = fa.pro;
  pro.q = q;
  pro.q_tok_stride = q_tok_stride;
  pro.q_head_stride = q_head_stride;
  pro.w = weights;
  pro.w_is_bf16 = weights_is_bf16;
  pro.w_stride = w_stride;
  pro.cos_sin = cos_sin;
  pro.cs_rows = cos_sin_rows;
  pro.lengths = lengths;
  pro.q_fp8_out = q_fp8;
  pro.w_out = w_out;
  pro.q_digits_out = q_digits;
  pro.k_rows = rows_args(k, k_stride, num_tokens, slot_mapping, kcache, k_page_stride, k_num_pages);
  if (cos_sin != nullptr) {
    pro.k_rows.positions = positions;
    pro.k_rows.ln_w = ln_w;
    pro.k_rows.ln_b = ln_b;
    pro.k_rows.eps = eps;
    pro.k_rows.cos_sin = cos_sin;
    pro.k_rows.cs_rows = cos_sin_rows;
  }
  pro.latent = rows_args(latent, latent_stride, num_tokens, slot_mapping, cache, page_stride, num_pages);
  pro.latent_dim = dim;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(plan.groups), num_tokens);
  if (plan.waves == 12)
    hipLaunchKernelGGL((filter_verify_kernel<12, false, true>), grid, dim3(64 * 12), plan.smem, s, fa);
  else
    hipLaunchKernelGGL((filter_verify_kernel<4, false, true>), grid, dim3(64 * 4), plan.smem, s, fa);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_filter_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                                      const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                      const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                      const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t k,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
  return run_filter<true>(TopkQuery{q_values, nullptr, q_scales, w}, kcache, page_stride, num_pages, block_table,
                          bt_stride, req_ids, lengths, num_tokens, max_len, k, workspace, workspace_bytes, stream);
}

extern "C" int ekv_indexer_select_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                                      const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                      const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                      const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t* topk_out,
                                      int64_t out_stride, int32_t k, void* workspace, int64_t workspace_bytes,
                                      int32_t* merged_out, int64_t merged_stride, int32_t merged_width,
                                      const int64_t* positions, int32_t window, int32_t merged_slots, void* stream) {
  return run_select<true>(TopkQuery{q_values, nullptr, q_scales, w}, kcache, page_stride, num_pages, block_table,
                          bt_stride, req_ids, lengths, num_tokens, max_len, topk_out, out_stride, k, workspace,
                          workspace_bytes, merged_out, merged_stride, merged_width, positions, window, merged_slots,
                          stream);
}

extern "C" int ekv_indexer_topk_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                                    const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                    const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                    const int32_t* lengths, int32_t num_tokens, int32_t max_len, int32_t* topk_out,
                                    int64_t out_stride, int32_t k, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  return run_topk<true>(TopkQuery{q_values, nullptr, q_scales, w}, kcache, page_stride, num_pages, block_table,
                        bt_stride, req_ids, lengths, num_tokens, max_len, topk_out, out_stride, k, workspace,
                        workspace_bytes, nullptr, 0, 0, nullptr, 0, 0, stream);
}

extern "C" int ekv_indexer_topk_merged_fp4(const uint8_t* q_values, const int32_t* q_scales, const float* w,
                                           const uint8_t* kcache, int64_t page_stride, int64_t num_pages,
                                           const int32_t* block_table, int64_t bt_stride, const int32_t* req_ids,
                                           const int32_t* lengths, int32_t num_tokens, int32_t max_len,
                                           int32_t* topk_out, int64_t out_stride, int32_t k, void* workspace,
                                           int64_t workspace_bytes, int32_t* merged_out, int64_t merged_stride,
                                           int32_t merged_width, const int64_t* positions, int32_t window,
                                           int32_t merged_slots, void* stream) {
  return run_topk<true>(TopkQuery{q_values, nullptr, q_scales, w}, kcache, page_stride, num_pages, block_table,
                        bt_stride, req_ids, lengths, num_tokens, max_len, topk_out, out_stride, k, workspace,
                        workspace_bytes, merged_out, merged_stride, merged_width, positions, window, merged_slots,
                        stream);
}
