// Lightning-indexer scoring and exact top-k.
//
// Scoring is exact.  Every e4m3fn value is an integer I = value * 2**9 with
// |I| < 2**18, split into three signed base-64 digits (int8).  A head's dot
// product over the 128 dims is the exact int64
//
//   D = sum_{a,b} 64**(a+b) * sum_d qdigit_a[d] * kdigit_b[d]
//
// whose nine digit-pair sums run on v_mfma_i32_16x16x64_i8 (exact int32
// accumulation; partial sums stay below 2**21).  Then
//   dot = fl32(D * 2**-18), p_h = fl32(w_h * max(dot, 0)),
//   heads summed in fp32 in a fixed order (see head sum below),
//   score = fl32(acc * kscale) + 0.
// The CPU oracle evaluates the same formula, so scores -- and hence the
// top-k with its lowest-index tie-break -- are bit-exact.
//
// MFMA layout (16x16x64 i8): lane l holds A row l%16 (a head of the head
// block) and B column l%16 (a token), K bytes [16*(l/16), +16) of a 64-byte
// half; C lane l holds rows 4*(l/16)+i, column l%16.
//
// The top-k kernel is a radix select on order-preserving uint32 keys (three
// passes of 11/11/10 bits over the row's scores, LDS histograms) followed by
// an ordered compaction: keys above the threshold key, then threshold ties by
// ascending index; the output indices are ascending, padded with -1.
#include "ekv_common.h"
#include "ekv_internal.h"

namespace ekv {

constexpr int kIdxDim = 128;
constexpr int kIdxHeads = 64;
constexpr int kIdxPageBytes = kPageTokens * kIdxDim;  // scales follow the values

struct ScoreArgs {
  const int8_t* q_digits;    // [T, 3, 64, 128]
  const float* w;            // [T, 64] folded head weights
  const uint8_t* kcache;     // [num_pages, page_stride]
  int64_t page_stride;
  int64_t num_pages;
  const int32_t* block_table;  // [B, bt_stride]
  int64_t bt_stride;
  const int32_t* req_ids;    // [T]
  const int32_t* lengths;    // [T] candidate count (implicit range) or null
  const int32_t* cand;       // [T, cand_stride] explicit token list or null
  const int32_t* cand_count; // [T] when cand != null
  int64_t cand_stride;
  float* scores;             // [T, scores_stride]
  int64_t scores_stride;
  int32_t max_len;           // candidates beyond this are ignored
};

constexpr int kScoreIters = 8;                        // 16-token blocks per wave
constexpr int kScoreChunk = 4 * 16 * kScoreIters;     // tokens per workgroup

__device__ __forceinline__ uint32_t plane_word(uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3, int p) {
  const uint32_t sel = static_cast<uint32_t>(p) | (static_cast<uint32_t>(4 + p) << 8) | 0x0c0c0000u;
  const uint32_t x01 = __builtin_amdgcn_perm(e1, e0, sel);
  const uint32_t x23 = __builtin_amdgcn_perm(e3, e2, sel);
  return x01 | (x23 << 16);
}

__global__ void __launch_bounds__(256) score_exact_kernel(ScoreArgs a) {
  __shared__ uint32_t s_table[256];
  const int tid = threadIdx.x;
  s_table[tid] = fp8_digit_pack(static_cast<uint32_t>(tid));
  const int t = blockIdx.y;
  const int n = min(a.cand ? a.cand_count[t] : a.lengths[t], a.max_len);
  const int64_t chunk0 = static_cast<int64_t>(blockIdx.x) * kScoreChunk;
  __syncthreads();
  if (chunk0 >= n) return;

  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;
  const int req = a.req_ids[t];
  const int32_t* bt = a.block_table + static_cast<int64_t>(req) * a.bt_stride;

  // q digit operands: [hb][digit][kh]
  i32x4 qd[4][3][2];
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int d = 0; d < 3; ++d)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const int8_t* src = a.q_digits + ((static_cast<int64_t>(t) * 3 + d) * kIdxHeads + 16 * hb + col) * kIdxDim +
                            64 * kh + 16 * g;
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        qd[hb][d][kh] = i32x4{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z),
                              static_cast<int>(v.w)};
      }
  float wv[4][4];
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[hb][i] = a.w[static_cast<int64_t>(t) * kIdxHeads + 16 * hb + 4 * g + i];

  for (int it = 0; it < kScoreIters; ++it) {
    const int64_t li = chunk0 + (static_cast<int64_t>(wave) * kScoreIters + it) * 16 + col;  // local index
    const bool valid = li < n;
    int64_t s = 0;
    if (valid) s = a.cand ? a.cand[static_cast<int64_t>(t) * a.cand_stride + li] : li;
    uint4 kb[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    float kscale = 0.0f;
    if (valid && (s >> 6) < a.bt_stride) {
      const int64_t page = bt[s >> 6];
      if (page >= 0 && page < a.num_pages) {
        const uint8_t* base = a.kcache + page * a.page_stride;
        const int row = static_cast<int>(s & 63);
        kb[0] = *reinterpret_cast<const uint4*>(base + row * kIdxDim + 16 * g);
        kb[1] = *reinterpret_cast<const uint4*>(base + row * kIdxDim + 64 + 16 * g);
        kscale = *reinterpret_cast<const float*>(base + kIdxPageBytes + row * 4);
      }
    }
    // digit planes of this lane's 32 key bytes: kd[digit][kh]
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
    // head sum in the fixed order: hb = 0..3, then i = 0..3, from +0
    float acc = 0.0f;
#pragma unroll
    for (int hb = 0; hb < 4; ++hb) {
      i32x4 c[5];
#pragma unroll
      for (int k = 0; k < 5; ++k) c[k] = i32x4{0, 0, 0, 0};
#pragma unroll
      for (int da = 0; da < 3; ++da)
#pragma unroll
        for (int db = 0; db < 3; ++db)
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
            c[da + db] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[hb][da][kh], kd[db][kh], c[da + db], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t D = static_cast<int64_t>(c[0][i]) + (static_cast<int64_t>(c[1][i]) << 6) +
                          (static_cast<int64_t>(c[2][i]) << 12) + (static_cast<int64_t>(c[3][i]) << 18) +
                          (static_cast<int64_t>(c[4][i]) << 24);
        const float dot = static_cast<float>(static_cast<double>(D) * 0x1p-18);
        const float r = fmaxf(dot, 0.0f);
        acc = acc + wv[hb][i] * r;
      }
    }
    const float a01 = acc + __shfl_xor(acc, 16);
    const float tot = a01 + __shfl_xor(a01, 32);
    if (valid && g == 0) a.scores[static_cast<int64_t>(t) * a.scores_stride + li] = tot * kscale + 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Exact top-k of one row per workgroup (1024 threads).
// ---------------------------------------------------------------------------
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;

struct SelectArgs {
  const float* scores;       // [T, scores_stride]
  int64_t scores_stride;
  const int32_t* lengths;    // [T] (implicit indices 0..n-1) or null
  const int32_t* cand;       // [T, cand_stride] explicit ascending indices or null
  const int32_t* cand_count;
  int64_t cand_stride;
  int32_t* out;              // [T, out_stride]
  int64_t out_stride;
  int32_t k;
  int32_t max_len;           // candidates beyond this are ignored
};

// Block-wide exclusive prefix of a 0/1 flag; returns the prefix, writes total.
__device__ __forceinline__ int block_flag_scan(bool flag, int* s_wave, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t bal = __ballot(flag);
  const int in_wave = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u));
  if (lane == 0) s_wave[wave] = __popcll(bal);
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const int c = s_wave[w];
    before += (w < wave) ? c : 0;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return before + in_wave;
}

__global__ void __launch_bounds__(kSelThreads) topk_select_kernel(SelectArgs a) {
  __shared__ uint32_t s_hist[2048];
  __shared__ uint32_t s_part[kSelThreads];
  __shared__ int s_wave[kSelWaves];
  __shared__ uint32_t s_res[2];
  const int tid = threadIdx.x;
  const int t = blockIdx.x;
  const int n = max(0, min(a.cand ? a.cand_count[t] : a.lengths[t], a.max_len));
  const float* sc = a.scores + static_cast<int64_t>(t) * a.scores_stride;
  const int32_t* idx = a.cand ? a.cand + static_cast<int64_t>(t) * a.cand_stride : nullptr;
  int32_t* out = a.out + static_cast<int64_t>(t) * a.out_stride;
  const int k = a.k;

  uint32_t kstar = 0;
  int need = 0;
  if (n > k) {
    uint32_t prefix = 0, mask = 0;
    int remaining = k;
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = shifts[pass];
      const int nb = 1 << widths[pass];
      for (int b = tid; b < 2048; b += kSelThreads) s_hist[b] = 0;
      __syncthreads();
      for (int i = tid; i < n; i += kSelThreads) {
        const uint32_t key = score_key(sc[i] + 0.0f);  // -0 ties with +0
        if ((key & mask) == prefix) atomicAdd(&s_hist[(key >> sh) & (nb - 1)], 1u);
      }
      __syncthreads();
      // suffix counts over bins, scanning from the top bin downwards:
      // thread i owns reversed bins r = 2i, 2i+1 (bin = nb-1-r).
      uint32_t c0 = 0, c1 = 0;
      const int r0 = 2 * tid, r1 = 2 * tid + 1;
      if (r0 < nb) c0 = s_hist[nb - 1 - r0];
      if (r1 < nb) c1 = s_hist[nb - 1 - r1];
      s_part[tid] = c0 + c1;
      __syncthreads();
      // inclusive scan of s_part (Hillis-Steele in LDS)
      for (int off = 1; off < kSelThreads; off <<= 1) {
        const uint32_t v = (tid >= off) ? s_part[tid - off] : 0u;
        __syncthreads();
        s_part[tid] += v;
        __syncthreads();
      }
      const uint32_t incl = s_part[tid];
      const uint32_t excl = incl - (c0 + c1);
      const uint32_t rem = static_cast<uint32_t>(remaining);
      if (r0 < nb && excl < rem && rem <= excl + c0) { s_res[0] = nb - 1 - r0; s_res[1] = excl; }
      if (r1 < nb && excl + c0 < rem && rem <= excl + c0 + c1) { s_res[0] = nb - 1 - r1; s_res[1] = excl + c0; }
      __syncthreads();
      const uint32_t bin = s_res[0];
      remaining -= static_cast<int>(s_res[1]);
      prefix |= bin << sh;
      mask |= static_cast<uint32_t>(nb - 1) << sh;
      __syncthreads();
    }
    kstar = prefix;
    need = remaining;  // threshold-valued elements to take, lowest index first
  }

  // ordered compaction
  int out_base = 0, eq_base = 0;
  for (int i0 = 0; i0 < n; i0 += kSelThreads) {
    const int i = i0 + tid;
    bool gt = false, eq = false;
    if (i < n) {
      if (n <= k) {
        gt = true;
      } else {
        const uint32_t key = score_key(sc[i] + 0.0f);  // -0 ties with +0
        gt = key > kstar;
        eq = key == kstar;
      }
    }
    int eq_total;
    const int eq_rank = block_flag_scan(eq, s_wave, eq_total);
    const bool sel = gt || (eq && eq_base + eq_rank < need);
    int sel_total;
    const int pos = block_flag_scan(sel, s_wave, sel_total);
    if (sel && out_base + pos < k) out[out_base + pos] = idx ? idx[i] : i;
    out_base += sel_total;
    eq_base += eq_total;
  }
  for (int i = out_base + tid; i < k; i += kSelThreads) out[i] = -1;
}

}  // namespace ekv

using namespace ekv;

extern "C" int64_t ekv_indexer_topk_workspace_size(int32_t num_tokens, int32_t max_len) {
  if (num_tokens <= 0 || max_len <= 0) return 0;
  return static_cast<int64_t>(num_tokens) * max_len * 4 + 256;
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
              nullptr, nullptr, 0, scores, scores_stride, max_len};
  dim3 grid((max_len + kScoreChunk - 1) / kScoreChunk, num_tokens);
  hipLaunchKernelGGL(score_exact_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
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
  SelectArgs s{scores, scores_stride, lengths, nullptr, nullptr, 0, out, out_stride, k, max_len};
  hipLaunchKernelGGL(topk_select_kernel, dim3(num_tokens), dim3(kSelThreads), 0,
                     static_cast<hipStream_t>(stream), s);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_topk(const int8_t* q_digits, const float* w, const uint8_t* kcache,
                                int64_t page_stride, int64_t num_pages, const int32_t* block_table,
                                int64_t bt_stride, const int32_t* req_ids, const int32_t* lengths,
                                int32_t num_tokens, int32_t max_len, int32_t* topk_out, int64_t out_stride,
                                int32_t k, void* workspace, int64_t workspace_bytes, void* stream) {
  EKV_CHECK(num_tokens >= 0 && max_len >= 0 && k > 0, "bad sizes");
  if (num_tokens == 0) return 0;
  const int64_t need = ekv_indexer_topk_workspace_size(num_tokens, max_len);
  EKV_CHECK(workspace != nullptr || need == 0, "workspace is null");
  if (workspace_bytes < need) {
    set_error("workspace too small (see ekv_indexer_topk_workspace_size)");
    return kWorkspaceTooSmall;
  }
  float* scores = static_cast<float*>(workspace);
  const int64_t sstride = max_len > 0 ? max_len : 1;
  int rc = 0;
  if (max_len > 0) {
    rc = ekv_indexer_score(q_digits, w, kcache, page_stride, num_pages, block_table, bt_stride, req_ids,
                           lengths, num_tokens, max_len, scores, sstride, stream);
    if (rc) return rc;
  }
  return ekv_topk_select(scores, sstride, lengths, num_tokens, max_len, topk_out, out_stride, k, stream);
}
