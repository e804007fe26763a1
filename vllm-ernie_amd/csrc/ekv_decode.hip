// Sparse MLA decode over gathered latent rows (DSA top-k + window, HCA
// compressed + window), with the per-head attention sink in the softmax
// denominator.
//
// Workgroup = (query row t, split s of its index row); one wave per 16 heads.
// Each tile of 32 index entries is gathered from the paged cache (fp8 rows of
// D bytes + fp32 scale per token, or bf16 flat rows), staged in LDS, and
// widened once to bf16 in two LDS images: K [entry][dim] (row-major, the B
// operand of S = Q K^T) and V^T [dim][entry] (the B operand of O = P V).
// Both products run on v_mfma_f32_16x16x32_bf16 with q held in registers for
// the whole workgroup.  The softmax is online in the log2 domain; the fp8
// row scale multiplies the scores and is folded into P for the values.
// Partial (O, m, l) per split go to a workspace; the combine kernel merges the
// splits, adds the sink and writes bf16 out and the natural-log lse
// (log sum_j exp(s_j), sink excluded).
#include "ekv_common.h"
#include "ekv_internal.h"

namespace ekv {

constexpr int kDv = 512;
constexpr int kTile = 32;
constexpr int kMaxWaves = 4;   // up to 64 heads (one wave per 16)
constexpr float kLog2e = 0x1.715476p+0f;
constexpr float kLn2 = 0x1.62e430p-1f;

struct DecodeArgs {
  const uint16_t* q;        // [T, H, D] bf16
  int64_t q_tok_stride, q_head_stride;
  const uint8_t* cache;     // fp8 pages [num_pages, page_stride] or bf16 rows
  int64_t page_stride;      // bytes (fp8 layout)
  int64_t num_rows;         // addressable rows (num_pages * 64)
  int32_t cache_bf16;       // 0 fp8 paged, 1 bf16 flat rows
  const int32_t* indices;   // [T, idx_stride]
  int64_t idx_stride;
  int32_t width;            // entries per index row
  const int32_t* lengths;   // [T] or null
  const int32_t* block_table;  // logical indices when non-null
  int64_t bt_stride;
  const int32_t* req_ids;   // [T] with block_table
  float scale;              // softmax scale
  int32_t heads;
  int32_t per_split;        // entries per split (multiple of kTile)
  float* ws_o;              // [T, NS, H, 512]
  float* ws_ml;             // [T, NS, H, 2]
  int32_t splits;
};

template <int D>
struct DecodeSmem {
  static constexpr int kStage = D + 16;     // fp8 staging row stride (bytes)
  static constexpr int kKRow = D + 8;       // bf16 K row stride (elements)
  static constexpr int kVRow = kTile + 8;   // bf16 V^T row stride (elements)
  uint8_t stage[kTile * kStage];
  uint16_t k[kTile * kKRow];
  uint16_t vt[kDv * kVRow];
  uint16_t p[kMaxWaves][16 * kTile];
  int64_t slot[kTile];
  float kscale[kTile];
};

__device__ __forceinline__ uint32_t byte_column(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, int i) {
  const uint32_t sel = static_cast<uint32_t>(i) | (static_cast<uint32_t>(4 + i) << 8) | 0x0c0c0000u;
  return __builtin_amdgcn_perm(w1, w0, sel) | (__builtin_amdgcn_perm(w3, w2, sel) << 16);
}

template <int D>
__global__ void __launch_bounds__(256) sparse_decode_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  DecodeSmem<D>& sm = *reinterpret_cast<DecodeSmem<D>*>(smem_raw);
  constexpr int KS = D / 32;  // k-steps of the QK product
  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;
  const int t = blockIdx.y, split = blockIdx.x;
  const int len = a.lengths ? min(a.lengths[t], a.width) : a.width;
  const int e_begin = split * a.per_split;
  const int e_end = min(e_begin + a.per_split, len);
  const int head0 = 16 * wave;

  // q operands (A of S = Q K^T): lane holds head head0 + col, dims 32ks + 8g .. +8
  bf16x8 qa[KS];
  {
    const uint16_t* qrow = a.q + static_cast<int64_t>(t) * a.q_tok_stride + (head0 + col) * a.q_head_stride;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 v = *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g);
      qa[ks] = __builtin_bit_cast(bf16x8, v);
    }
  }
  f32x4 o[kDv / 16];
#pragma unroll
  for (int i = 0; i < kDv / 16; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m2[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  float lsum[4] = {0.f, 0.f, 0.f, 0.f};
  const float sc2 = a.scale * kLog2e;

  for (int e0 = e_begin; e0 < e_end; e0 += kTile) {
    // 1. indices -> slots and scales
    if (tid < kTile) {
      const int e = e0 + tid;
      int64_t slot = -1;
      if (e < e_end) {
        int64_t idx = a.indices[static_cast<int64_t>(t) * a.idx_stride + e];
        if (idx >= 0 && a.block_table != nullptr) {
          const int64_t blk = idx >> 6;
          idx = (blk < a.bt_stride)
                    ? static_cast<int64_t>(a.block_table[static_cast<int64_t>(a.req_ids[t]) * a.bt_stride + blk]) *
                              kPageTokens + (idx & 63)
                    : -1;
        }
        slot = (idx >= 0 && idx < a.num_rows) ? idx : -1;
      }
      sm.slot[tid] = slot;
      float ks = 0.0f;
      if (slot >= 0) {
        ks = a.cache_bf16 ? 1.0f
                          : *reinterpret_cast<const float*>(a.cache + (slot / kPageTokens) * a.page_stride +
                                                            kPageTokens * D + (slot % kPageTokens) * 4);
      }
      sm.kscale[tid] = ks;
    }
    __syncthreads();
    // 2. gather rows
    if (!a.cache_bf16) {
      constexpr int kParts = D / 16;
      for (int c = tid; c < kTile * kParts; c += nthreads) {
        const int r = c / kParts, part = c % kParts;
        const int64_t slot = sm.slot[r];
        uint4 v = make_uint4(0, 0, 0, 0);
        if (slot >= 0)
          v = *reinterpret_cast<const uint4*>(a.cache + (slot / kPageTokens) * a.page_stride +
                                              (slot % kPageTokens) * D + 16 * part);
        *reinterpret_cast<uint4*>(&sm.stage[r * DecodeSmem<D>::kStage + 16 * part]) = v;
      }
    } else {
      constexpr int kParts = D / 8;
      for (int c = tid; c < kTile * kParts; c += nthreads) {
        const int r = c / kParts, part = c % kParts;
        const int64_t slot = sm.slot[r];
        uint4 v = make_uint4(0, 0, 0, 0);
        if (slot >= 0)
          v = *reinterpret_cast<const uint4*>(a.cache + slot * (2 * D) + 16 * part);
        *reinterpret_cast<uint4*>(&sm.k[r * DecodeSmem<D>::kKRow + 8 * part]) = v;
      }
    }
    __syncthreads();
    // 3. widen to bf16 K rows and V^T columns, 4 entries x 4 dims per item
    {
      constexpr int kDimGroups = D / 4;
      for (int it = tid; it < (kTile / 4) * kDimGroups; it += nthreads) {
        const int rg = it / kDimGroups, dg = it % kDimGroups;
        const int r0 = 4 * rg, d0 = 4 * dg;
        if (!a.cache_bf16) {
          uint32_t w[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            w[r] = *reinterpret_cast<const uint32_t*>(&sm.stage[(r0 + r) * DecodeSmem<D>::kStage + d0]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            uint32_t lo, hi;
            fp8x4_to_bf16x4(w[r], lo, hi);
            *reinterpret_cast<uint2*>(&sm.k[(r0 + r) * DecodeSmem<D>::kKRow + d0]) = make_uint2(lo, hi);
          }
          if (d0 < kDv) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              uint32_t lo, hi;
              fp8x4_to_bf16x4(byte_column(w[0], w[1], w[2], w[3], i), lo, hi);
              *reinterpret_cast<uint2*>(&sm.vt[(d0 + i) * DecodeSmem<D>::kVRow + r0]) = make_uint2(lo, hi);
            }
          }
        } else if (d0 < kDv) {
          uint2 w[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            w[r] = *reinterpret_cast<const uint2*>(&sm.k[(r0 + r) * DecodeSmem<D>::kKRow + d0]);
          // 16-bit transpose of a 4x4 block
          const uint32_t c0lo = __builtin_amdgcn_perm(w[1].x, w[0].x, 0x05040100u);
          const uint32_t c0hi = __builtin_amdgcn_perm(w[3].x, w[2].x, 0x05040100u);
          const uint32_t c1lo = __builtin_amdgcn_perm(w[1].x, w[0].x, 0x07060302u);
          const uint32_t c1hi = __builtin_amdgcn_perm(w[3].x, w[2].x, 0x07060302u);
          const uint32_t c2lo = __builtin_amdgcn_perm(w[1].y, w[0].y, 0x05040100u);
          const uint32_t c2hi = __builtin_amdgcn_perm(w[3].y, w[2].y, 0x05040100u);
          const uint32_t c3lo = __builtin_amdgcn_perm(w[1].y, w[0].y, 0x07060302u);
          const uint32_t c3hi = __builtin_amdgcn_perm(w[3].y, w[2].y, 0x07060302u);
          *reinterpret_cast<uint2*>(&sm.vt[(d0 + 0) * DecodeSmem<D>::kVRow + r0]) = make_uint2(c0lo, c0hi);
          *reinterpret_cast<uint2*>(&sm.vt[(d0 + 1) * DecodeSmem<D>::kVRow + r0]) = make_uint2(c1lo, c1hi);
          *reinterpret_cast<uint2*>(&sm.vt[(d0 + 2) * DecodeSmem<D>::kVRow + r0]) = make_uint2(c2lo, c2hi);
          *reinterpret_cast<uint2*>(&sm.vt[(d0 + 3) * DecodeSmem<D>::kVRow + r0]) = make_uint2(c3lo, c3hi);
        }
      }
    }
    __syncthreads();
    // 4. S = Q K^T for this wave's 16 heads x 32 entries
    f32x4 s[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      s[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = &sm.k[(16 * nt + col) * DecodeSmem<D>::kKRow + 8 * g];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 kb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(krow + 32 * ks));
        s[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], kb, s[nt], 0, 0, 0);
      }
    }
    // 5. online softmax (log2 domain); lane owns heads 4g+i, entries 16nt+col
    float pv[2][4];
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x0 = (sm.slot[col] >= 0) ? s[0][i] * (sc2 * sm.kscale[col]) : -INFINITY;
      float x1 = (sm.slot[16 + col] >= 0) ? s[1][i] * (sc2 * sm.kscale[16 + col]) : -INFINITY;
      float mx = fmaxf(x0, x1);
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 16));
      const float mnew = fmaxf(m2[i], mx);
      if (mnew == -INFINITY) {
        alpha[i] = 1.0f;
        pv[0][i] = 0.0f;
        pv[1][i] = 0.0f;
      } else {
        alpha[i] = exp2f(m2[i] - mnew);
        pv[0][i] = exp2f(x0 - mnew);
        pv[1][i] = exp2f(x1 - mnew);
      }
      lsum[i] = lsum[i] * alpha[i] + (pv[0][i] + pv[1][i]);
      m2[i] = mnew;
    }
#pragma unroll
    for (int nt = 0; nt < kDv / 16; ++nt) {
      o[nt][0] *= alpha[0]; o[nt][1] *= alpha[1]; o[nt][2] *= alpha[2]; o[nt][3] *= alpha[3];
    }
    // 6. P' = P * kscale (bf16) to LDS in A layout source order [head][entry]
    {
      uint16_t* pw = sm.p[wave];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const float ks = sm.kscale[16 * nt + col];
#pragma unroll
        for (int i = 0; i < 4; ++i) pw[(4 * g + i) * kTile + 16 * nt + col] = f32_to_bf16(pv[nt][i] * ks);
      }
    }
    __syncthreads();
    // 7. O += P' V
    {
      const bf16x8 pa = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&sm.p[wave][col * kTile + 8 * g]));
#pragma unroll
      for (int nt = 0; nt < kDv / 16; ++nt) {
        const bf16x8 vb = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(&sm.vt[(16 * nt + col) * DecodeSmem<D>::kVRow + 8 * g]));
        o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, o[nt], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // partial results: l summed over the 16 lanes of each head
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) lsum[i] += __shfl_xor(lsum[i], off, 16);
  }
  const int64_t base = (static_cast<int64_t>(t) * a.splits + split) * a.heads;
#pragma unroll
  for (int nt = 0; nt < kDv / 16; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a.ws_o[(base + head0 + 4 * g + i) * kDv + 16 * nt + col] = o[nt][i];
  if (col == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a.ws_ml[(base + head0 + 4 * g + i) * 2 + 0] = m2[i];
      a.ws_ml[(base + head0 + 4 * g + i) * 2 + 1] = lsum[i];
    }
  }
}

// One workgroup of 128 threads per (t, h): merge the splits, add the sink.
__global__ void __launch_bounds__(128) decode_combine_kernel(
    const float* ws_o, const float* ws_ml, int32_t splits, int32_t heads, const float* sinks,
    uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride, float* lse, int64_t lse_stride) {
  const int t = blockIdx.y, h = blockIdx.x, tid = threadIdx.x;
  float M = -INFINITY;
  for (int s = 0; s < splits; ++s) M = fmaxf(M, ws_ml[((static_cast<int64_t>(t) * splits + s) * heads + h) * 2]);
  float L = 0.0f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (M != -INFINITY) {
    for (int s = 0; s < splits; ++s) {
      const int64_t b = (static_cast<int64_t>(t) * splits + s) * heads + h;
      const float ms = ws_ml[b * 2];
      if (ms == -INFINITY) continue;
      const float f = exp2f(ms - M);
      L += ws_ml[b * 2 + 1] * f;
      const float4 v = *reinterpret_cast<const float4*>(ws_o + b * kDv + 4 * tid);
      acc[0] += v.x * f; acc[1] += v.y * f; acc[2] += v.z * f; acc[3] += v.w * f;
    }
  }
  float den = L;
  float numf = 1.0f;
  if (sinks != nullptr) {
    const float sk = sinks[h] * kLog2e;
    const float Mp = fmaxf(M, sk);
    if (Mp != -INFINITY) {
      numf = (M == -INFINITY) ? 0.0f : exp2f(M - Mp);
      den = L * numf + exp2f(sk - Mp);
    }
  }
  const float inv = (den > 0.0f) ? numf / den : 0.0f;
  uint16_t* orow = out + static_cast<int64_t>(t) * out_tok_stride + h * out_head_stride;
  const uint32_t w0 = static_cast<uint32_t>(f32_to_bf16(acc[0] * inv)) | (static_cast<uint32_t>(f32_to_bf16(acc[1] * inv)) << 16);
  const uint32_t w1 = static_cast<uint32_t>(f32_to_bf16(acc[2] * inv)) | (static_cast<uint32_t>(f32_to_bf16(acc[3] * inv)) << 16);
  *reinterpret_cast<uint2*>(orow + 4 * tid) = make_uint2(w0, w1);
  if (tid == 0 && lse != nullptr)
    lse[static_cast<int64_t>(t) * lse_stride + h] = (L > 0.0f) ? (M + log2f(L)) * kLn2 : -INFINITY;
}

}  // namespace ekv

using namespace ekv;

static int decode_splits(int32_t num_tokens, int32_t width) {
  const int tiles = (width + kTile - 1) / kTile;
  int splits = (512 + num_tokens - 1) / (num_tokens > 0 ? num_tokens : 1);
  if (splits > tiles) splits = tiles;
  if (splits < 1) splits = 1;
  return splits;
}

extern "C" int64_t ekv_sparse_mla_decode_workspace_size(int32_t num_tokens, int32_t heads, int32_t width) {
  if (num_tokens <= 0 || heads <= 0) return 0;
  const int64_t splits = decode_splits(num_tokens, width);
  return static_cast<int64_t>(num_tokens) * splits * heads * (kDv + 2) * 4 + 256;
}

extern "C" int ekv_sparse_mla_decode(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                     int32_t num_tokens, int32_t heads, int32_t dim, const uint8_t* cache,
                                     int32_t cache_bf16, int64_t page_stride, int64_t num_pages,
                                     const int32_t* indices, int64_t idx_stride, int32_t width,
                                     const int32_t* lengths, const int32_t* block_table, int64_t bt_stride,
                                     const int32_t* req_ids, const float* sinks, float scale, uint16_t* out,
                                     int64_t out_tok_stride, int64_t out_head_stride, float* lse,
                                     int64_t lse_stride, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  EKV_CHECK(num_tokens >= 0 && width >= 0, "sizes must be >= 0");
  if (num_tokens == 0) return 0;
  EKV_CHECK(dim == 512 || dim == 576, "dim must be 512 or 576");
  EKV_CHECK(heads > 0 && heads % 16 == 0 && heads <= 16 * kMaxWaves, "heads must be a multiple of 16, <= 64");
  EKV_CHECK(q && cache && indices && out, "null pointer");
  EKV_CHECK(block_table == nullptr || req_ids != nullptr, "block_table needs req_ids");
  EKV_CHECK(q_tok_stride % 8 == 0 && q_head_stride % 8 == 0 && aligned16(q), "q must be 16-byte aligned rows");
  EKV_CHECK(out_tok_stride % 4 == 0 && out_head_stride % 4 == 0 && aligned8(out), "out rows must be 8-byte aligned");
  EKV_CHECK(cache_bf16 || (page_stride >= kPageTokens * (dim + 4) && page_stride % 16 == 0), "bad page_stride");
  EKV_CHECK(aligned16(cache), "cache must be 16-byte aligned");
  const int64_t need = ekv_sparse_mla_decode_workspace_size(num_tokens, heads, width);
  EKV_CHECK(workspace != nullptr, "workspace is null");
  if (workspace_bytes < need) {
    set_error("workspace too small (see ekv_sparse_mla_decode_workspace_size)");
    return kWorkspaceTooSmall;
  }
  const int splits = decode_splits(num_tokens, width);
  const int tiles = (width + kTile - 1) / kTile;
  const int per_split = ((tiles + splits - 1) / splits) * kTile;
  float* ws_o = static_cast<float*>(workspace);
  float* ws_ml = ws_o + static_cast<int64_t>(num_tokens) * splits * heads * kDv;
  DecodeArgs a{q, q_tok_stride, q_head_stride, cache, page_stride,
               num_pages * kPageTokens, cache_bf16, indices, idx_stride, width,
               lengths, block_table, bt_stride, req_ids, scale, heads, per_split, ws_o, ws_ml, splits};
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(splits, num_tokens);
  dim3 block(4 * heads);
  if (dim == 576) {
    const size_t smem = sizeof(DecodeSmem<576>);
    hipFuncSetAttribute(reinterpret_cast<const void*>(sparse_decode_kernel<576>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
    hipLaunchKernelGGL(sparse_decode_kernel<576>, grid, block, smem, s, a);
  } else {
    const size_t smem = sizeof(DecodeSmem<512>);
    hipFuncSetAttribute(reinterpret_cast<const void*>(sparse_decode_kernel<512>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
    hipLaunchKernelGGL(sparse_decode_kernel<512>, grid, block, smem, s, a);
  }
  int rc = ekv_launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(heads, num_tokens), dim3(128), 0, s, ws_o, ws_ml, splits, heads,
                     sinks, out, out_tok_stride, out_head_stride, lse, lse_stride);
  return ekv_launch_status();
}
