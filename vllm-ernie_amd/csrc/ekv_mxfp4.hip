// MXFP4 quantization and the MXFP4 indexer K insert.
//
// Format (OCP MX): groups of 32 values share one E8M0 scale byte; each value
// is an e2m1 code, two per byte with the even element in the low nibble.  A
// 128-wide indexer row is 64 packed bytes + 4 scale bytes = 68 bytes, stored
// in 64-token pages as all packed values first (row r at 64 r), then all
// scale bytes (row r at 64 * 64 + 4 r).
//
// Quantization of a group (restating triton_kernels' downcast_to_mxfp with
// the round-up scale mode, which nvidia/attention.py:990-1008 calls):
//   scale = 2^ceil(log2(amax / 6)): fl32(amax / 6) rounded up to a power of
//           two from its bits (E8M0 byte = that exponent field; 0 for amax 0);
//   y     = x * (1 / scale), exact, |y| <= 6;
//   code  = nearest e2m1 value, ties to the larger magnitude, sign kept.
// One thread per 32-value group: 64 bytes in, 16 bytes + 1 scale byte out.

#include "ekv_common.h"
#include "ekv_internal.h"

namespace ekv {
namespace {

constexpr int kFp4IdxDim = 128;
constexpr int kFp4IdxGroups = kFp4IdxDim / kMxBlock;   // 4
constexpr int kFp4ValueBytes = kFp4IdxDim / 2;         // 64
constexpr int kFp4PageValues = kPageTokens * kFp4ValueBytes;

// 32 bf16 values at p (16-byte aligned) -> 16 packed bytes; returns the
// scale byte.
__device__ __forceinline__ uint32_t mxfp4_group(const uint16_t* p, uint4& packed) {
  uint32_t raw[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 v = reinterpret_cast<const uint4*>(p)[j];
    raw[4 * j] = v.x;
    raw[4 * j + 1] = v.y;
    raw[4 * j + 2] = v.z;
    raw[4 * j + 3] = v.w;
  }
  float x[32];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    x[2 * i] = __uint_as_float(raw[i] << 16);
    x[2 * i + 1] = __uint_as_float(raw[i] & 0xffff0000u);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
  const uint32_t sb = mxfp4_scale_byte(amax);
  const float inv = sb ? __fdiv_rn(1.0f, __uint_as_float(sb << 23)) : 0.0f;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 32; ++i) w[i >> 3] |= e2m1_code(x[i] * inv) << (4 * (i & 7));
  packed = make_uint4(w[0], w[1], w[2], w[3]);
  return sb;
}

// Rows r = tok * heads + h of x (x + tok * tok_stride + h * head_stride), dim
// values each: values at values + r * values_stride (dim / 2 bytes), scale
// bytes at scales + r * scales_stride.  With w_out, the thread of group 0 of
// row r also writes w_out[r] = fl32(weights[tok, h] * fl32(128^-0.5 * 64^-0.5)).
struct Mxfp4RowsArgs {
  const uint16_t* x;
  int64_t tok_stride, head_stride;
  int32_t heads, groups;  // groups = dim / 32
  int64_t total;          // rows * groups
  uint8_t* values;
  int64_t values_stride;
  uint8_t* scales;
  int64_t scales_stride;
  const void* weights;
  int32_t weights_is_bf16;
  int64_t w_stride;
  float* w_out;
};

__global__ void __launch_bounds__(256) mxfp4_rows_kernel(Mxfp4RowsArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int64_t r = i / a.groups;
  const int grp = static_cast<int>(i - r * a.groups);
  const int64_t tok = r / a.heads, h = r - tok * a.heads;
  uint4 packed;
  const uint32_t sb = mxfp4_group(a.x + tok * a.tok_stride + h * a.head_stride + kMxBlock * grp, packed);
  *reinterpret_cast<uint4*>(a.values + r * a.values_stride + 16 * grp) = packed;
  a.scales[r * a.scales_stride + grp] = static_cast<uint8_t>(sb);
  if (a.w_out && grp == 0) {
    const float ws = 0x1.6a09e6p-7f;  // fl32(128**-0.5 * 64**-0.5)
    const int64_t wi = tok * a.w_stride + h;
    const float wv = a.weights_is_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(a.weights)[wi])
                                       : static_cast<const float*>(a.weights)[wi];
    a.w_out[r] = wv * ws;
  }
}

// K insert: row t of k (128 wide) into the page row of slot_mapping[t].
__global__ void __launch_bounds__(256) k_insert_fp4_kernel(const uint16_t* k, int64_t k_stride, int32_t num_tokens,
                                                           const int64_t* slots, uint8_t* kcache, int64_t page_stride,
                                                           int64_t num_pages) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(num_tokens) * kFp4IdxGroups) return;
  const int64_t t = i / kFp4IdxGroups;
  const int grp = static_cast<int>(i % kFp4IdxGroups);
  const int64_t slot = slots[t];
  if (slot < 0) return;  // padding token
  const int64_t page = slot / kPageTokens;
  if (page >= num_pages) return;
  const int off = static_cast<int>(slot % kPageTokens);
  uint4 packed;
  const uint32_t sb = mxfp4_group(k + t * k_stride + kMxBlock * grp, packed);
  uint8_t* base = kcache + page * page_stride;
  *reinterpret_cast<uint4*>(base + off * kFp4ValueBytes + 16 * grp) = packed;
  base[kFp4PageValues + off * kFp4IdxGroups + grp] = static_cast<uint8_t>(sb);
}

// Store of already quantized rows: byte j < 64 of row t is value byte j,
// 64 <= j < 68 scale byte j - 64.
__global__ void __launch_bounds__(256) store_fp4_kernel(const uint8_t* values, int64_t values_stride,
                                                        const uint8_t* scales, int64_t scales_stride,
                                                        int32_t num_tokens, const int64_t* slots, uint8_t* kcache,
                                                        int64_t page_stride, int64_t num_pages) {
  constexpr int kRow = kFp4ValueBytes + kFp4IdxGroups;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(num_tokens) * kRow) return;
  const int64_t t = i / kRow;
  const int j = static_cast<int>(i % kRow);
  const int64_t slot = slots[t];
  if (slot < 0) return;
  const int64_t page = slot / kPageTokens;
  if (page >= num_pages) return;
  const int off = static_cast<int>(slot % kPageTokens);
  uint8_t* base = kcache + page * page_stride;
  if (j < kFp4ValueBytes)
    base[off * kFp4ValueBytes + j] = values[t * values_stride + j];
  else
    base[kFp4PageValues + off * kFp4IdxGroups + (j - kFp4ValueBytes)] = scales[t * scales_stride + (j - kFp4ValueBytes)];
}

unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

}  // namespace
}  // namespace ekv

using namespace ekv;

extern "C" int ekv_mxfp4_quant(const uint16_t* x, int64_t x_tok_stride, int64_t x_head_stride, int32_t num_tokens,
                               int32_t heads, int32_t dim, uint8_t* values, int64_t values_stride, uint8_t* scales,
                               int64_t scales_stride, void* stream) {
  EKV_CHECK(num_tokens >= 0 && heads > 0 && dim > 0 && dim % kMxBlock == 0, "dim must be a positive multiple of 32");
  if (num_tokens == 0) return 0;
  EKV_CHECK(x && values && scales, "null pointer");
  EKV_CHECK(aligned16(x) && x_tok_stride % 8 == 0 && x_head_stride % 8 == 0,
            "x must be 16-byte aligned with strides that are multiples of 8 elements");
  EKV_CHECK(aligned16(values) && values_stride % 16 == 0 && values_stride >= dim / 2,
            "values must be 16-byte aligned with a stride of >= dim / 2 bytes, a multiple of 16");
  EKV_CHECK(scales_stride >= dim / kMxBlock, "scales_stride must be >= dim / 32");
  const int64_t total = static_cast<int64_t>(num_tokens) * heads * (dim / kMxBlock);
  Mxfp4RowsArgs a{x, x_tok_stride, x_head_stride, heads, dim / kMxBlock, total, values, values_stride, scales,
                  scales_stride, nullptr, 0, 0, nullptr};
  hipLaunchKernelGGL(mxfp4_rows_kernel, dim3(blocks_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_q_quant_fp4(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                       const void* weights, int32_t weights_is_bf16, int64_t w_stride,
                                       int32_t num_tokens, int32_t heads, uint8_t* q_values, int32_t* q_scales,
                                       float* w_out, void* stream) {
  EKV_CHECK(num_tokens >= 0 && heads > 0, "bad sizes");
  if (num_tokens == 0) return 0;
  EKV_CHECK(q && weights && q_values && q_scales && w_out, "null pointer");
  EKV_CHECK(aligned16(q) && q_tok_stride % 8 == 0 && q_head_stride % 8 == 0,
            "q must be 16-byte aligned with strides that are multiples of 8 elements");
  EKV_CHECK(aligned16(q_values) && aligned4(q_scales), "misaligned q_values / q_scales");
  EKV_CHECK(w_stride >= heads, "w_stride must be >= heads");
  const int64_t total = static_cast<int64_t>(num_tokens) * heads * kFp4IdxGroups;
  Mxfp4RowsArgs a{q, q_tok_stride, q_head_stride, heads, kFp4IdxGroups, total, q_values, kFp4ValueBytes,
                  reinterpret_cast<uint8_t*>(q_scales), kFp4IdxGroups, weights, weights_is_bf16, w_stride, w_out};
  hipLaunchKernelGGL(mxfp4_rows_kernel, dim3(blocks_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_k_insert_fp4(const uint16_t* k, int64_t k_stride, int32_t num_tokens,
                                        const int64_t* slot_mapping, uint8_t* kcache, int64_t page_stride,
                                        int64_t num_pages, void* stream) {
  EKV_CHECK(num_tokens >= 0 && num_pages >= 0, "bad sizes");
  if (num_tokens == 0) return 0;
  EKV_CHECK(k && slot_mapping && kcache, "null pointer");
  EKV_CHECK(aligned16(k) && k_stride % 8 == 0 && k_stride >= kFp4IdxDim,
            "k must be 16-byte aligned with a stride of >= 128 elements, a multiple of 8");
  EKV_CHECK(aligned16(kcache) && page_stride % 16 == 0 && page_stride >= kPageTokens * (kFp4ValueBytes + 4),
            "kcache must be 16-byte aligned with a page stride of >= 64 * 68 bytes, a multiple of 16");
  const int64_t total = static_cast<int64_t>(num_tokens) * kFp4IdxGroups;
  hipLaunchKernelGGL(k_insert_fp4_kernel, dim3(blocks_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), k,
                     k_stride, num_tokens, slot_mapping, kcache, page_stride, num_pages);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_store_fp4(const uint8_t* values, int64_t values_stride, const uint8_t* scales,
                                     int64_t scales_stride, int32_t num_tokens, const int64_t* slot_mapping,
                                     uint8_t* kcache, int64_t page_stride, int64_t num_pages, void* stream) {
  EKV_CHECK(num_tokens >= 0 && num_pages >= 0, "bad sizes");
  if (num_tokens == 0) return 0;
  EKV_CHECK(values && scales && slot_mapping && kcache, "null pointer");
  EKV_CHECK(values_stride >= kFp4ValueBytes && scales_stride >= kFp4IdxGroups, "row strides too small");
  EKV_CHECK(page_stride >= kPageTokens * (kFp4ValueBytes + 4), "page_stride must be >= 64 * 68 bytes");
  const int64_t total = static_cast<int64_t>(num_tokens) * (kFp4ValueBytes + kFp4IdxGroups);
  hipLaunchKernelGGL(store_fp4_kernel, dim3(blocks_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), values,
                     values_stride, scales, scales_stride, num_tokens, slot_mapping, kcache, page_stride, num_pages);
  return ekv_launch_status();
}
