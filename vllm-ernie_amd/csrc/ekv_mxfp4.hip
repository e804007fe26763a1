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
#include "ekv_rows.h"

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

// ---------------------------------------------------------------------------
// DSA decode prologue with MXFP4 indexer keys: the indexer prep of q and k
// (with cos_sin), the MXFP4 K insert, the MXFP4 q quant with the weight
// fold, the latent append and the windowed lengths, in one launch.  A
// 128-wide row is held by a 16-lane group (lane j: elements 8j .. 8j+7, the
// prep's layout); the 32-value group g is lanes 4g .. 4g+3, whose max is
// exchanged between them, and lane j's 8 codes are word j % 4 of the group's
// 16 packed bytes -- the bytes of mxfp4_group.
// ---------------------------------------------------------------------------
struct DsaPrologueFp4Args {
  AppendArgs k_rows;         // indexer K rows -> MXFP4 rows of kcache (prep fields with cos_sin)
  AppendArgs latent;         // latent rows -> fp8 rows of cache
  const uint16_t* q;         // [T, heads, 128] bf16
  int64_t q_tok_stride, q_head_stride;
  const void* w;
  int32_t w_is_bf16;
  int64_t w_stride;
  int32_t heads;
  uint8_t* q_values;         // [T, heads, 64]
  int32_t* q_scales;         // [T, heads] (byte g: group g)
  float* w_out;              // [T, heads]
  const float* cos_sin;      // [cs_rows, 64] or null (no prep)
  int32_t cs_rows;
  const int64_t* positions;  // [T]
  int32_t window;
  int32_t* lengths;          // [T]
  int32_t q_blocks, k_blocks, latent_blocks;
};

// MXFP4 of the row in v (lane j of its 16-lane group): lane j's packed word
// and, for its group, the scale byte.
__device__ __forceinline__ uint32_t mxfp4_lane(const float (&v)[8], uint32_t& sb) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  sb = mxfp4_scale_byte(amax);
  const float inv = sb ? __fdiv_rn(1.0f, __uint_as_float(sb << 23)) : 0.0f;
  uint32_t w = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) w |= e2m1_code(v[i] * inv) << (4 * i);
  return w;
}

template <int D>
__global__ void __launch_bounds__(256) dsa_prologue_fp4_kernel(DsaPrologueFp4Args a) {
  int b = blockIdx.x;
  const int j = threadIdx.x & 15;
  const int T = a.k_rows.num_tokens;
  if (b < a.q_blocks) {  // q rows (token, head), 16 per workgroup
    const int64_t row = static_cast<int64_t>(b) * 16 + (threadIdx.x >> 4);
    if (row >= static_cast<int64_t>(T) * a.heads) return;  // (whole 16-lane groups)
    const int64_t t = row / a.heads;
    const int h = static_cast<int>(row % a.heads);
    float v[8];
    unpack_bf16x8(*reinterpret_cast<const uint4*>(a.q + t * a.q_tok_stride + h * a.q_head_stride + 8 * j), v);
    if (a.cos_sin != nullptr) {
      const int64_t pos = a.positions[t];
      row_rope_neox64(v, (pos >= 0 && pos < a.cs_rows) ? a.cos_sin + pos * 64 : nullptr, j);
      row_hadamard(v, j);
    }
    uint32_t sb;
    const uint32_t w = mxfp4_lane(v, sb);
    *reinterpret_cast<uint32_t*>(a.q_values + row * kFp4ValueBytes + 4 * j) = w;
    if ((j & 3) == 0) reinterpret_cast<uint8_t*>(a.q_scales)[row * 4 + (j >> 2)] = static_cast<uint8_t>(sb);
    if (j == 0) {
      const int64_t wi = t * a.w_stride + h;
      const float wv = a.w_is_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(a.w)[wi])
                                   : static_cast<const float*>(a.w)[wi];
      a.w_out[row] = wv * 0x1.6a09e6p-7f;  // fl32(128**-0.5 * 64**-0.5)
    }
    return;
  }
  b -= a.q_blocks;
  if (b < a.k_blocks) {  // indexer K rows, 16 per workgroup
    const AppendArgs& k = a.k_rows;
    const int64_t t = static_cast<int64_t>(b) * 16 + (threadIdx.x >> 4);
    if (t >= T) return;
    float v[8];
    unpack_bf16x8(*reinterpret_cast<const uint4*>(k.rows + t * k.row_stride + 8 * j), v);
    if (k.cos_sin != nullptr) {
      const int64_t pos = k.positions[t];
      row_layer_norm(v, k.ln_w, k.ln_b, k.eps, j);
      row_rope_neox64(v, (pos >= 0 && pos < k.cs_rows) ? k.cos_sin + pos * 64 : nullptr, j);
      row_hadamard(v, j);
    }
    uint32_t sb;
    const uint32_t w = mxfp4_lane(v, sb);
    const int64_t slot = k.slot_mapping[t];
    if (slot < 0) return;  // padding token
    const int64_t page = slot / kPageTokens;
    if (page >= k.num_pages) return;
    const int off = static_cast<int>(slot % kPageTokens);
    uint8_t* base = k.cache + page * k.page_stride;
    *reinterpret_cast<uint32_t*>(base + off * kFp4ValueBytes + 4 * j) = w;
    if ((j & 3) == 0) base[kFp4PageValues + off * kFp4IdxGroups + (j >> 2)] = static_cast<uint8_t>(sb);
    return;
  }
  b -= a.k_blocks;
  if (b < a.latent_blocks) {
    append_rows<D, 1>(a.latent, b);
    return;
  }
  b -= a.latent_blocks;
  const int i = b * 256 + threadIdx.x;
  if (i < T) a.lengths[i] = static_cast<int32_t>(max(a.positions[i] + 1 - a.window, static_cast<int64_t>(0)));
}

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

extern "C" int ekv_dsa_decode_prologue_fp4(const uint16_t* k, int64_t k_stride, uint8_t* kcache, int64_t k_page_stride,
                                           int64_t k_num_pages, const uint16_t* latent, int64_t latent_stride,
                                           int32_t dim, uint8_t* cache, int64_t page_stride, int64_t num_pages,
                                           const int64_t* slot_mapping, int32_t num_tokens, const uint16_t* q,
                                           int64_t q_tok_stride, int64_t q_head_stride, const void* weights,
                                           int32_t weights_is_bf16, int64_t w_stride, int32_t heads,
                                           uint8_t* q_values, int32_t* q_scales, float* w_out,
                                           const int64_t* positions, int32_t window, int32_t* lengths,
                                           const float* ln_w, const float* ln_b, float eps, const float* cos_sin,
                                           int32_t cos_sin_rows, void* stream) {
  EKV_CHECK(num_tokens >= 0 && window >= 0 && heads > 0, "bad sizes");
  EKV_CHECK(cos_sin == nullptr || (ln_w && ln_b && cos_sin_rows >= 0 && aligned16(ln_w) && aligned16(ln_b) &&
                                   aligned16(cos_sin)),
            "the indexer prep needs 16-byte aligned ln_w, ln_b and cos_sin");
  if (num_tokens == 0) return 0;
  EKV_CHECK(dim == 512 || dim == 576, "latent dim must be 512 or 576");
  EKV_CHECK(k && slot_mapping && kcache && latent && cache && q && weights && q_values && q_scales && w_out &&
                positions && lengths,
            "null pointer");
  EKV_CHECK(aligned16(k) && k_stride % 8 == 0 && k_stride >= kFp4IdxDim,
            "k must be 16-byte aligned with a stride of >= 128 elements, a multiple of 8");
  EKV_CHECK(aligned16(kcache) && k_page_stride % 16 == 0 && k_page_stride >= kPageTokens * (kFp4ValueBytes + 4),
            "kcache must be 16-byte aligned with a page stride of >= 64 * 68 bytes, a multiple of 16");
  EKV_CHECK(latent_stride >= dim && latent_stride % 8 == 0 && aligned16(latent) && aligned16(cache) &&
                page_stride >= kPageTokens * (dim + 4) && page_stride % 16 == 0,
            "latent rows and cache must be 16-byte aligned, page_stride >= 64 rows + 64 scales");
  EKV_CHECK(aligned16(q) && q_tok_stride % 8 == 0 && q_head_stride % 8 == 0,
            "q must be 16-byte aligned with strides that are multiples of 8 elements");
  EKV_CHECK(aligned16(q_values) && aligned4(q_scales), "misaligned q_values / q_scales");
  EKV_CHECK(w_stride >= heads, "w_stride must be >= heads");
  DsaPrologueFp4Args a{};
  a.k_rows.rows = k;
  a.k_rows.row_stride = k_stride;
  a.k_rows.num_tokens = num_tokens;
  a.k_rows.slot_mapping = slot_mapping;
  a.k_rows.cache = kcache;
  a.k_rows.page_stride = k_page_stride;
  a.k_rows.num_pages = k_num_pages;
  if (cos_sin != nullptr) {
    a.k_rows.positions = positions;
    a.k_rows.ln_w = ln_w;
    a.k_rows.ln_b = ln_b;
    a.k_rows.eps = eps;
    a.k_rows.cos_sin = cos_sin;
    a.k_rows.cs_rows = cos_sin_rows;
  }
  a.latent.rows = latent;
  a.latent.row_stride = latent_stride;
  a.latent.num_tokens = num_tokens;
  a.latent.slot_mapping = slot_mapping;
  a.latent.cache = cache;
  a.latent.page_stride = page_stride;
  a.latent.num_pages = num_pages;
  a.q = q;
  a.q_tok_stride = q_tok_stride;
  a.q_head_stride = q_head_stride;
  a.w = weights;
  a.w_is_bf16 = weights_is_bf16;
  a.w_stride = w_stride;
  a.heads = heads;
  a.q_values = q_values;
  a.q_scales = q_scales;
  a.w_out = w_out;
  a.cos_sin = cos_sin;
  a.cs_rows = cos_sin_rows;
  a.positions = positions;
  a.window = window;
  a.lengths = lengths;
  const int64_t q_rows = static_cast<int64_t>(num_tokens) * heads;
  EKV_CHECK(q_rows < (int64_t{1} << 34), "too many q rows");
  a.q_blocks = static_cast<int32_t>((q_rows + 15) / 16);
  a.k_blocks = (num_tokens + 15) / 16;
  a.latent_blocks = (num_tokens + append_block_rows(dim, 1) - 1) / append_block_rows(dim, 1);
  const int len_blocks = (num_tokens + 255) / 256;
  const dim3 grid(static_cast<unsigned>(a.q_blocks + a.k_blocks + a.latent_blocks + len_blocks));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dim == 576) hipLaunchKernelGGL(dsa_prologue_fp4_kernel<576>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(dsa_prologue_fp4_kernel<512>, grid, dim3(256), 0, s, a);
  return ekv_launch_status();
}
