// Latent page transcoders between this library's fp8 page and vLLM's
// fp8_ds_mla page (the FlashMLA sparse KV dtype), for KV connectors that move
// pages in the upstream format.
//
// Own page (576-wide latent): 64 rows of 576 e4m3fn codes, then 64 fp32
// per-row power-of-two scales.  fp8_ds_mla page: 64 token-major rows of 656
// bytes -- 512 e4m3fn codes (dims 0..511), four fp32 scales (scale t for dims
// 128t .. 128t+127), 64 bf16 values (dims 512..575).
//
// Export (own -> ds_mla) is lossless: codes 0..511 are copied, the row scale
// fills the four tile slots, and dims 512..575 become bf16 exactly (an e4m3
// value times a power of two).  Import (ds_mla -> own) dequantizes the row in
// fp32 (code * tile scale; bf16 as is) and quantizes it as the row append
// does: one UE8M0 scale per row, round to nearest even.
// One wave per row: export writes 41 16-byte chunks of the 656-byte row;
// import gives each lane 8 codes of dims 0..511 and one bf16 of 512..575.

#include "ekv_common.h"
#include "ekv_internal.h"

namespace ekv {
namespace {

constexpr int kOwnDim = 576;
constexpr int kNope = 512;
constexpr int kDsRow = 656;
constexpr int kDsScales = kNope;        // byte offset of the tile scales
constexpr int kDsRope = kNope + 16;     // byte offset of the bf16 dims
constexpr int kRowsPerBlock = 4;        // one wave per row

struct PageMap {
  const uint8_t* src;
  int64_t src_stride, src_pages;
  const int32_t* src_ids;
  uint8_t* dst;
  int64_t dst_stride, dst_pages;
  const int32_t* dst_ids;  // null: page i of the call goes to dst page i
  int32_t n;
};

// Source and destination page bases of item i, or false when either id is
// out of range (the item is skipped).
__device__ __forceinline__ bool map_pages(const PageMap& m, int i, const uint8_t*& s, uint8_t*& d) {
  const int64_t sp = m.src_ids[i];
  const int64_t dp = m.dst_ids ? static_cast<int64_t>(m.dst_ids[i]) : static_cast<int64_t>(i);
  if (sp < 0 || sp >= m.src_pages || dp < 0 || dp >= m.dst_pages) return false;
  s = m.src + sp * m.src_stride;
  d = m.dst + dp * m.dst_stride;
  return true;
}

__global__ void __launch_bounds__(64 * kRowsPerBlock) export_ds_mla_kernel(PageMap m) {
  const int item = blockIdx.x / (kPageTokens / kRowsPerBlock);
  const int r = (blockIdx.x % (kPageTokens / kRowsPerBlock)) * kRowsPerBlock + (threadIdx.x >> 6);
  const int c = threadIdx.x & 63;  // 16-byte chunk of the output row
  const uint8_t* src;
  uint8_t* dst;
  if (item >= m.n || c >= kDsRow / 16 || !map_pages(m, item, src, dst)) return;
  const uint8_t* row = src + r * kOwnDim;
  const float scale = *reinterpret_cast<const float*>(src + kPageTokens * kOwnDim + r * 4);
  uint4 v;
  if (c < kNope / 16) {
    v = *reinterpret_cast<const uint4*>(row + 16 * c);
  } else if (c == kNope / 16) {
    const uint32_t sb = __float_as_uint(scale);
    v = make_uint4(sb, sb, sb, sb);
  } else {  // dims 512 + 8j .. +8 to bf16
    const int j = c - kNope / 16 - 1;
    const uint2 codes = *reinterpret_cast<const uint2*>(row + kNope + 8 * j);
    const f32x4 a = fp8x4_to_f32(codes.x), b = fp8x4_to_f32(codes.y);
    auto pk = [&](float x, float y) {
      return static_cast<uint32_t>(f32_to_bf16(x * scale)) | (static_cast<uint32_t>(f32_to_bf16(y * scale)) << 16);
    };
    v = make_uint4(pk(a[0], a[1]), pk(a[2], a[3]), pk(b[0], b[1]), pk(b[2], b[3]));
  }
  *reinterpret_cast<uint4*>(dst + r * kDsRow + 16 * c) = v;
}

__global__ void __launch_bounds__(64 * kRowsPerBlock) import_ds_mla_kernel(PageMap m) {
  const int item = blockIdx.x / (kPageTokens / kRowsPerBlock);
  const int r = (blockIdx.x % (kPageTokens / kRowsPerBlock)) * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const uint8_t* src;
  uint8_t* dst;
  if (item >= m.n || !map_pages(m, item, src, dst)) return;
  const uint8_t* row = src + r * kDsRow;
  const float tile = *reinterpret_cast<const float*>(row + kDsScales + 4 * (lane >> 4));  // dims 8 lane ..
  const uint2 codes = *reinterpret_cast<const uint2*>(row + 8 * lane);
  const f32x4 a = fp8x4_to_f32(codes.x), b = fp8x4_to_f32(codes.y);
  float v[9] = {a[0] * tile, a[1] * tile, a[2] * tile, a[3] * tile,
                b[0] * tile, b[1] * tile, b[2] * tile, b[3] * tile,
                bf16_to_f32(*reinterpret_cast<const uint16_t*>(row + kDsRope + 2 * lane))};
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 9; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = wave_max_xor(amax, 64);
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  const uint32_t lo = f32x2_to_fp8(v[0] * inv, v[1] * inv) | (f32x2_to_fp8(v[2] * inv, v[3] * inv) << 16);
  const uint32_t hi = f32x2_to_fp8(v[4] * inv, v[5] * inv) | (f32x2_to_fp8(v[6] * inv, v[7] * inv) << 16);
  uint8_t* out = dst + r * kOwnDim;
  *reinterpret_cast<uint2*>(out + 8 * lane) = make_uint2(lo, hi);
  out[kNope + lane] = static_cast<uint8_t>(f32x2_to_fp8(v[8] * inv, 0.0f) & 0xffu);
  if (lane == 0) *reinterpret_cast<float*>(dst + kPageTokens * kOwnDim + r * 4) = exp2i(e);
}

int check_map(const PageMap& m, int64_t src_min, int64_t dst_min) {
  EKV_CHECK(m.n >= 0 && m.src_pages >= 0 && m.dst_pages >= 0, "bad sizes");
  if (m.n == 0) return 0;
  EKV_CHECK(m.src && m.dst && m.src_ids, "null pointer");
  EKV_CHECK(aligned16(m.src) && aligned16(m.dst) && m.src_stride % 16 == 0 && m.dst_stride % 16 == 0,
            "pages must be 16-byte aligned with strides that are multiples of 16");
  EKV_CHECK(m.src_stride >= src_min && m.dst_stride >= dst_min, "page stride too small for 64 rows");
  return 0;
}

}  // namespace
}  // namespace ekv

using namespace ekv;

extern "C" int ekv_export_fp8_ds_mla_pages(const uint8_t* cache, int64_t page_stride, int64_t num_pages,
                                           const int32_t* src_pages, int32_t n, uint8_t* out,
                                           int64_t out_page_stride, int64_t out_num_pages,
                                           const int32_t* dst_pages, void* stream) {
  const PageMap m{cache, page_stride, num_pages, src_pages, out, out_page_stride, out_num_pages, dst_pages, n};
  int rc = check_map(m, int64_t{kPageTokens} * (kOwnDim + 4), int64_t{kPageTokens} * kDsRow);
  if (rc || n == 0) return rc;
  hipLaunchKernelGGL(export_ds_mla_kernel, dim3(static_cast<unsigned>(n) * (kPageTokens / kRowsPerBlock)),
                     dim3(64 * kRowsPerBlock), 0, static_cast<hipStream_t>(stream), m);
  return ekv_launch_status();
}

extern "C" int ekv_import_fp8_ds_mla_pages(const uint8_t* src, int64_t src_page_stride, int64_t src_num_pages,
                                           const int32_t* src_pages, int32_t n, uint8_t* cache, int64_t page_stride,
                                           int64_t num_pages, const int32_t* dst_pages, void* stream) {
  const PageMap m{src, src_page_stride, src_num_pages, src_pages, cache, page_stride, num_pages, dst_pages, n};
  int rc = check_map(m, int64_t{kPageTokens} * kDsRow, int64_t{kPageTokens} * (kOwnDim + 4));
  if (rc || n == 0) return rc;
  hipLaunchKernelGGL(import_ds_mla_kernel, dim3(static_cast<unsigned>(n) * (kPageTokens / kRowsPerBlock)),
                     dim3(64 * kRowsPerBlock), 0, static_cast<hipStream_t>(stream), m);
  return ekv_launch_status();
}
