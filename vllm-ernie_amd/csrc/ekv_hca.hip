// HCA 128->1 span compressor (the C128 compression of an HCA layer).
//
// One workgroup per span that completes in this call: the span's 128 rows of
// kv_score (the compressor projection [kv | score], bf16) come from this
// call's input for positions >= the sequence's first new position, and from
// the per-sequence state ring (positions % 256) for earlier positions.  Per
// channel c the workgroup forms
//
//   g_i = score_i[c] + ape[i, c];  m = max_i g_i;  e_i = exp_ekv(g_i - m)
//   Z = sum_i e_i;  N = sum_i e_i * kv_i[c]   (sequential over i, fp32)
//   x_c = N / Z
//
// then RMSNorm over the row (sum of squares: per thread over its 4 channels,
// then thread 0 over the threads in order), interleaved RoPE on the last 64
// channels at position 128*j (cos/sin table row j), and the per-token UE8M0
// fp8 quant; the row is written to the compressed page slot of span j.
//
// Must run before ekv_hca_append of the same call (the append overwrites the
// state ring rows this kernel may still read).  Built with -ffp-contract=off
// and correctly rounded fp32 division / square root: the CPU oracle evaluates
// the same operations in the same order.
#include "ekv_common.h"
#include "ekv_internal.h"

namespace ekv {

// exp(x) for x <= 0 as 2**n * P(f): n = rint(x * log2 e), f = x * log2 e - n,
// P = degree-6 Taylor polynomial of 2**f (coefficients ln2^k / k!), Horner.
__device__ __forceinline__ float exp_ekv(float x) {
  const float t = x * 0x1.715476p+0f;
  if (t < -125.0f) return 0.0f;
  const float n = rintf(t);
  const float f = t - n;
  float p = 0x1.430912p-13f;
  p = p * f + 0x1.5d87fep-10f;
  p = p * f + 0x1.3b2ab6p-7f;
  p = p * f + 0x1.c6b08ep-5f;
  p = p * f + 0x1.ebfbe0p-3f;
  p = p * f + 0x1.62e430p-1f;
  p = p * f + 0x1.0p+0f;
  return ldexpf(p, static_cast<int>(n));
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
};

template <int D>
__global__ void __launch_bounds__(256) hca_compress_kernel(CompressArgs a) {
  constexpr int kThreads = D / 4;  // threads owning 4 channels each
  __shared__ float s_part[kThreads];
  __shared__ float s_bcast[2];
  const int tid = threadIdx.x;
  const int b = blockIdx.y;
  const int t0 = a.qsl[b];
  const int n = a.qsl[b + 1] - t0;
  if (n <= 0) return;
  const int64_t p0 = a.positions[t0];
  const int64_t pl = p0 + n - 1;
  const int64_t j = p0 / kSpan + blockIdx.x;
  if (j * kSpan + kSpan - 1 > pl) return;  // span not completed by this call
  if (j >= a.max_spans) return;
  const int st = a.state_slot != nullptr ? a.state_slot[b] : -1;
  const bool active = tid < kThreads;
  const int c0 = 4 * tid;

  auto row_ptr = [&](int i) -> const uint16_t* {
    const int64_t p = j * kSpan + i;
    if (p >= p0) return a.kv_score + (t0 + (p - p0)) * a.kvs_stride;
    if (st < 0 || st >= a.num_state) return nullptr;
    return a.state + (static_cast<int64_t>(st) * kStateRing + p % kStateRing) * (2 * D);
  };

  float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  if (active) {
    for (int i = 0; i < kSpan; ++i) {
      const uint16_t* r = row_ptr(i);
      const uint2 sv = r ? *reinterpret_cast<const uint2*>(r + D + c0) : make_uint2(0, 0);
      const float4 ap = *reinterpret_cast<const float4*>(a.ape + i * D + c0);
      const float g0 = __uint_as_float(sv.x << 16) + ap.x;
      const float g1 = __uint_as_float(sv.x & 0xffff0000u) + ap.y;
      const float g2 = __uint_as_float(sv.y << 16) + ap.z;
      const float g3 = __uint_as_float(sv.y & 0xffff0000u) + ap.w;
      m[0] = fmaxf(m[0], g0); m[1] = fmaxf(m[1], g1); m[2] = fmaxf(m[2], g2); m[3] = fmaxf(m[3], g3);
    }
  }
  float Z[4] = {0.f, 0.f, 0.f, 0.f}, N[4] = {0.f, 0.f, 0.f, 0.f};
  if (active) {
    for (int i = 0; i < kSpan; ++i) {
      const uint16_t* r = row_ptr(i);
      const uint2 sv = r ? *reinterpret_cast<const uint2*>(r + D + c0) : make_uint2(0, 0);
      const uint2 kv = r ? *reinterpret_cast<const uint2*>(r + c0) : make_uint2(0, 0);
      const float4 ap = *reinterpret_cast<const float4*>(a.ape + i * D + c0);
      const float g[4] = {__uint_as_float(sv.x << 16) + ap.x, __uint_as_float(sv.x & 0xffff0000u) + ap.y,
                          __uint_as_float(sv.y << 16) + ap.z, __uint_as_float(sv.y & 0xffff0000u) + ap.w};
      const float v[4] = {__uint_as_float(kv.x << 16), __uint_as_float(kv.x & 0xffff0000u),
                          __uint_as_float(kv.y << 16), __uint_as_float(kv.y & 0xffff0000u)};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float e = exp_ekv(g[k] - m[k]);
        Z[k] = Z[k] + e;
        N[k] = N[k] + e * v[k];
      }
    }
  }
  float x[4];
  float part = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    x[k] = active ? __fdiv_rn(N[k], Z[k]) : 0.0f;
    part = part + x[k] * x[k];
  }
  if (active) s_part[tid] = part;
  __syncthreads();
  if (tid == 0) {
    float S = 0.0f;
    for (int i = 0; i < kThreads; ++i) S = S + s_part[i];
    const float ms = __fdiv_rn(S, static_cast<float>(D));
    s_bcast[0] = __fdiv_rn(1.0f, __fsqrt_rn(ms + a.eps));
  }
  __syncthreads();
  const float rn = s_bcast[0];
  float y[4] = {0.f, 0.f, 0.f, 0.f};
  float amax = 0.0f;
  if (active) {
    const float4 w = *reinterpret_cast<const float4*>(a.norm_w + c0);
    y[0] = (x[0] * rn) * w.x; y[1] = (x[1] * rn) * w.y; y[2] = (x[2] * rn) * w.z; y[3] = (x[3] * rn) * w.w;
    if (c0 >= D - 64) {
      const float* cs = a.cos_sin + j * 64;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int pi = (c0 - (D - 64)) / 2 + q;
        const float c = cs[pi], s = cs[32 + pi];
        const float x0 = y[2 * q], x1 = y[2 * q + 1];
        y[2 * q] = x0 * c - x1 * s;
        y[2 * q + 1] = x0 * s + x1 * c;
      }
    }
    amax = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
  }
  // block max of amax (order-free): wave reduce, then 4 wave partials
  amax = wave_max_xor(amax, 64);
  __shared__ float s_wmax[4];
  if ((tid & 63) == 0) s_wmax[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(s_wmax[0], s_wmax[1]), fmaxf(s_wmax[2], s_wmax[3]));
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  const int64_t slot = static_cast<int64_t>(a.comp_bt[static_cast<int64_t>(b) * a.comp_bt_stride + j / kPageTokens]) *
                           kPageTokens + j % kPageTokens;
  if (slot < 0 || slot >= a.num_pages * kPageTokens) return;
  uint8_t* page = a.pool + (slot / kPageTokens) * a.page_stride;
  const int64_t off = slot % kPageTokens;
  if (active) {
    const uint32_t lo = f32x2_to_fp8(y[0] * inv, y[1] * inv);
    const uint32_t hi = f32x2_to_fp8(y[2] * inv, y[3] * inv);
    *reinterpret_cast<uint32_t*>(page + off * D + c0) = lo | (hi << 16);
  }
  if (tid == 0) *reinterpret_cast<float*>(page + kPageTokens * D + off * 4) = exp2i(e);
}

}  // namespace ekv

using namespace ekv;

extern "C" int ekv_hca_compress(const uint16_t* kv_score, int64_t kvs_stride, const int64_t* positions,
                                const int32_t* qsl, int32_t num_seqs, int32_t max_query_len, int32_t dim,
                                const uint16_t* state, const int32_t* state_slot, int32_t num_state,
                                const float* ape, const float* norm_w, float eps, const float* cos_sin,
                                int32_t max_spans, const int32_t* comp_block_table, int32_t comp_bt_stride,
                                uint8_t* pool, int64_t page_stride, int64_t num_pages, void* stream) {
  EKV_CHECK(num_seqs >= 0 && max_query_len >= 0, "sizes must be >= 0");
  if (num_seqs == 0 || max_query_len == 0) return 0;
  EKV_CHECK(dim == 512 || dim == 576, "HCA dim must be 512 or 576");
  EKV_CHECK(kv_score && positions && qsl && ape && norm_w && cos_sin && comp_block_table && pool,
            "null pointer");
  EKV_CHECK(kvs_stride >= 2 * dim && kvs_stride % 4 == 0, "kv_score stride must be >= 2*dim, multiple of 4");
  EKV_CHECK(page_stride >= kPageTokens * (dim + 4) && page_stride % 16 == 0, "bad page_stride");
  EKV_CHECK(aligned16(ape) && aligned16(norm_w) && aligned8(kv_score) && aligned16(pool) &&
                (state == nullptr || aligned8(state)),
            "misaligned buffers");
  CompressArgs a{kv_score, kvs_stride, positions, qsl, state, state_slot, num_state, ape, norm_w, eps,
                 cos_sin, max_spans, comp_block_table, comp_bt_stride, pool, page_stride, num_pages};
  // spans that can complete among max_query_len new positions
  const int spans = max_query_len / kSpan + 1;
  dim3 grid(spans, num_seqs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dim == 512) hipLaunchKernelGGL(hca_compress_kernel<512>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(hca_compress_kernel<576>, grid, dim3(256), 0, s, a);
  return ekv_launch_status();
}
