// Write-side and small kernels of the ERNIE KV-cache path.
//
//  * kv_append_quant   latent / indexer-K append: bf16 row -> per-token UE8M0
//                      fp8 row scattered by slot (values-then-scales pages),
//                      optionally also into the window ring and the
//                      compressor state ring (HCA layers).
//  * merge_swa_topk    [topk[:n] | seq-w .. seq-1 | -1 ...] per row.
//  * hadamard_rows     orthonormal Sylvester Walsh-Hadamard of 128-wide rows.
//  * indexer_q_quant   per-(token, head) UE8M0 fp8 q, scale folded into the
//                      head weights, plus the int8 digit planes of q used by
//                      the exact scorer.
//  * windowed_lengths  indexer candidate count max(pos + 1 - window, 0).
//  * hca_decode_indices  [compressed slots | window ring slots | -1 ...].
//
// Built with -ffp-contract=off: the arithmetic is mirrored bit for bit by the
// CPU oracle, so no multiply-add may be fused behind its back.
#include "ekv_common.h"
#include "ekv_internal.h"

#include <algorithm>
#include "ekv_rows.h"

namespace ekv {

template <int D>
__global__ void __launch_bounds__(256) kv_append_quant_kernel(AppendArgs a) {
  append_rows<D, kAppendSeq<D>>(a, blockIdx.x);
}

// HCA append over the grid of hca_append_grid.
template <int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8)))
hca_append_kernel(AppendArgs a, int main_blocks, int tail_rows) {
  hca_append_block<D>(a, static_cast<int>(blockIdx.x), main_blocks, tail_rows);
}

// ---------------------------------------------------------------------------
// merge_swa_topk   (attention.py:582-641)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) merge_swa_topk_kernel(
    const int32_t* topk, int64_t topk_stride, int32_t* out, int64_t out_stride,
    const int64_t* positions, int32_t k, int32_t width, int32_t window) {
  const int64_t row = blockIdx.x;
  const int64_t seq = positions[row] + 1;
  const int64_t n = min(max(seq - window, static_cast<int64_t>(0)), static_cast<int64_t>(k));
  const int64_t w = min(seq, static_cast<int64_t>(window));
  for (int c = threadIdx.x; c < width; c += blockDim.x) {
    int64_t v;
    if (c < n) v = topk[row * topk_stride + c];
    else if (c < n + w) v = seq - w + (c - n);
    else v = -1;
    out[row * out_stride + c] = static_cast<int32_t>(v);
  }
}

// ---------------------------------------------------------------------------
// hadamard_rows: one wave per 128-wide row; lane l holds elements 2l, 2l+1.
// Butterfly spans 1, 2, ..., 64 with (a, b) -> (a + b, a - b), then times
// fl32(1/sqrt(128)), rounded to bf16.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) hadamard_rows_kernel(
    const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, int32_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const uint32_t w = *reinterpret_cast<const uint32_t*>(x + r * x_stride + 2 * lane);
  float e0 = __uint_as_float(w << 16);
  float e1 = __uint_as_float(w & 0xffff0000u);
  float a0 = e0 + e1, a1 = e0 - e1;  // span 1, in-lane
  e0 = a0; e1 = a1;
#pragma unroll
  for (int h = 2; h < 128; h <<= 1) {
    const int m = h >> 1;  // partner lane offset
    const float p0 = __shfl_xor(e0, m);
    const float p1 = __shfl_xor(e1, m);
    const bool lower = ((2 * lane) & h) == 0;
    e0 = lower ? (e0 + p0) : (p0 - e0);
    e1 = lower ? (e1 + p1) : (p1 - e1);
  }
  const float s = 0x1.6a09e6p-4f;  // fl32(1/sqrt(128))
  const uint32_t o = static_cast<uint32_t>(f32_to_bf16(e0 * s)) |
                     (static_cast<uint32_t>(f32_to_bf16(e1 * s)) << 16);
  *reinterpret_cast<uint32_t*>(y + r * y_stride + 2 * lane) = o;
}

// ---------------------------------------------------------------------------
// indexer prep (Ernie5_5Indexer.forward up to the quantization): k_norm
// LayerNorm of k, NeoX RoPE on dims 0..63 of q and k, Hadamard.  One 16-lane
// group per 128-wide row; lane j of the group holds elements 8j .. 8j+7 (fp32
// copies of bf16 values).  Cross-lane partners are lane ^ 1, 2, 4, 8, inside
// the group.
// ---------------------------------------------------------------------------
struct PrepArgs {
  const uint16_t* q;  // [T, heads, 128] bf16
  int64_t q_tok_stride, q_head_stride;
  const uint16_t* k;  // [T, 128] bf16
  int64_t k_stride;
  int32_t num_tokens, heads;
  const float* ln_w;  // [128]
  const float* ln_b;  // [128]
  float eps;
  const float* cos_sin;  // [cs_rows, 64]: cos 32 | sin 32
  int32_t cs_rows;
  const int64_t* positions;  // [T]
  uint16_t* q_out;           // [T, heads, 128]
  uint16_t* k_out;           // [T, 128]
};

// Rows of workgroup `block` (16 per workgroup): q rows (token, head) first,
// then k rows.  Positions outside the cos/sin table leave the row unrotated.
__device__ __forceinline__ void prep_rows(const PrepArgs& a, int block) {
  const int j = threadIdx.x & 15;
  const int64_t row = static_cast<int64_t>(block) * 16 + (threadIdx.x >> 4);
  const int64_t q_rows = static_cast<int64_t>(a.num_tokens) * a.heads;
  if (row >= q_rows + a.num_tokens) return;  // whole 16-lane group exits together
  const bool is_q = row < q_rows;
  const int64_t t = is_q ? row / a.heads : row - q_rows;
  const uint16_t* src = is_q ? a.q + t * a.q_tok_stride + (row % a.heads) * a.q_head_stride : a.k + t * a.k_stride;
  float v[8];
  unpack_bf16x8(*reinterpret_cast<const uint4*>(src + 8 * j), v);
  const int64_t pos = a.positions[t];
  const float* cs = (pos >= 0 && pos < a.cs_rows) ? a.cos_sin + pos * 64 : nullptr;
  if (!is_q) row_layer_norm(v, a.ln_w, a.ln_b, a.eps, j);
  row_rope_neox64(v, cs, j);
  row_hadamard(v, j);
  uint16_t* dst = is_q ? a.q_out + row * 128 : a.k_out + t * 128;
  *reinterpret_cast<uint4*>(dst + 8 * j) = pack_bf16x8(v);
}

__global__ void __launch_bounds__(256) indexer_prep_kernel(PrepArgs a) { prep_rows(a, blockIdx.x); }

// ---------------------------------------------------------------------------
// indexer_q_quant: one 16-lane group per (token, head) row of 128.
// ---------------------------------------------------------------------------
struct QQuantArgs {
  const uint16_t* q;         // [T, heads, 128] bf16
  int64_t q_tok_stride, q_head_stride;
  const void* w;             // [T, w_stride] bf16 or fp32
  int32_t w_is_bf16;
  int64_t w_stride;
  int32_t num_tokens, heads;
  uint8_t* q_fp8;            // [T, heads, 128]
  float* w_out;              // [T, heads]
  int8_t* q_digits;          // [T, 3, heads, 128] or null
  // indexer q prep before the quantization (optional): q is the raw
  // projection, made hadamard(rope(q)) with cos_sin row positions[t]
  const float* cos_sin;      // [cs_rows, 64]; nullptr = no prep
  int32_t cs_rows;
  const int64_t* positions;
};

// Rows (token, head) 16 * block .. +15, 16 lanes per row.
__device__ __forceinline__ void q_quant_rows(const QQuantArgs& qa, int block) {
  const uint16_t* q = qa.q;
  const int64_t q_tok_stride = qa.q_tok_stride, q_head_stride = qa.q_head_stride;
  const void* w = qa.w;
  const int32_t w_is_bf16 = qa.w_is_bf16;
  const int64_t w_stride = qa.w_stride;
  const int32_t num_tokens = qa.num_tokens, heads = qa.heads;
  uint8_t* q_fp8 = qa.q_fp8;
  float* w_out = qa.w_out;
  int8_t* q_digits = qa.q_digits;
  const int lane = threadIdx.x & 63;
  const int ln = lane & 15;
  const int64_t row = static_cast<int64_t>(block) * 16 + (threadIdx.x >> 4);
  if (row >= static_cast<int64_t>(num_tokens) * heads) return;
  const int64_t t = row / heads;
  const int h = static_cast<int>(row % heads);
  const uint16_t* src = q + t * q_tok_stride + h * q_head_stride;
  uint4 wv = *reinterpret_cast<const uint4*>(src + 8 * ln);
  uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(ww[i] << 16);
    v[2 * i + 1] = __uint_as_float(ww[i] & 0xffff0000u);
  }
  if (qa.cos_sin != nullptr) {  // uniform over the launch
    const int64_t pos = qa.positions[t];
    row_rope_neox64(v, (pos >= 0 && pos < qa.cs_rows) ? qa.cos_sin + pos * 64 : nullptr, ln);
    row_hadamard(v, ln);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = wave_max_xor(amax, 16);
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  uint32_t b0 = f32x2_to_fp8(v[0] * inv, v[1] * inv);
  uint32_t b1 = f32x2_to_fp8(v[2] * inv, v[3] * inv);
  uint32_t b2 = f32x2_to_fp8(v[4] * inv, v[5] * inv);
  uint32_t b3 = f32x2_to_fp8(v[6] * inv, v[7] * inv);
  uint32_t lo = b0 | (b1 << 16), hi = b2 | (b3 << 16);
  *reinterpret_cast<uint2*>(q_fp8 + row * 128 + 8 * ln) = make_uint2(lo, hi);
  if (q_digits != nullptr) {
    // planes [t][digit][h][128]
    uint32_t d[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t code = ((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xffu;
      const uint32_t pk = fp8_digit_pack(code);
#pragma unroll
      for (int p = 0; p < 3; ++p) d[p][i >> 2] |= ((pk >> (8 * p)) & 0xffu) << (8 * (i & 3));
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      int8_t* dst = q_digits + ((t * 3 + p) * heads + h) * 128 + 8 * ln;
      *reinterpret_cast<uint2*>(dst) = make_uint2(d[p][0], d[p][1]);
    }
  }
  if (ln == 0) {
    float wt = w_is_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(w)[t * w_stride + h])
                         : static_cast<const float*>(w)[t * w_stride + h];
    const float ws = 0x1.6a09e6p-7f;  // fl32(128**-0.5 * 64**-0.5)
    w_out[t * heads + h] = (wt * exp2i(e)) * ws;
  }
}

__global__ void __launch_bounds__(256) indexer_q_quant_kernel(QQuantArgs a) { q_quant_rows(a, blockIdx.x); }

__global__ void fp8_digit_table_kernel(uint32_t* table) {
  const int i = threadIdx.x;
  if (i < 256) table[i] = fp8_digit_pack(static_cast<uint32_t>(i));
}

// ---------------------------------------------------------------------------
// windowed_lengths and hca_decode_indices
// ---------------------------------------------------------------------------
__global__ void windowed_lengths_kernel(const int64_t* positions, int32_t n, int32_t window,
                                        int32_t* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = static_cast<int32_t>(max(positions[i] + 1 - window, static_cast<int64_t>(0)));
}

__global__ void __launch_bounds__(256) hca_decode_indices_kernel(HcaIndexArgs a) {
  hca_index_block(a, blockIdx.x, blockIdx.y);
}

// ---------------------------------------------------------------------------
// DSA decode prologue: the new token's indexer K row and latent row appended
// (fp8 + UE8M0), the indexer q quantized and the windowed lengths, in one
// launch.  Workgroups [0, k_blocks) append K rows, then latent rows, then q
// rows; the last ones write the lengths.
// ---------------------------------------------------------------------------
struct DsaPrologueArgs {
  AppendArgs k_rows;         // indexer K (D = 128)
  AppendArgs latent;         // latent rows (D = the kernel's D)
  QQuantArgs q;
  const int64_t* positions;  // [T]
  int32_t window;
  int32_t* lengths;          // [T]
  int32_t k_blocks, latent_blocks, q_blocks;
};

template <int D>
__global__ void __launch_bounds__(256) dsa_prologue_kernel(DsaPrologueArgs a) {
  int b = blockIdx.x;
  if (b < a.k_blocks) {
    append_rows<128, 1>(a.k_rows, b);
    return;
  }
  b -= a.k_blocks;
  if (b < a.latent_blocks) {
    append_rows<D, 1>(a.latent, b);
    return;
  }
  b -= a.latent_blocks;
  if (b < a.q_blocks) {
    q_quant_rows(a.q, b);
    return;
  }
  b -= a.q_blocks;
  const int i = b * 256 + threadIdx.x;
  if (i < a.q.num_tokens)
    a.lengths[i] = static_cast<int32_t>(max(a.positions[i] + 1 - a.window, static_cast<int64_t>(0)));
}

int launch_hca_append(const AppendArgs& a, int dim, int num_seqs, bool rows, bool tail, hipStream_t s) {
  int main_blocks = 0, tail_rows = 0;
  const int64_t blocks = hca_append_grid(a, dim, num_seqs, rows, tail, main_blocks, tail_rows);
  EKV_CHECK(blocks < (int64_t{1} << 31), "too many rows");
  if (blocks == 0) return 0;
  dim3 grid(static_cast<uint32_t>(blocks));
  if (dim == 512) hipLaunchKernelGGL(hca_append_kernel<512>, grid, dim3(256), 0, s, a, main_blocks, tail_rows);
  else hipLaunchKernelGGL(hca_append_kernel<576>, grid, dim3(256), 0, s, a, main_blocks, tail_rows);
  return ekv_launch_status();
}

}  // namespace ekv

// ===========================================================================
// C ABI
// ===========================================================================
using namespace ekv;

namespace {

// Argument checks shared by the entry points that append rows / quantize q.
int check_append(const uint16_t* rows, int64_t row_stride, int32_t dim, const int64_t* slot_mapping,
                 const uint8_t* cache, int64_t page_stride) {
  EKV_CHECK(rows && slot_mapping && cache, "null pointer");
  EKV_CHECK(dim == 128 || dim == 512 || dim == 576, "dim must be 128, 512 or 576");
  EKV_CHECK(row_stride >= dim && row_stride % 8 == 0, "row_stride must be >= dim and a multiple of 8");
  EKV_CHECK(page_stride >= kPageTokens * (dim + 4) && page_stride % 16 == 0,
            "page_stride must hold 64 rows + 64 scales and be a multiple of 16");
  EKV_CHECK(aligned16(rows) && aligned16(cache), "rows and cache must be 16-byte aligned");
  return 0;
}

int check_q_quant(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride, const void* weights,
                  int32_t heads, const uint8_t* q_fp8, const float* w_out, const int8_t* q_digits) {
  EKV_CHECK(q && weights && q_fp8 && w_out, "null pointer");
  EKV_CHECK(heads > 0 && q_head_stride % 8 == 0 && q_tok_stride % 8 == 0, "strides must be multiples of 8");
  EKV_CHECK(aligned16(q) && aligned8(q_fp8) && (q_digits == nullptr || aligned8(q_digits)), "misaligned buffers");
  return 0;
}

AppendArgs append_args(const uint16_t* rows, int64_t row_stride, int32_t num_tokens, const int64_t* slot_mapping,
                       uint8_t* cache, int64_t page_stride, int64_t num_pages) {
  AppendArgs a{};
  a.rows = rows; a.row_stride = row_stride; a.num_tokens = num_tokens; a.slot_mapping = slot_mapping;
  a.cache = cache; a.page_stride = page_stride; a.num_pages = num_pages;
  return a;
}

}  // namespace

extern "C" int ekv_kv_append_quant(const uint16_t* rows, int64_t row_stride, int32_t num_tokens,
                                   int32_t dim, const int64_t* slot_mapping, uint8_t* cache,
                                   int64_t page_stride, int64_t num_pages, void* stream) {
  EKV_CHECK(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  int rc = check_append(rows, row_stride, dim, slot_mapping, cache, page_stride);
  if (rc) return rc;
  const AppendArgs a = append_args(rows, row_stride, num_tokens, slot_mapping, cache, page_stride, num_pages);
  const int rows_per_block = append_block_rows(dim, dim == 128 ? kAppendSeq<128> : kAppendSeq<576>);
  dim3 grid((num_tokens + rows_per_block - 1) / rows_per_block);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dim == 128) hipLaunchKernelGGL(kv_append_quant_kernel<128>, grid, dim3(256), 0, s, a);
  else if (dim == 512) hipLaunchKernelGGL(kv_append_quant_kernel<512>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(kv_append_quant_kernel<576>, grid, dim3(256), 0, s, a);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_k_insert(const uint16_t* k, int64_t k_stride, int32_t num_tokens,
                                    const int64_t* slot_mapping, uint8_t* kcache, int64_t page_stride,
                                    int64_t num_pages, void* stream) {
  return ekv_kv_append_quant(k, k_stride, num_tokens, 128, slot_mapping, kcache, page_stride,
                             num_pages, stream);
}

extern "C" int ekv_hca_append(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                              int64_t kvs_stride, int32_t num_tokens, int32_t dim,
                              const int64_t* slot_mapping, const int64_t* positions,
                              const int32_t* token_seq, const int32_t* qsl, int32_t num_seqs,
                              uint8_t* pool, int64_t page_stride, int64_t num_pages,
                              const int32_t* ring_pages, int32_t ring_stride, int32_t ring,
                              uint16_t* state, const int32_t* state_slot, int32_t num_state,
                              void* stream) {
  EKV_CHECK(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  AppendArgs a;
  const int rc = hca_append_args(a, latent, latent_stride, kv_score, kvs_stride, num_tokens, dim, slot_mapping,
                                 positions, token_seq, qsl, num_seqs, pool, page_stride, num_pages, ring_pages,
                                 ring_stride, ring, state, state_slot, num_state);
  if (rc) return rc;
  return launch_hca_append(a, dim, num_seqs, true, true, static_cast<hipStream_t>(stream));
}

extern "C" int ekv_hca_append_bf16(const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                                   int64_t kvs_stride, int32_t num_tokens, int32_t dim,
                                   const int64_t* slot_mapping, const int64_t* positions,
                                   const int32_t* token_seq, const int32_t* qsl, int32_t num_seqs,
                                   uint16_t* pool, int64_t page_stride, int64_t num_pages,
                                   const int32_t* ring_pages, int32_t ring_stride, int32_t ring,
                                   uint16_t* state, const int32_t* state_slot, int32_t num_state,
                                   void* stream) {
  EKV_CHECK(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  AppendArgs a;
  const int rc = hca_append_args(a, latent, latent_stride, kv_score, kvs_stride, num_tokens, dim, slot_mapping,
                                 positions, token_seq, qsl, num_seqs, reinterpret_cast<uint8_t*>(pool), page_stride,
                                 num_pages, ring_pages, ring_stride, ring, state, state_slot, num_state, true);
  if (rc) return rc;
  return launch_hca_append(a, dim, num_seqs, true, true, static_cast<hipStream_t>(stream));
}

extern "C" int ekv_merge_swa_topk(const int32_t* topk, int64_t topk_stride, int32_t* out,
                                  int64_t out_stride, const int64_t* positions, int32_t num_tokens,
                                  int32_t topk_width, int32_t out_width, int32_t window, void* stream) {
  EKV_CHECK(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  EKV_CHECK(topk && out && positions, "null pointer");
  EKV_CHECK(out_width >= topk_width + window, "width must be >= topk + window");
  hipLaunchKernelGGL(merge_swa_topk_kernel, dim3(num_tokens), dim3(256), 0, static_cast<hipStream_t>(stream),
                     topk, topk_stride, out, out_stride, positions, topk_width, out_width, window);
  return ekv_launch_status();
}

extern "C" int ekv_hadamard_rows(const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride,
                                 int32_t rows, int32_t dim, void* stream) {
  EKV_CHECK(rows >= 0, "rows must be >= 0");
  if (rows == 0) return 0;
  EKV_CHECK(dim == 128, "hadamard_rows supports 128-wide rows");
  EKV_CHECK(x && y && x_stride >= 128 && y_stride >= 128 && x_stride % 2 == 0 && y_stride % 2 == 0,
            "bad pointers or strides");
  EKV_CHECK(aligned4(x) && aligned4(y), "rows must be 4-byte aligned");
  hipLaunchKernelGGL(hadamard_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, x_stride, y, y_stride, rows);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_prep(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride, const uint16_t* k,
                                int64_t k_stride, int32_t num_tokens, int32_t heads, const float* ln_w,
                                const float* ln_b, float eps, const float* cos_sin, int32_t cos_sin_rows,
                                const int64_t* positions, uint16_t* q_out, uint16_t* k_out, void* stream) {
  EKV_CHECK(num_tokens >= 0 && heads >= 0, "sizes must be >= 0");
  if (num_tokens == 0) return 0;
  EKV_CHECK(q && k && ln_w && ln_b && cos_sin && positions && q_out && k_out, "null pointer");
  EKV_CHECK(q_head_stride >= 128 && q_tok_stride >= heads * q_head_stride && k_stride >= 128 &&
                q_head_stride % 8 == 0 && q_tok_stride % 8 == 0 && k_stride % 8 == 0,
            "q [T, heads, 128] and k [T, 128] rows must be 16-byte aligned, 128 wide");
  EKV_CHECK(aligned16(q) && aligned16(k) && aligned16(q_out) && aligned16(k_out) && aligned16(ln_w) &&
                aligned16(ln_b) && aligned16(cos_sin),
            "buffers must be 16-byte aligned");
  EKV_CHECK(cos_sin_rows >= 0, "cos_sin_rows must be >= 0");
  PrepArgs a{q, q_tok_stride, q_head_stride, k, k_stride, num_tokens, heads, ln_w, ln_b, eps, cos_sin, cos_sin_rows,
             positions, q_out, k_out};
  const int64_t rows = static_cast<int64_t>(num_tokens) * (heads + 1);
  EKV_CHECK((rows + 15) / 16 < (int64_t{1} << 31), "too many rows");
  hipLaunchKernelGGL(indexer_prep_kernel, dim3(static_cast<uint32_t>((rows + 15) / 16)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_q_quant(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                   const void* weights, int32_t weights_is_bf16, int64_t w_stride,
                                   int32_t num_tokens, int32_t heads, uint8_t* q_fp8, float* w_out,
                                   int8_t* q_digits, void* stream) {
  EKV_CHECK(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  int rc = check_q_quant(q, q_tok_stride, q_head_stride, weights, heads, q_fp8, w_out, q_digits);
  if (rc) return rc;
  const int64_t rows = static_cast<int64_t>(num_tokens) * heads;
  const QQuantArgs a{q, q_tok_stride, q_head_stride, weights, weights_is_bf16, w_stride, num_tokens, heads,
                     q_fp8, w_out, q_digits};
  hipLaunchKernelGGL(indexer_q_quant_kernel, dim3(static_cast<unsigned>((rows + 15) / 16)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}

extern "C" int ekv_dsa_decode_prologue(const uint16_t* k, int64_t k_stride, uint8_t* kcache, int64_t k_page_stride,
                                       int64_t k_num_pages, const uint16_t* latent, int64_t latent_stride,
                                       int32_t dim, uint8_t* cache, int64_t page_stride, int64_t num_pages,
                                       const int64_t* slot_mapping, int32_t num_tokens, const uint16_t* q,
                                       int64_t q_tok_stride, int64_t q_head_stride, const void* weights,
                                       int32_t weights_is_bf16, int64_t w_stride, int32_t heads, uint8_t* q_fp8,
                                       float* w_out, int8_t* q_digits, const int64_t* positions, int32_t window,
                                       int32_t* lengths, const float* ln_w, const float* ln_b, float eps,
                                       const float* cos_sin, int32_t cos_sin_rows, void* stream) {
  EKV_CHECK(num_tokens >= 0 && window >= 0, "bad sizes");
  EKV_CHECK(cos_sin == nullptr || (ln_w && ln_b && cos_sin_rows >= 0 && aligned16(ln_w) && aligned16(ln_b) &&
                                   aligned16(cos_sin)),
            "the indexer prep needs 16-byte aligned ln_w, ln_b and cos_sin");
  if (num_tokens == 0) return 0;
  EKV_CHECK(dim == 512 || dim == 576, "latent dim must be 512 or 576");
  int rc = check_append(k, k_stride, 128, slot_mapping, kcache, k_page_stride);
  if (rc) return rc;
  rc = check_append(latent, latent_stride, dim, slot_mapping, cache, page_stride);
  if (rc) return rc;
  rc = check_q_quant(q, q_tok_stride, q_head_stride, weights, heads, q_fp8, w_out, q_digits);
  if (rc) return rc;
  EKV_CHECK(positions && lengths, "null pointer");
  DsaPrologueArgs a{};
  a.k_rows = append_args(k, k_stride, num_tokens, slot_mapping, kcache, k_page_stride, k_num_pages);
  a.latent = append_args(latent, latent_stride, num_tokens, slot_mapping, cache, page_stride, num_pages);
  a.q = QQuantArgs{q, q_tok_stride, q_head_stride, weights, weights_is_bf16, w_stride, num_tokens, heads,
                   q_fp8, w_out, q_digits, cos_sin, cos_sin_rows, positions};
  if (cos_sin != nullptr) {
    a.k_rows.positions = positions;
    a.k_rows.ln_w = ln_w;
    a.k_rows.ln_b = ln_b;
    a.k_rows.eps = eps;
    a.k_rows.cos_sin = cos_sin;
    a.k_rows.cs_rows = cos_sin_rows;
  }
  a.positions = positions;
  a.window = window;
  a.lengths = lengths;
  a.k_blocks = (num_tokens + append_block_rows(128, 1) - 1) / append_block_rows(128, 1);
  a.latent_blocks = (num_tokens + append_block_rows(dim, 1) - 1) / append_block_rows(dim, 1);
  a.q_blocks = static_cast<int32_t>((static_cast<int64_t>(num_tokens) * heads + 15) / 16);
  const int len_blocks = (num_tokens + 255) / 256;
  const dim3 grid(a.k_blocks + a.latent_blocks + a.q_blocks + len_blocks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dim == 576) hipLaunchKernelGGL(dsa_prologue_kernel<576>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(dsa_prologue_kernel<512>, grid, dim3(256), 0, s, a);
  return ekv_launch_status();
}

extern "C" int ekv_indexer_windowed_lengths(const int64_t* positions, int32_t num_tokens, int32_t window,
                                            int32_t* out, void* stream) {
  EKV_CHECK(num_tokens >= 0 && window >= 0, "bad sizes");
  if (num_tokens == 0) return 0;
  EKV_CHECK(positions && out, "null pointer");
  hipLaunchKernelGGL(windowed_lengths_kernel, dim3((num_tokens + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), positions, num_tokens, window, out);
  return ekv_launch_status();
}

extern "C" int ekv_hca_decode_indices(const int64_t* positions, const int32_t* req_ids, int32_t num_tokens,
                                      const int32_t* comp_block_table, int32_t comp_bt_stride,
                                      const int32_t* ring_pages, int32_t ring_stride, int32_t ring,
                                      int32_t window, const int32_t* query_start_loc,
                                      const int64_t* slot_mapping, int32_t* out, int64_t out_stride,
                                      int32_t width, int32_t* lengths, void* stream) {
  EKV_CHECK(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return 0;
  EKV_CHECK(positions && req_ids && comp_block_table && ring_pages && out && lengths, "null pointer");
  EKV_CHECK(ring >= window && ring % kPageTokens == 0, "ring must be a multiple of 64 and >= window");
  EKV_CHECK((query_start_loc == nullptr) == (slot_mapping == nullptr),
            "query_start_loc and slot_mapping go together");
  EKV_CHECK(width >= 0 && out_stride >= width, "out_stride must be >= width >= 0");
  const HcaIndexArgs a{positions, req_ids, comp_block_table, comp_bt_stride, ring_pages, ring_stride, ring,
                       window, query_start_loc, slot_mapping, out, out_stride, width, lengths};
  const dim3 grid(static_cast<unsigned>(num_tokens), static_cast<unsigned>(hca_index_blocks_per_row(width)));
  hipLaunchKernelGGL(hca_decode_indices_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}

extern "C" int ekv_fp8_digit_table(uint32_t* table, void* stream) {
  EKV_CHECK(table != nullptr, "null pointer");
  hipLaunchKernelGGL(fp8_digit_table_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), table);
  return ekv_launch_status();
}
