// Post-attention fused quantization (the step after the sparse decode).
//
//  * sigmoid_mul_quant_kernel: x * sigmoid(gate) in bf16 (the roundings of
//    torch's `x * torch.sigmoid(gate)`: s = bf16(sigmoid(gate)), y =
//    bf16(x * s)), quantized to fp8 e4m3 in 1 x 128 groups with UE8M0
//    scales, four group exponents (+127) packed per int32, the scale buffer
//    column-major [packs][rows_aligned].  One wave per (row, 512 columns):
//    lane l takes columns 8l .. 8l+7, a group is 16 lanes.  sigmoid is
//    evaluated in fp64 and rounded once to fp32 (the correctly rounded fp32
//    sigmoid in all but vanishing cases), then to bf16.
//  * vha_inv_rope_quant_kernel: per token, the VHA head mix Y = M O (64 x 64
//    bf16 mix over 64 heads of 512 bf16 channels, fp32 accumulation), the
//    inverse RoPE of the interleaved rope pairs (channels nope_dim ..), and a
//    UE8M0 fp8 quant per (head, 128 channels), written as
//    [group][token][head in group * 512 + channel] with exponent byte c of
//    scale int32 [group][head in group][token] for chunk c.  Four waves, wave
//    w = channels [128 w, 128 w + 128): Y^T = O^T M^T on
//    v_mfma_f32_16x16x32_bf16 with A = O^T read from the token's rows in LDS
//    by transposing reads (ds_read_b64_tr_b16) and B = M^T rows from
//    registers; a lane's accumulator holds 4 consecutive channels of one
//    head, so a rope pair never leaves its lane.
#include "ekv_common.h"
#include "ekv_internal.h"

#include <type_traits>

namespace ekv {

typedef short q_i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) q_i16x4 q_lds_i16x4;

__device__ __forceinline__ float row16_max_f(float v) {
  // max over each row of 16 lanes (DPP rotations), every lane receiving it
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x128>{}));
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x124>{}));
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x122>{}));
  return fmaxf(v, dpp(v, std::integral_constant<int, 0x121>{}));
}

// ---------------------------------------------------------------------------
// sigmoid-mul quant
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) sigmoid_mul_quant_kernel(const uint16_t* x, int64_t x_stride,
                                                                const uint16_t* gate, int64_t gate_stride,
                                                                int32_t rows, int32_t packs, uint8_t* out,
                                                                int64_t out_stride, int32_t* scale,
                                                                int64_t scale_stride) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // (row, pack)
  if (unit >= static_cast<int64_t>(rows) * packs) return;
  const int64_t row = unit / packs;
  const int pack = static_cast<int>(unit % packs);
  const int64_t c0 = static_cast<int64_t>(pack) * 512 + 8 * lane;
  const uint4 xv = *reinterpret_cast<const uint4*>(x + row * x_stride + c0);
  const uint4 gv = *reinterpret_cast<const uint4*>(gate + row * gate_stride + c0);
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
  float y[8];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float xf = bf16_to_f32(static_cast<uint16_t>(xw[j >> 1] >> (16 * (j & 1))));
    const float gf = bf16_to_f32(static_cast<uint16_t>(gw[j >> 1] >> (16 * (j & 1))));
    const float sg = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(gf))));  // one rounding to fp32
    const float s = bf16_to_f32(f32_to_bf16(sg));
    y[j] = bf16_to_f32(f32_to_bf16(xf * s));  // the product of two bf16 values is exact in fp32
    amax = fmaxf(amax, fabsf(y[j]));
  }
  amax = row16_max_f(amax);
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  const uint32_t lo = f32x2_to_fp8(y[0] * inv, y[1] * inv) | (f32x2_to_fp8(y[2] * inv, y[3] * inv) << 16);
  const uint32_t hi = f32x2_to_fp8(y[4] * inv, y[5] * inv) | (f32x2_to_fp8(y[6] * inv, y[7] * inv) << 16);
  *reinterpret_cast<uint2*>(out + row * out_stride + c0) = make_uint2(lo, hi);
  // packed exponents of the pack's 4 groups: group g's byte from lane 16 g
  const uint32_t byte = static_cast<uint32_t>(e + 127) & 0xffu;
  const uint32_t b0 = __shfl(byte, 0), b1 = __shfl(byte, 16), b2 = __shfl(byte, 32), b3 = __shfl(byte, 48);
  if (lane == 0)
    scale[static_cast<int64_t>(pack) * scale_stride + row] = static_cast<int32_t>(b0 | (b1 << 8) | (b2 << 16) | (b3 << 24));
}

// ---------------------------------------------------------------------------
// VHA mix + inverse RoPE + quant
// ---------------------------------------------------------------------------
constexpr int kVhaHeads = 64;
constexpr int kVhaDim = 512;
constexpr int kVhaRowB = 2 * kVhaDim + 16;  // bf16 row stride in LDS (padded)

struct VhaArgs {
  const uint16_t* o;        // [T, >= 64, 512] bf16
  int64_t o_tok_stride, o_head_stride;
  const uint16_t* mix;      // [64, 64] bf16
  const int64_t* positions; // [T]
  const float* cos_sin;     // [P, cs_stride]: cos (rope_dim / 2) | sin
  int64_t cs_stride;
  int32_t num_tokens, aligned_tokens;
  int32_t heads_per_group, nope_dim, half_rope;
  uint8_t* out;             // [G, T, heads_per_group * 512] fp8
  uint8_t* scale;           // [G, heads_per_group, aligned_tokens] int32, as bytes
};

constexpr int kVhaLds = kVhaHeads * kVhaRowB;

__global__ void __launch_bounds__(256) vha_inv_rope_quant_kernel(VhaArgs a) {
  extern __shared__ __align__(16) uint8_t s_o[];  // kVhaLds bytes: the token's 64 rows
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // channel chunk
  const int kg = lane >> 4, col = lane & 15;
  // B = M^T (input heads x output heads): lane (head 16 hb + col, kg) holds
  // M[head][32 ks + 8 kg .. +7]
  bf16x8 mb[4][2];
#pragma unroll
  for (int hb = 0; hb < 4; ++hb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      mb[hb][ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(a.mix + (16 * hb + col) * kVhaHeads +
                                                                               32 * ks + 8 * kg));
  for (int tok = blockIdx.x; tok < a.aligned_tokens; tok += gridDim.x) {
    if (tok >= a.num_tokens) {  // padding rows of the scale buffer: zero bytes
      const int h = tid >> 2, c = tid & 3;
      const int grp = h / a.heads_per_group, hig = h % a.heads_per_group;
      a.scale[((static_cast<int64_t>(grp) * a.heads_per_group + hig) * a.aligned_tokens + tok) * 4 + c] = 0;
      continue;
    }
    __syncthreads();  // the previous token's reads of s_o are done
    // the token's 64 x 512 bf16 rows into LDS (16-byte loads)
#pragma unroll
    for (int j = 0; j < (kVhaHeads * kVhaDim * 2 / 16) / 256; ++j) {
      const int idx = tid + 256 * j;
      const int h = idx >> 6, part = idx & 63;
      const uint4 v = *reinterpret_cast<const uint4*>(a.o + static_cast<int64_t>(tok) * a.o_tok_stride +
                                                      h * a.o_head_stride + 8 * part);
      *reinterpret_cast<uint4*>(s_o + h * kVhaRowB + 16 * part) = v;
    }
    __syncthreads();
    // Y^T[channel][head] for this wave's 8 channel blocks x 4 head blocks
    f32x4 acc[4][8];
#pragma unroll
    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) acc[hb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const int ch = 128 * wave + 16 * cb + 4 * (col & 3);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // A = O^T: element m of read h2 is O[32 ks + 8 kg + 4 h2 + m][16 cb + (this lane's column)]
        const int r0 = 32 * ks + 8 * kg + (col >> 2);
        const q_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (q_lds_i16x4*)((__attribute__((address_space(3))) uint8_t*)(s_o + r0 * kVhaRowB + 2 * ch)));
        const q_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (q_lds_i16x4*)((__attribute__((address_space(3))) uint8_t*)(s_o + (r0 + 4) * kVhaRowB + 2 * ch)));
        const q_i16x4 both[2] = {lo, hi};
        const bf16x8 av = __builtin_bit_cast(bf16x8, both);
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) acc[hb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, mb[hb][ks], acc[hb][cb], 0, 0, 0);
      }
    }
    // lane: head h = 16 hb + col, channels 128 wave + 16 cb + 4 kg + i
    const int64_t pos = a.positions[tok];
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const int c0 = 128 * wave + 16 * cb + 4 * kg;
      if (c0 + 3 >= a.nope_dim) {  // inverse rotation of the pairs (c0, c0+1), (c0+2, c0+3)
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const int c = c0 + 2 * pr;
          if (c < a.nope_dim) continue;
          const int r = (c - a.nope_dim) >> 1;
          const float cs = a.cos_sin[pos * a.cs_stride + r], sn = a.cos_sin[pos * a.cs_stride + a.half_rope + r];
#pragma unroll
          for (int hb = 0; hb < 4; ++hb) {
            const float ev = acc[hb][cb][2 * pr], od = acc[hb][cb][2 * pr + 1];
            acc[hb][cb][2 * pr] = ev * cs + od * sn;
            acc[hb][cb][2 * pr + 1] = od * cs - ev * sn;
          }
        }
      }
    }
#pragma unroll
    for (int hb = 0; hb < 4; ++hb) {
      float amax = 0.0f;
#pragma unroll
      for (int cb = 0; cb < 8; ++cb)
#pragma unroll
        for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(acc[hb][cb][i]));
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      const int e = ue8m0_exponent(amax);
      const float inv = exp2i(-e);
      const int h = 16 * hb + col;
      const int grp = h / a.heads_per_group, hig = h % a.heads_per_group;
      uint8_t* orow = a.out + (static_cast<int64_t>(grp) * a.num_tokens + tok) * (a.heads_per_group * kVhaDim) +
                      hig * kVhaDim;
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        const uint32_t w01 = f32x2_to_fp8(acc[hb][cb][0] * inv, acc[hb][cb][1] * inv);
        const uint32_t w23 = f32x2_to_fp8(acc[hb][cb][2] * inv, acc[hb][cb][3] * inv);
        *reinterpret_cast<uint32_t*>(orow + 128 * wave + 16 * cb + 4 * kg) = w01 | (w23 << 16);
      }
      if (kg == 0)
        a.scale[((static_cast<int64_t>(grp) * a.heads_per_group + hig) * a.aligned_tokens + tok) * 4 + wave] =
            static_cast<uint8_t>(e + 127);
    }
  }
}

}  // namespace ekv

using namespace ekv;

extern "C" int ekv_sigmoid_mul_quant_fp8(const uint16_t* x, int64_t x_stride, const uint16_t* gate,
                                         int64_t gate_stride, int32_t num_rows, int32_t hidden, uint8_t* out,
                                         int64_t out_stride, int32_t* scale, int64_t scale_stride, void* stream) {
  EKV_CHECK(num_rows >= 0 && hidden > 0 && hidden % 512 == 0, "hidden must be a positive multiple of 512");
  if (num_rows == 0) return 0;
  EKV_CHECK(x && gate && out && scale, "null pointer");
  EKV_CHECK(aligned16(x) && aligned16(gate) && x_stride % 8 == 0 && gate_stride % 8 == 0,
            "x and gate rows must be 16-byte aligned");
  EKV_CHECK(aligned8(out) && out_stride % 8 == 0 && out_stride >= hidden, "out rows must be 8-byte aligned");
  EKV_CHECK(aligned4(scale) && scale_stride >= num_rows, "scale_stride must be >= num_rows");
  const int packs = hidden / 512;
  const int64_t units = static_cast<int64_t>(num_rows) * packs;
  hipLaunchKernelGGL(sigmoid_mul_quant_kernel, dim3(static_cast<uint32_t>((units + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, x_stride, gate, gate_stride, num_rows, packs, out,
                     out_stride, scale, scale_stride);
  return ekv_launch_status();
}

extern "C" int ekv_vha_inv_rope_fp8_quant(const uint16_t* o, int64_t o_tok_stride, int64_t o_head_stride,
                                          int32_t num_tokens, int32_t heads, const uint16_t* mix,
                                          const int64_t* positions, const float* cos_sin, int64_t cs_stride,
                                          int32_t n_groups, int32_t nope_dim, int32_t rope_dim, uint8_t* out,
                                          int32_t* scale, int32_t aligned_tokens, void* stream) {
  EKV_CHECK(num_tokens >= 0 && aligned_tokens >= num_tokens, "aligned_tokens must be >= num_tokens");
  if (aligned_tokens == 0) return 0;
  EKV_CHECK(heads == kVhaHeads, "the fused VHA quant takes 64 heads");
  EKV_CHECK(n_groups > 0 && heads % n_groups == 0, "n_groups must divide heads");
  EKV_CHECK(nope_dim + rope_dim == kVhaDim && nope_dim % 4 == 0 && rope_dim > 0, "head_dim = nope + rope = 512");
  EKV_CHECK(o && mix && positions && cos_sin && out && scale, "null pointer");
  EKV_CHECK(aligned16(o) && o_tok_stride % 8 == 0 && o_head_stride % 8 == 0 && aligned16(mix),
            "o and mix must be 16-byte aligned rows");
  EKV_CHECK(aligned4(out) && aligned4(scale), "misaligned outputs");
  EKV_CHECK(cs_stride >= rope_dim, "cos_sin rows must hold rope_dim entries");
  VhaArgs a{o, o_tok_stride, o_head_stride, mix, positions, cos_sin, cs_stride, num_tokens, aligned_tokens,
            heads / n_groups, nope_dim, rope_dim / 2, out, reinterpret_cast<uint8_t*>(scale)};
  const int grid = aligned_tokens < 1024 ? aligned_tokens : 1024;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(vha_inv_rope_quant_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kVhaLds);
  hipLaunchKernelGGL(vha_inv_rope_quant_kernel, dim3(grid), dim3(256), kVhaLds, static_cast<hipStream_t>(stream), a);
  return ekv_launch_status();
}
