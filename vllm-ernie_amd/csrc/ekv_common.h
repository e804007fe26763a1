// Shared device helpers for the ERNIE KV-cache kernels (gfx950 / CDNA4).
//
// fp8 is OCP e4m3fn.  The hardware conversions used here were checked on the
// device against the e4m3fn definition: v_cvt_pk_fp8_f32 rounds to nearest
// even for |x| <= 448 (4M values incl. every midpoint), v_cvt_pk_f32_fp8
// decodes all 256 codes exactly.  Every caller clamps to +-448 first.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ekv {

constexpr int kPageTokens = 64;     // DSA_BLOCK_SIZE
constexpr float kE4M3Max = 448.0f;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round to nearest even (inputs are finite).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Exponent e of the UE8M0 scale 2**e for a row amax:
//   r = fl32(max(amax, 1e-10) * fl32(1/448));  e = ceil(log2(r)) taken exactly
// from r's bits (r is always a normal float here).
__device__ __forceinline__ int ue8m0_exponent(float amax) {
  float r = fmaxf(amax, 0x1.b7cdfep-34f) * 0x1.24924ap-9f;  // fl32(1e-10), fl32(1/448)
  uint32_t u = __float_as_uint(r);
  int e = static_cast<int>((u >> 23) & 0xffu) - 127;
  return (u & 0x7fffffu) ? e + 1 : e;
}

// Cross-workgroup hand-offs (a workgroup publishes results with
// agent-scope stores or atomics, then arrives on a counter with a relaxed
// agent-scope atomic add; the last to arrive reads the others' results with
// agent-scope loads).  The ordering they need comes from the hardware: on
// gfx950 agent-scope stores, loads and atomics bypass the non-coherent
// caches (sc1), `s_waitcnt 0` retires every memory operation the wave has
// issued, and loads issued after an atomic's returned value is tested are
// issued after it.  An acquire / release pair would add a whole-L2
// write-back and invalidate per arrival.  The compiler must not move memory
// accesses across the wait, nor hoist the last arriver's loads above its
// test: handoff_wait() is the wait between two compiler-only fences, and
// compiler_fence() follows each arrival test.
__device__ __forceinline__ void compiler_fence() { __atomic_signal_fence(__ATOMIC_SEQ_CST); }

__device__ __forceinline__ void handoff_wait() {
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(0);
  compiler_fence();
}

__device__ __forceinline__ float exp2i(int e) {  // 2**e for e in [-126, 127]
  return __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
}

// Two fp32 -> two e4m3fn bytes (low 16 bits), after clamping to +-448.
__device__ __forceinline__ uint32_t f32x2_to_fp8(float a, float b) {
  a = fminf(fmaxf(a, -kE4M3Max), kE4M3Max);
  b = fminf(fmaxf(b, -kE4M3Max), kE4M3Max);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}

// Four e4m3fn bytes packed in a word -> four floats.
__device__ __forceinline__ f32x4 fp8x4_to_f32(uint32_t w) {
  f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  return f32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Four e4m3fn bytes -> four bf16 packed in two words (exact: every e4m3fn
// value is a bf16 value, so the high half of its fp32 image is the bf16).
__device__ __forceinline__ void fp8x4_to_bf16x4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  lo = __builtin_amdgcn_perm(__float_as_uint(a[1]), __float_as_uint(a[0]), 0x07060302u);
  hi = __builtin_amdgcn_perm(__float_as_uint(b[1]), __float_as_uint(b[0]), 0x07060302u);
}

// Order-preserving uint32 key of an fp32 score (larger score -> larger key).
__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// bf16 bits of the smallest bf16 >= f (finite f): a conservative upper bound.
__device__ __forceinline__ uint16_t bf16_round_up(float f) {
  const uint32_t u = __float_as_uint(f);
  uint32_t hi = u >> 16;
  if (!(u >> 31) && (u & 0xffffu)) hi += 1u;  // positive with dropped bits: next bf16 up
  return static_cast<uint16_t>(hi);           // negative: truncation moves toward +inf
}

// Signed base-64 digits of the integer I = value * 2**9 of an e4m3fn code
// (|I| < 2**18): byte p of the result is digit p as two's complement int8,
// so I = d0 + 64*d1 + 4096*d2 exactly.
__device__ __forceinline__ uint32_t fp8_digit_pack(uint32_t code) {
  const uint32_t ex = (code >> 3) & 15u, m = code & 7u;
  uint32_t mag = ex ? ((8u + m) << (ex - 1)) : m;
  if (ex == 15u && m == 7u) mag = 0;  // NaN code: never produced by the quantizer
  const uint32_t d0 = mag & 63u, d1 = (mag >> 6) & 63u, d2 = mag >> 12;
  if (code & 0x80u) {
    return (static_cast<uint32_t>(-static_cast<int>(d0)) & 0xffu) |
           ((static_cast<uint32_t>(-static_cast<int>(d1)) & 0xffu) << 8) |
           ((static_cast<uint32_t>(-static_cast<int>(d2)) & 0xffu) << 16);
  }
  return d0 | (d1 << 8) | (d2 << 16);
}

// ---------------------------------------------------------------------------
// MXFP4 (OCP MX e2m1 values, one E8M0 scale byte per 32 values).
// ---------------------------------------------------------------------------
constexpr int kMxBlock = 32;

// E8M0 byte of a 32-value group with max |x| = amax: the exponent field of
// fl32(amax / 6) rounded up to a power of two (0 when the quotient is 0).
__device__ __forceinline__ uint32_t mxfp4_scale_byte(float amax) {
  const uint32_t bits = __float_as_uint(__fdiv_rn(amax, 6.0f));
  return ((bits + 0x7fffffu) & 0x7f800000u) >> 23;
}

// e2m1 code of y (|y| <= 6 after scaling): nearest, a tie going to the larger
// magnitude (one is added below the two kept bits, then they are shifted
// out), saturating at 6, sign kept (a small negative y gives code 8, -0).
__device__ __forceinline__ uint32_t e2m1_code(float y) {
  const uint32_t u = __float_as_uint(y);
  const uint32_t sign = u >> 31, e = (u >> 23) & 0xffu, m = u & 0x7fffffu;
  uint32_t m2 = m;
  if (e < 127u) {
    const uint32_t adj = 126u - e;  // aligns a value below 1 to the e2m1 subnormal
    m2 = adj < 32u ? (0x400000u | (m >> 1)) >> adj : 0u;
  }
  const uint32_t e2 = (e > 126u ? e : 126u) - 126u;
  const uint32_t c = min((((e2 << 2) | (m2 >> 21)) + 1u) >> 1, 7u);
  return (sign << 3) | c;
}

// 2**(byte - 127), the value of an E8M0 byte (byte 0 is 2**-127).
__device__ __forceinline__ float e8m0_value(uint32_t byte) {
  return byte ? __uint_as_float(byte << 23) : 0x1p-127f;
}

// Four e2m1 codes (one per byte, low nibble) -> the int8 values 2 * e2m1
// (0, +-1, 2, 3, 4, 6, 8, 12), byte for byte.
__device__ __forceinline__ uint32_t e2m1x4_to_i8(uint32_t n) {
  const uint32_t m = n & 0x07070707u;
  const uint32_t pos = __builtin_amdgcn_perm(0x0c080604u, 0x03020100u, m);
  const uint32_t neg = __builtin_amdgcn_perm(0xf4f8fafcu, 0xfdfeff00u, m);
  const uint32_t s = ((n >> 3) & 0x01010101u) * 0xffu;
  return (pos & ~s) | (neg & s);
}

// Four packed e2m1 bytes (eight values) -> eight int8 2 * e2m1 values: the
// low nibbles (even elements) in the low word, the high nibbles in the high
// word.  Dot products over all eight are unchanged by this element order as
// long as both operands use it.
__device__ __forceinline__ int64_t fp4x8_to_i8(uint32_t w) {
  const uint32_t lo = e2m1x4_to_i8(w & 0x0f0f0f0fu), hi = e2m1x4_to_i8((w >> 4) & 0x0f0f0f0fu);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T wave_max_xor(T v, int width) {
  for (int m = width >> 1; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, width));
  return v;
}

}  // namespace ekv
