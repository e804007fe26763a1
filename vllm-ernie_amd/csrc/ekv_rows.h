// Device-side row append shared by the write kernels: a bf16 row ->
// per-token UE8M0 scale + e4m3 codes stored in a values-then-scales page
// pool, the per-call row append, and the HCA tail (window ring and
// compressor state ring rows of each sequence).
#pragma once

#include "ekv_common.h"
#include "ekv_internal.h"

namespace ekv {

// ---------------------------------------------------------------------------
// kv_append_quant
// ---------------------------------------------------------------------------
struct AppendArgs {
  const uint16_t* rows;      // [T, row_stride] bf16
  int64_t row_stride;        // elements
  int32_t num_tokens;
  const int64_t* slot_mapping;  // [T], < 0 -> skip
  uint8_t* cache;            // [num_pages, page_stride]
  int64_t page_stride;
  int64_t num_pages;
  // HCA extras (all optional)
  const int64_t* positions;  // [T]
  const int32_t* token_seq;  // [T], < 0 -> padding
  const int32_t* qsl;        // [B + 1]
  const int32_t* ring_pages; // [B, ring_stride]
  int32_t ring_stride;
  int32_t ring;              // ring length R (multiple of 64)
  const uint16_t* kv_score;  // [T, kvs_stride] bf16, 2*D wide
  int64_t kvs_stride;
  uint16_t* state;           // [num_state, 256, 2*D] bf16
  const int32_t* state_slot; // [B]
  int32_t num_state;
  // indexer K prep before the quantization (D = 128 only; optional): rows
  // are the raw projection, made hadamard(rope(k_norm(row))) with the
  // LayerNorm (ln_w, ln_b, eps) and cos_sin row positions[t]
  const float* ln_w;
  const float* ln_b;
  float eps;
  const float* cos_sin;      // [cs_rows, 64]; nullptr = no prep
  int32_t cs_rows;
  // HCA pools of bf16 rows (page = 64 rows of D bf16 values, no scales):
  // the rows are stored as they come, not quantized
  int32_t bf16_rows;
};

// ---------------------------------------------------------------------------
// Indexer prep on a 128-wide row held by a 16-lane group: lane j holds
// elements 8j .. 8j+7 (fp32 copies of bf16 values); cross-lane partners are
// lane ^ 1, 2, 4, 8, inside the group.  k_norm LayerNorm, NeoX RoPE on dims
// 0..63 and the Hadamard of Ernie5_5Indexer.forward.
// ---------------------------------------------------------------------------
// Sum of the row: per lane ((v0+v1)+(v2+v3))+((v4+v5)+(v6+v7)), then a
// butterfly over the 16 lanes (partners 1, 2, 4, 8); every lane ends with the
// same balanced-tree total.
__device__ __forceinline__ float row_sum16(const float (&v)[8]) {
  float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) s = s + __shfl_xor(s, off);
  return s;
}

// y = bf16((d * rstd) * w + b), d = x - mean, over the 128-wide row.
__device__ __forceinline__ void row_layer_norm(float (&v)[8], const float* w, const float* b, float eps, int j) {
  const float mean = __fdiv_rn(row_sum16(v), 128.0f);
  float d[8], sq[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    d[e] = v[e] - mean;
    sq[e] = d[e] * d[e];
  }
  const float var = __fdiv_rn(row_sum16(sq), 128.0f);
  const float rstd = __fdiv_rn(1.0f, __fsqrt_rn(var + eps));
  const float4 w0 = *reinterpret_cast<const float4*>(w + 8 * j), w1 = *reinterpret_cast<const float4*>(w + 8 * j + 4);
  const float4 b0 = *reinterpret_cast<const float4*>(b + 8 * j), b1 = *reinterpret_cast<const float4*>(b + 8 * j + 4);
  const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = bf16_to_f32(f32_to_bf16((d[e] * rstd) * ww[e] + bb[e]));
}

// The cos / sin entries lane j of a 16-lane row group uses in
// row_rope_neox64 (lanes 0..7; cs == nullptr: none).
struct RopeLane {
  float c[8], sn[8];
  bool on;
};
__device__ __forceinline__ RopeLane rope_lane(const float* cs, int j) {
  RopeLane r;
  r.on = cs != nullptr && j < 8;
  const int i0 = 8 * (j & 3);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    r.c[e] = r.on ? cs[i0 + e] : 0.0f;
    r.sn[e] = r.on ? cs[32 + i0 + e] : 0.0f;
  }
  return r;
}

// NeoX rotation of dims 0..63 by (cos_i, sin_i) = (cs[i], cs[32 + i]): dim i
// (lanes 0..3) pairs with dim i + 32 (lanes 4..7); cs == nullptr leaves the
// row as it is.  The _lane form takes lane j's entries already loaded.
__device__ __forceinline__ void row_rope_neox64_lane(float (&v)[8], const RopeLane& r, int j) {
  float p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = __shfl_xor(v[e], 4);
  if (!r.on) return;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float res = (j < 4) ? (v[e] * r.c[e]) - (p[e] * r.sn[e])   // x1 c - x2 s
                              : (v[e] * r.c[e]) + (p[e] * r.sn[e]);  // x2 c + x1 s
    v[e] = bf16_to_f32(f32_to_bf16(res));
  }
}
__device__ __forceinline__ void row_rope_neox64(float (&v)[8], const float* cs, int j) {
  row_rope_neox64_lane(v, rope_lane(cs, j), j);
}

// Orthonormal Walsh-Hadamard of the row: spans 1, 2, ..., 64 with
// (a, b) -> (a + b, a - b), then times fl32(1/sqrt(128)), rounded to bf16.
__device__ __forceinline__ void row_hadamard(float (&v)[8], int j) {
#pragma unroll
  for (int h = 1; h < 8; h <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if ((e & h) == 0) {
        const float a = v[e], b = v[e + h];
        v[e] = a + b;
        v[e + h] = a - b;
      }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    const bool lower = (j & m) == 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __shfl_xor(v[e], m);
      v[e] = lower ? (v[e] + p) : (p - v[e]);
    }
  }
  const float s = 0x1.6a09e6p-4f;  // fl32(1/sqrt(128))
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = bf16_to_f32(f32_to_bf16(v[e] * s));
}

__device__ __forceinline__ void unpack_bf16x8(uint4 w, float (&v)[8]) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(ww[i] << 16);
    v[2 * i + 1] = __uint_as_float(ww[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 pack_bf16x8(const float (&v)[8]) {
  uint32_t ww[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ww[i] = (__float_as_uint(v[2 * i]) >> 16) | (__float_as_uint(v[2 * i + 1]) & 0xffff0000u);
  return make_uint4(ww[0], ww[1], ww[2], ww[3]);
}

// One row's fp8 image: lane `ln` of the row's kLanes lanes holds the 8-byte
// pieces ln, ln + kLanes, ... of the D fp8 codes, plus the row's scale.
template <int D, int kLanes>
struct Fp8Row {
  static constexpr int kChunks = D / 8;  // 16-byte bf16 chunks per row
  static constexpr int kPerLane = (kChunks + kLanes - 1) / kLanes;
  uint2 packed[kPerLane];
  float scale;
};

template <int D, int kLanes>
__device__ __forceinline__ void load_bf16_row(const uint16_t* src, int ln,
                                              uint4 (&raw)[Fp8Row<D, kLanes>::kPerLane]) {
  using R = Fp8Row<D, kLanes>;
#pragma unroll
  for (int k = 0; k < R::kPerLane; ++k) {
    const int c = ln + k * kLanes;
    raw[k] = c < R::kChunks ? *reinterpret_cast<const uint4*>(src + 8 * c) : make_uint4(0, 0, 0, 0);
  }
}

// Per-token UE8M0 scale and e4m3 codes of one bf16 row (kLanes lanes).
template <int D, int kLanes>
__device__ __forceinline__ Fp8Row<D, kLanes> quantize_row(const uint4 (&raw)[Fp8Row<D, kLanes>::kPerLane]) {
  using R = Fp8Row<D, kLanes>;
  float v[R::kPerLane][8];
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < R::kPerLane; ++k) {
    const uint32_t ww[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[k][2 * i] = __uint_as_float(ww[i] << 16);
      v[k][2 * i + 1] = __uint_as_float(ww[i] & 0xffff0000u);
      amax = fmaxf(amax, fmaxf(fabsf(v[k][2 * i]), fabsf(v[k][2 * i + 1])));
    }
  }
  amax = wave_max_xor(amax, kLanes);
  const int e = ue8m0_exponent(amax);
  const float inv = exp2i(-e);
  R out;
  out.scale = exp2i(e);
#pragma unroll
  for (int k = 0; k < R::kPerLane; ++k) {
    const uint32_t b0 = f32x2_to_fp8(v[k][0] * inv, v[k][1] * inv);
    const uint32_t b1 = f32x2_to_fp8(v[k][2] * inv, v[k][3] * inv);
    const uint32_t b2 = f32x2_to_fp8(v[k][4] * inv, v[k][5] * inv);
    const uint32_t b3 = f32x2_to_fp8(v[k][6] * inv, v[k][7] * inv);
    out.packed[k] = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
  }
  return out;
}

// Store a quantized row at `slot` of a values-then-scales page pool; slots
// outside the pool (negative = skip) are not written.
template <int D, int kLanes>
__device__ __forceinline__ void store_fp8_row(const AppendArgs& a, int64_t slot, int ln,
                                              const Fp8Row<D, kLanes>& row) {
  using R = Fp8Row<D, kLanes>;
  if (slot < 0 || slot >= a.num_pages * kPageTokens) return;
  uint8_t* page = a.cache + (slot / kPageTokens) * a.page_stride;
  const int64_t off = slot % kPageTokens;
#pragma unroll
  for (int k = 0; k < R::kPerLane; ++k) {
    const int c = ln + k * kLanes;
    if (c < R::kChunks) *reinterpret_cast<uint2*>(page + off * D + 8 * c) = row.packed[k];
  }
  if (ln == 0) *reinterpret_cast<float*>(page + kPageTokens * D + off * 4) = row.scale;
}

// Store a bf16 row at `slot`: quantized into a values-then-scales fp8 page
// pool, or as it is into a pool of bf16 rows (a.bf16_rows).
template <int D, int kLanes>
__device__ __forceinline__ void store_row(const AppendArgs& a, int64_t slot, int ln,
                                          const uint4 (&raw)[Fp8Row<D, kLanes>::kPerLane]) {
  using R = Fp8Row<D, kLanes>;
  if (!a.bf16_rows) {
    store_fp8_row<D, kLanes>(a, slot, ln, quantize_row<D, kLanes>(raw));
    return;
  }
  if (slot < 0 || slot >= a.num_pages * kPageTokens) return;
  uint8_t* row = a.cache + (slot / kPageTokens) * a.page_stride + (slot % kPageTokens) * (2 * D);
#pragma unroll
  for (int k = 0; k < R::kPerLane; ++k) {
    const int c = ln + k * kLanes;
    if (c < R::kChunks) *reinterpret_cast<uint4*>(row + 16 * c) = raw[k];
  }
}

// Rows of workgroup `block`, stored at their slot_mapping slots: kWaves
// waves, each taking kSeq groups of kRowsPerWave rows (4 rows of 16 lanes for
// D = 128, else one row of 64 lanes).  A wave issues the loads of all its
// rows (and their slots) before it quantizes and stores any of them.
template <int D, int kSeq, int kWaves = 4>
__device__ __forceinline__ void append_rows(const AppendArgs& a, int block) {
  constexpr int kRowsPerWave = (D == 128) ? 4 : 1;
  constexpr int kLanes = 64 / kRowsPerWave;       // lanes per row
  using R = Fp8Row<D, kLanes>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / kLanes;                  // row within the wave
  const int ln = lane % kLanes;                   // lane within the row
  const int64_t t_first = (static_cast<int64_t>(block) * kWaves + wave) * kSeq * kRowsPerWave + sub;

  uint4 raw[kSeq][R::kPerLane];
  int64_t slot[kSeq];
#pragma unroll
  for (int r = 0; r < kSeq; ++r) {
    const int64_t t = t_first + r * kRowsPerWave;
    const int64_t tt = t < a.num_tokens ? t : 0;
    load_bf16_row<D, kLanes>(a.rows + tt * a.row_stride, ln, raw[r]);
    slot[r] = a.slot_mapping[tt];
    if constexpr (D == 128) {
      if (a.cos_sin != nullptr) {  // uniform: every row of the launch or none
        float v[8];
        unpack_bf16x8(raw[r][0], v);
        const int64_t pos = a.positions[tt];
        row_layer_norm(v, a.ln_w, a.ln_b, a.eps, ln);
        row_rope_neox64(v, (pos >= 0 && pos < a.cs_rows) ? a.cos_sin + pos * 64 : nullptr, ln);
        row_hadamard(v, ln);
        raw[r][0] = pack_bf16x8(v);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kSeq; ++r) {
    if (t_first + r * kRowsPerWave >= a.num_tokens) return;  // whole row group exits together
    store_row<D, kLanes>(a, slot[r], ln, raw[r]);
  }
}

// HCA extras of one call, for the last rows of each sequence: row k from the
// end of sequence b (position last - k, positions of a sequence's rows in a
// call being consecutive) goes to the window ring when k < ring, and its
// kv_score row to the compressor state ring when k < 256.  This takes rows
// k_lo <= k < k_hi of sequence b, kBatch per wave and step (the loads of a
// step issued before its stores), over the workgroup's kWaves waves.  Of the
// state rows it writes those whose ring slot p % 256 lies in
// [alias_lo, alias_lo + alias_n) exactly when `in_alias`, and ring rows only
// when `ring_rows`.
template <int D, int kWaves, int kBatch>
__device__ __forceinline__ void hca_tail_range(const AppendArgs& a, int b, int k_lo, int k_hi, bool ring_rows = true,
                                               int alias_lo = 0, int alias_n = 0, bool in_alias = false) {
  using R = Fp8Row<D, 64>;
  constexpr int kStateChunks = 2 * R::kChunks;            // 16-byte chunks of a kv_score row
  constexpr int kStatePerLane = (kStateChunks + 63) / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t0 = a.qsl[b];
  const int n = a.qsl[b + 1] - t0;
  const int64_t last = a.positions[t0] + n - 1;
  const int st = a.state != nullptr ? a.state_slot[b] : -1;
  const bool state_ok = st >= 0 && st < a.num_state;
  const bool ring_ok = ring_rows && a.ring_pages != nullptr;
  if (k_hi > n) k_hi = n;
  for (int kb = k_lo + wave * kBatch; kb < k_hi; kb += kWaves * kBatch) {
    uint4 raw[kBatch][R::kPerLane];
    uint4 sv[kBatch][kStatePerLane];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k = kb + u < k_hi ? kb + u : kb;
      const int64_t t = t0 + n - 1 - k;
      if (ring_ok) load_bf16_row<D, 64>(a.rows + t * a.row_stride, lane, raw[u]);
      if (state_ok && k < kStateRing) {
        const uint4* sp = reinterpret_cast<const uint4*>(a.kv_score + t * a.kvs_stride);
#pragma unroll
        for (int i = 0; i < kStatePerLane; ++i) {
          const int c = lane + 64 * i;
          sv[u][i] = c < kStateChunks ? sp[c] : make_uint4(0, 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k = kb + u;
      if (k >= k_hi) break;
      const int64_t p = last - k;
      if (ring_ok && k < a.ring) {
        const int64_t rp = p % a.ring;
        const int64_t sl =
            static_cast<int64_t>(a.ring_pages[static_cast<int64_t>(b) * a.ring_stride + rp / kPageTokens]) *
                kPageTokens + rp % kPageTokens;
        store_row<D, 64>(a, sl, lane, raw[u]);
      }
      const int64_t rel = p % kStateRing - alias_lo;
      if (state_ok && k < kStateRing && (rel >= 0 && rel < alias_n) == in_alias) {
        uint4* d =
            reinterpret_cast<uint4*>(a.state + (static_cast<int64_t>(st) * kStateRing + p % kStateRing) * (2 * D));
#pragma unroll
        for (int i = 0; i < kStatePerLane; ++i) {
          const int c = lane + 64 * i;
          if (c < kStateChunks) d[c] = sv[u][i];
        }
      }
    }
  }
}

// Rows from the end of a sequence that hca_tail_range has to cover: the
// window ring's and the state ring's, whichever is longer.
inline int hca_tail_span(bool ring_ok, int ring) { return ring_ok && ring > kStateRing ? ring : kStateRing; }

// Rows per workgroup of append_rows<D, kSeq, waves>.
constexpr int append_block_rows(int d, int seq, int waves = 4) { return waves * seq * (d == 128 ? 4 : 1); }

// Rows each wave keeps in flight in the standalone append launches.
template <int D>
constexpr int kAppendSeq = (D == 128) ? 1 : 4;

// HCA append grid: workgroups [0, main_blocks) store every row at its slot,
// the rest write the window ring and state ring rows of each sequence's
// tail, kTailBlockRows rows of one sequence each.  Returns the block count.
constexpr int kTailBlockRows = 16;
inline int64_t hca_append_grid(const AppendArgs& a, int dim, int num_seqs, bool rows, bool tail, int& main_blocks,
                               int& tail_rows) {
  const int rows_per_block = append_block_rows(dim, kAppendSeq<576>);
  main_blocks = rows ? (a.num_tokens + rows_per_block - 1) / rows_per_block : 0;
  // each sequence's last max(ring, 256) rows, in whole tail workgroups
  tail_rows = (hca_tail_span(a.ring_pages != nullptr, a.ring) + kTailBlockRows - 1) / kTailBlockRows * kTailBlockRows;
  const bool any_tail = tail && (a.ring_pages != nullptr || a.state != nullptr);
  return main_blocks + (any_tail ? static_cast<int64_t>(num_seqs) * (tail_rows / kTailBlockRows) : 0);
}

// One append grid block: a row block or a tail block (256 threads).
template <int D>
__device__ __forceinline__ void hca_append_block(const AppendArgs& a, int block, int main_blocks, int tail_rows) {
  if (block < main_blocks) {
    append_rows<D, kAppendSeq<D>>(a, block);
    return;
  }
  const int tb = block - main_blocks;
  const int blocks_per_seq = tail_rows / kTailBlockRows;
  const int k_lo = (tb % blocks_per_seq) * kTailBlockRows;
  hca_tail_range<D, 4, 1>(a, tb / blocks_per_seq, k_lo, k_lo + kTailBlockRows);
}


// Argument checks and AppendArgs of an HCA append (the latent rows, the
// window ring and the compressor state ring); 0 or an error status.
inline int hca_append_args(AppendArgs& a, const uint16_t* latent, int64_t latent_stride, const uint16_t* kv_score,
                           int64_t kvs_stride, int32_t num_tokens, int32_t dim, const int64_t* slot_mapping,
                           const int64_t* positions, const int32_t* token_seq, const int32_t* qsl,
                           int32_t num_seqs, uint8_t* pool, int64_t page_stride, int64_t num_pages,
                           const int32_t* ring_pages, int32_t ring_stride, int32_t ring, uint16_t* state,
                           const int32_t* state_slot, int32_t num_state, bool bf16_rows = false) {
  EKV_CHECK(num_tokens >= 0 && num_seqs >= 0, "sizes must be >= 0");
  EKV_CHECK(dim == 512 || dim == 576, "HCA dim must be 512 or 576");
  EKV_CHECK(latent && slot_mapping && positions && token_seq && qsl && pool, "null pointer");
  EKV_CHECK(latent_stride >= dim && latent_stride % 8 == 0, "bad latent_stride");
  EKV_CHECK(page_stride >= kPageTokens * (bf16_rows ? 2 * dim : dim + 4) && page_stride % 16 == 0,
            "bad page_stride");
  EKV_CHECK(ring_pages == nullptr || (ring >= kWindow && ring % kPageTokens == 0 && ring_stride >= ring / kPageTokens),
            "ring must be a multiple of 64, >= 128, with ring_stride >= ring/64");
  EKV_CHECK(state == nullptr || (kv_score && state_slot && kvs_stride >= 2 * dim && kvs_stride % 8 == 0),
            "state needs kv_score (stride >= 2*dim, multiple of 8) and state_slot");
  EKV_CHECK(aligned16(latent) && aligned16(pool) && (state == nullptr || (aligned16(state) && aligned16(kv_score))),
            "buffers must be 16-byte aligned");
  a = AppendArgs{};
  a.rows = latent; a.row_stride = latent_stride; a.num_tokens = num_tokens; a.slot_mapping = slot_mapping;
  a.cache = pool; a.page_stride = page_stride; a.num_pages = num_pages;
  a.positions = positions; a.token_seq = token_seq; a.qsl = qsl;
  a.ring_pages = ring_pages; a.ring_stride = ring_stride; a.ring = ring;
  a.kv_score = kv_score; a.kvs_stride = kvs_stride; a.state = state; a.state_slot = state_slot;
  a.num_state = num_state;
  a.bf16_rows = bf16_rows ? 1 : 0;
  return 0;
}

// Launch the HCA append of `a` on s: the rows at their slots (`rows`) and/or
// each sequence's window-ring and state-ring tail (`tail`); 0 or an error
// status.  Defined with the append kernels.
int launch_hca_append(const AppendArgs& a, int dim, int num_seqs, bool rows, bool tail, hipStream_t s);

// ---------------------------------------------------------------------------
// HCA decode index rows: [compressed slots 0..n_c-1 | window slots of
// positions p-w+1..p | -1 ...], n_c = (p+1)/128, w = min(p+1, window), and
// the row lengths.  Window entries of positions at or after the first
// position of the row's request in this call come from the call's own slots
// (call_slots, by the request's qsl range) when call_slots is given, others
// from the ring.  Block (t, y) of 256 threads writes entries
// [kIdxPerBlock y, kIdxPerBlock (y + 1)) of row t, kIdxPerThread per thread
// with their table loads issued together.
// ---------------------------------------------------------------------------
struct HcaIndexArgs {
  const int64_t* positions;
  const int32_t* req_ids;
  const int32_t* comp_bt;
  int32_t comp_bt_stride;
  const int32_t* ring_pages;
  int32_t ring_stride;
  int32_t ring;
  int32_t window;
  const int32_t* qsl;
  const int64_t* call_slots;
  int32_t* out;
  int64_t out_stride;
  int32_t width;
  int32_t* lengths;
};

constexpr int kIdxPerThread = 4;
constexpr int kIdxPerBlock = 256 * kIdxPerThread;

__host__ __device__ inline int hca_index_blocks_per_row(int width) {
  return width > kIdxPerBlock ? (width + kIdxPerBlock - 1) / kIdxPerBlock : 1;
}

__device__ __forceinline__ void hca_index_block(const HcaIndexArgs& a, int64_t t, int y) {
  const int64_t p = a.positions[t];
  const int64_t b = a.req_ids[t];
  const int64_t t0 = a.call_slots ? a.qsl[b] : 0;
  const int64_t call_first = a.call_slots ? a.positions[t0] : INT64_MAX;
  const int64_t nc = (p + 1) / kSpan;
  const int64_t w = min(p + 1, static_cast<int64_t>(a.window));
  const int64_t len = min(nc + w, static_cast<int64_t>(a.width));
  int64_t v[kIdxPerThread];
#pragma unroll
  for (int j = 0; j < kIdxPerThread; ++j) {
    const int c = y * kIdxPerBlock + j * 256 + static_cast<int>(threadIdx.x);
    v[j] = -1;
    if (c < nc) {
      v[j] = static_cast<int64_t>(a.comp_bt[b * a.comp_bt_stride + c / kPageTokens]) * kPageTokens + c % kPageTokens;
    } else if (c < len) {
      const int64_t pos = p - w + 1 + (c - nc);
      if (pos >= call_first) {
        const int64_t sv = a.call_slots[t0 + (pos - call_first)];
        v[j] = sv < 0 ? -1 : sv;
      } else {
        const int64_t r = pos % a.ring;
        v[j] = static_cast<int64_t>(a.ring_pages[b * a.ring_stride + r / kPageTokens]) * kPageTokens +
               r % kPageTokens;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kIdxPerThread; ++j) {
    const int c = y * kIdxPerBlock + j * 256 + static_cast<int>(threadIdx.x);
    if (c < a.width) a.out[t * a.out_stride + c] = static_cast<int32_t>(v[j]);
  }
  if (y == 0 && threadIdx.x == 0) a.lengths[t] = static_cast<int32_t>(len);
}

}  // namespace ekv
