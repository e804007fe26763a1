// Sparse MLA decode over gathered latent rows (DSA top-k + window, HCA
// compressed + window), with the per-head attention sink in the softmax
// denominator.
//
// Workgroup = (query row t, split s of its index row), 512 threads in two
// roles, one barrier per tile of 32 index entries.  Between two barriers:
//   * score waves 0..3 (q for heads 16w .. 16w+15 held in registers) first
//     finish tile t-1 (below), then compute S = Q K^T of tile t on
//     v_mfma_f32_16x16x32_bf16 from a bf16 K image in LDS, run the online
//     softmax and write P (bf16, row scale folded in) for their heads; fp8
//     K fragments become bf16 in registers (exact conversion);
//   * data waves 4..7 finish tile t-1, store tile t+1 (the rows as cached:
//     e4m3fn bytes, or bf16) into the next of three K images, and issue the
//     loads of tile t+3 (8 rows per wave, row addresses in scalar registers,
//     256-byte coalesced loads into registers, two tiles in flight);
//   * "finish tile t-1" = O[:, 64w .. 64w+63] += P V for all heads, every wave
//     taking its 64 channels.  The B operand (V, entries x channels) is read
//     straight from the row-major K image with a transposing LDS read
//     (ds_read_b64_tr_b8 for fp8 rows, ds_read_b64_tr_b16 for bf16); no
//     separate V^T image is built.
// A prologue resolves every index entry of the split to a cache slot (block
// table lookup) and fp32 row scale once.  The softmax reference max only
// moves when a score exceeds it by more than 8 (log2 units), so O is rescaled
// rarely.  Each split leaves O / l in bf16 plus (m, l) in fp32; the combine
// kernel merges the splits, adds the sink and writes bf16 out and the
// natural-log lse (log sum_j exp(s_j), sink excluded).
#include "ekv_common.h"
#include "ekv_internal.h"

#include <type_traits>

namespace ekv {

constexpr int kDv = 512;
constexpr int kTile = 32;
constexpr int kScoreWaves = 4;               // up to 64 heads (one wave per 16)
constexpr int kDataWaves = 4;
constexpr int kThreads = 64 * (kScoreWaves + kDataWaves);
constexpr int kRowsPerDataWave = kTile / kDataWaves;   // 8
constexpr int kKImages = 3;                  // tile t-1 (P V), t (S), t+1 (being stored)
constexpr int kMaxSplitEntries = 1024;       // index entries one workgroup resolves
constexpr int kTargetGroups = 256;           // one workgroup per CU
constexpr float kRescaleSlack = 8.0f;        // log2 units: P <= 2**8 between rescales
constexpr float kLog2e = 0x1.715476p+0f;
constexpr float kLn2 = 0x1.62e430p-1f;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

struct DecodeArgs {
  const uint16_t* q;        // [T, H, D] bf16
  int64_t q_tok_stride, q_head_stride;
  const uint8_t* cache;     // fp8 pages [num_pages, page_stride] or bf16 rows
  int64_t page_stride;      // bytes (fp8 layout)
  int64_t num_rows;         // addressable rows (num_pages * 64), < 2**31
  const int32_t* indices;   // [T, idx_stride]
  int64_t idx_stride;
  int32_t width;            // entries per index row
  const int32_t* lengths;   // [T] or null
  const int32_t* block_table;  // logical indices when non-null
  int64_t bt_stride;
  const int32_t* req_ids;   // [T] with block_table
  float scale;              // softmax scale
  int32_t heads;
  int32_t per_split;        // entries per split (multiple of kTile, <= kMaxSplitEntries)
  float* ws_o;              // [T, NS, H, 512] fp32, O / l of the split
  float* ws_ml;             // [T, NS, H, 2] (m in log2 units, l)
  int32_t splits;
};

// K images hold the tile's rows as stored: raw e4m3fn bytes (fp8 cache) or
// bf16.  The fp8 row stride D + 8 bytes is 8 (mod 16) words: the 16 rows a
// QK fragment read touches land on distinct bank pairs.
template <int D, bool BF16>
struct DecodeSmem {
  static constexpr int kKRowB = BF16 ? 2 * (D + 8) : D + 8;  // K row stride (bytes)
  static constexpr int kImgB = kTile * kKRowB;
  static constexpr int kPRow = kTile + 8;   // bf16 P row stride (elements)
  __align__(16) uint8_t img[kKImages * kImgB];
  uint16_t p[2][64 * kPRow];                // P of tiles t (written) and t-1 (read)
  float alpha[2][64];                       // rescale factor per head (valid when grow[.][head / 16])
  int32_t grow[2][kScoreWaves];
  float row_l[64];
  int32_t slot[kMaxSplitEntries];
  float kscale[kMaxSplitEntries];
};

// Four e4m3fn bytes -> four bf16 (exact: every e4m3fn value is a bf16 value).
__device__ __forceinline__ uint2 fp8x4_bf16(uint32_t w) {
  const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
  return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

// Max / sum over each row of 16 lanes, every lane receiving the result:
// DPP row rotations by 8, 4, 2, 1 (VALU only, no LDS round trip).
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0x128>(v));  // row_ror:8
  v = fmaxf(v, dpp_f32<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_f32<0x122>(v));  // row_ror:2
  return fmaxf(v, dpp_f32<0x121>(v));  // row_ror:1
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0x128>(v);
  v += dpp_f32<0x124>(v);
  v += dpp_f32<0x122>(v);
  return v + dpp_f32<0x121>(v);
}

__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};  // round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

// ds_read_b64_tr_b16: in each row of 16 lanes, lane j receives 16-bit element
// j % 4 of the 8 bytes addressed by lanes j / 4 + 4m (m = 0..3).
__device__ __forceinline__ i16x4 lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)((__attribute__((address_space(3))) uint16_t*)(p)));
}

// ---------------------------------------------------------------------------
// Data role: rows 8u .. 8u+7 of a tile, 4-channel units lane + 64 j.
template <int D, bool BF16>
struct RowRegs {
  using Unit = typename std::conditional<BF16, uint2, uint32_t>::type;
  static constexpr int kUnits = D / 4;                   // 4-channel units per row
  static constexpr int kJ = (kUnits + 63) / 64;
  Unit v[kRowsPerDataWave][kJ];
  float ks;                                              // lane r < 8: fp32 scale of row r
  uint32_t valid;                                        // bit rr: row rr holds data (wave-uniform)
  bool live;                                             // the tile exists
};

// Issue every load of tile `tile` for this data wave.  Masked rows and tiles
// past the end read the first cache row and stay flagged invalid, so that the
// wait before each store to LDS counts exactly the loads issued after it.
template <int D, bool BF16>
__device__ __forceinline__ void fetch_rows(const DecodeArgs& a, const DecodeSmem<D, BF16>& sm, int u, int tile, int ntiles,
                                           RowRegs<D, BF16>& rr) {
  using RR = RowRegs<D, BF16>;
  const bool live = tile < ntiles;
  const int tb = (live ? tile : 0) * kTile + kRowsPerDataWave * u;
  const int lane = threadIdx.x & 63;
  uint32_t valid = 0;
  // One LDS read gives lane r the slot of row r; rows then become uniform.
  const int my_slot = sm.slot[tb + (lane & (kRowsPerDataWave - 1))];
  const int ks_slot = (live && my_slot >= 0) ? my_slot : 0;
  // Keep each tile's loads in issue order relative to the other tiles' loads
  // (the register buffers are consumed oldest first).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < kRowsPerDataWave; ++r) {
    const int slot = __builtin_amdgcn_readlane(my_slot, r);
    const bool ok = live && slot >= 0;
    const int s = ok ? slot : 0;
    const uint8_t* row = BF16 ? a.cache + static_cast<int64_t>(s) * (2 * D)
                              : a.cache + static_cast<int64_t>(s >> 6) * a.page_stride + (s & 63) * D;
    valid |= static_cast<uint32_t>(ok) << r;
#pragma unroll
    for (int j = 0; j < RR::kJ; ++j) {
      const int unit = (RR::kUnits % 64 == 0 || lane + 64 * j < RR::kUnits) ? lane + 64 * j : RR::kUnits - 1;
      rr.v[r][j] = *reinterpret_cast<const typename RR::Unit*>(row + unit * sizeof(typename RR::Unit));
    }
  }
  // the rows' fp32 scales, lane r for row r (after the values of the page)
  if constexpr (BF16) rr.ks = 1.0f;
  else rr.ks = *reinterpret_cast<const float*>(a.cache + static_cast<int64_t>(ks_slot >> 6) * a.page_stride +
                                                kPageTokens * D + (ks_slot & 63) * 4);
  __builtin_amdgcn_sched_barrier(0);
  rr.valid = valid;
  rr.live = live;
}

// Store the wave's 8 rows into a K image as they are (masked rows become
// zero, so that P = 0 never meets a non-finite value in P V).  Lanes past the
// end of a row repeat its last unit: a duplicate store of equal data.
template <int D, bool BF16>
__device__ __forceinline__ void store_rows(const RowRegs<D, BF16>& rr, int u, int tile, DecodeSmem<D, BF16>& sm,
                                           uint8_t* k) {
  using RR = RowRegs<D, BF16>;
  using SM = DecodeSmem<D, BF16>;
  const int lane = threadIdx.x & 63;
  if (rr.live && lane < kRowsPerDataWave)
    sm.kscale[tile * kTile + kRowsPerDataWave * u + lane] = ((rr.valid >> lane) & 1u) ? rr.ks : 0.0f;
#pragma unroll
  for (int r = 0; r < kRowsPerDataWave; ++r) {
    const bool ok = (rr.valid >> r) & 1u;
    uint8_t* row = k + (kRowsPerDataWave * u + r) * SM::kKRowB;
#pragma unroll
    for (int j = 0; j < RR::kJ; ++j) {
      const int unit = (RR::kUnits % 64 == 0 || lane + 64 * j < RR::kUnits) ? lane + 64 * j : RR::kUnits - 1;
      if constexpr (BF16) *reinterpret_cast<uint2*>(row + 8 * unit) = ok ? rr.v[r][j] : make_uint2(0u, 0u);
      else *reinterpret_cast<uint32_t*>(row + 4 * unit) = ok ? rr.v[r][j] : 0u;
    }
  }
}

// Eight e4m3fn bytes -> bf16x8 (exact).
__device__ __forceinline__ bf16x8 fp8x8_bf16(uint2 w) {
  const uint2 lo = fp8x4_bf16(w.x), hi = fp8x4_bf16(w.y);
  return __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// ds_read_b64_tr_b8: in each row of 16 lanes, lane j receives byte j % 8 of
// the 8 bytes addressed by lanes j / 8 + 2m (m = 0..7), as byte m.
typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 lds_read_tr8(const uint8_t* p) {
  const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
      (__attribute__((address_space(3))) i32x2*)((__attribute__((address_space(3))) uint8_t*)(p)));
  return make_uint2(static_cast<uint32_t>(v.x), static_cast<uint32_t>(v.y));
}

// ---------------------------------------------------------------------------
// O[:, 64w .. 64w+63] += P V for every head group (all waves).  o[hf][nt]
// holds heads 16hf + 4g + i, channels 64w + 16nt + col.
template <int D, bool BF16>
__device__ __forceinline__ void accumulate_pv(const DecodeSmem<D, BF16>& sm, const uint8_t* kimg, int pb, int hgroups,
                                              f32x4 (&o)[4][4]) {
  using SM = DecodeSmem<D, BF16>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int g = lane >> 4, col = lane & 15;
  // B operand: entries 8g .. 8g+7 at channel 64w + 16nt + col.
  bf16x8 vb[4];
  if constexpr (BF16) {
    // two 16-bit transposed reads of rows 8g + 4h + col/4, channels
    // 64w + 16nt + 4 (col % 4) .. +3
    const uint16_t* vbase = reinterpret_cast<const uint16_t*>(kimg + (8 * g + (col >> 2)) * SM::kKRowB) + 64 * wave +
                            4 * (col & 3);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const i16x4 lo = lds_read_tr16(vbase + 16 * nt);
      const i16x4 hi = lds_read_tr16(vbase + 2 * SM::kKRowB + 16 * nt);
      const i16x4 both[2] = {lo, hi};
      vb[nt] = __builtin_bit_cast(bf16x8, both);
    }
  } else {
    // one 8-bit transposed read: lane col of row block g addresses row
    // 8g + col/2, channels 64w + 16nt + 8 (col % 2) .. +7
    const uint8_t* vbase = kimg + (8 * g + (col >> 1)) * SM::kKRowB + 64 * wave + 8 * (col & 1);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) vb[nt] = fp8x8_bf16(lds_read_tr8(vbase + 16 * nt));
  }
  // All operands are read before the first product; the rescale (rare) and
  // the products of head groups past `hgroups` (unused) need no branches.
  bf16x8 pa[4];
#pragma unroll
  for (int hf = 0; hf < 4; ++hf)
    pa[hf] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&sm.p[pb][(16 * hf + col) * SM::kPRow + 8 * g]));
  const int4 gr = *reinterpret_cast<const int4*>(sm.grow[pb]);
  const int grow_any = (gr.x | (hgroups > 1 ? gr.y : 0) | (hgroups > 2 ? gr.z : 0) | (hgroups > 3 ? gr.w : 0));
  if (__builtin_amdgcn_readfirstlane(grow_any)) {
    const int grs[4] = {gr.x, gr.y, gr.z, gr.w};
#pragma unroll
    for (int hf = 0; hf < 4; ++hf) {
      if (!grs[hf]) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float al = sm.alpha[pb][16 * hf + 4 * g + i];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) o[hf][nt][i] *= al;
      }
    }
  }
#pragma unroll
  for (int hf = 0; hf < 4; ++hf)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) o[hf][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[hf], vb[nt], o[hf][nt], 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Score role: S = Q K^T for heads 16w .. 16w+15 over one tile, online softmax,
// P (times the row scale, bf16) and the rescale factors to LDS buffer pb.
struct SoftmaxState {
  float m2[4];    // reference max (log2 units) of heads 4g + i
  float lsum[4];  // this lane's share of the denominator relative to m2
};

template <int D, bool BF16>
__device__ __forceinline__ void score_tile(DecodeSmem<D, BF16>& sm, const uint8_t* kimg, int pb, int tb, float sc2,
                                           const bf16x8 (&qa)[D / 32], SoftmaxState& st) {
  using SM = DecodeSmem<D, BF16>;
  constexpr int KS = D / 32;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int g = lane >> 4, col = lane & 15;
  // Four independent accumulation chains (entry half x even/odd k-step).
  f32x4 s2[2][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) s2[nt][0] = s2[nt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  // B operand: entry 16nt + col, dims 32ks + 8g .. +7.
  const uint8_t* kbase = kimg + col * SM::kKRowB + (BF16 ? 16 : 8) * g;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const uint8_t* src = kbase + 16 * nt * SM::kKRowB + (BF16 ? 64 : 32) * ks;
      bf16x8 kb;
      if constexpr (BF16) kb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(src));
      else kb = fp8x8_bf16(*reinterpret_cast<const uint2*>(src));
      s2[nt][ks & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], kb, s2[nt][ks & 1], 0, 0, 0);
    }
  }
  const f32x4 s[2] = {s2[0][0] + s2[0][1], s2[1][0] + s2[1][1]};
  // lane owns heads 4g+i, entries 16nt+col
  const bool ok0 = sm.slot[tb + col] >= 0, ok1 = sm.slot[tb + 16 + col] >= 0;
  const float ks0 = sm.kscale[tb + col], ks1 = sm.kscale[tb + 16 + col];
  float x[2][4], mx[4];
  bool grow = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[0][i] = ok0 ? s[0][i] * (sc2 * ks0) : -INFINITY;
    x[1][i] = ok1 ? s[1][i] * (sc2 * ks1) : -INFINITY;
    const float m = row16_max(fmaxf(x[0][i], x[1][i]));
    mx[i] = m;
    grow |= m > st.m2[i] + kRescaleSlack || (st.m2[i] == -INFINITY && m != -INFINITY);
  }
  const bool any = __any(grow);
  if (any) {  // wave-uniform: move every head's reference to its max so far
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mnew = fmaxf(st.m2[i], mx[i]);
      float al = 1.0f;
      if (mnew != -INFINITY) {
        al = (st.m2[i] == -INFINITY) ? 0.0f : exp2f(st.m2[i] - mnew);
        st.lsum[i] *= al;
        st.m2[i] = mnew;
      }
      if (col == 0) sm.alpha[pb][16 * wave + 4 * g + i] = al;
    }
  }
  if (lane == 0) sm.grow[pb][wave] = any ? 1 : 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool live = st.m2[i] != -INFINITY;
    const float p0 = live ? exp2f(x[0][i] - st.m2[i]) : 0.0f;
    const float p1 = live ? exp2f(x[1][i] - st.m2[i]) : 0.0f;
    st.lsum[i] += p0 + p1;
    uint16_t* prow = &sm.p[pb][(16 * wave + 4 * g + i) * SM::kPRow];
    const uint32_t pk = bf16x2_bits(p0 * ks0, p1 * ks1);
    prow[col] = static_cast<uint16_t>(pk & 0xffffu);
    prow[16 + col] = static_cast<uint16_t>(pk >> 16);
  }
}

// ---------------------------------------------------------------------------
template <int D, bool BF16>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
sparse_decode_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  using SM = DecodeSmem<D, BF16>;
  SM& sm = *reinterpret_cast<SM*>(smem_raw);
  auto kimg = [&](int i) -> uint8_t* { return sm.img + i * SM::kImgB; };
  constexpr int KS = D / 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int t = blockIdx.y, split = blockIdx.x;
  const int hgroups = a.heads / 16;
  const bool scorer = wave < kScoreWaves;

  // q operands of the score waves (A of S = Q K^T): head 16w + col, dims 32ks + 8g .. +8
  bf16x8 qa[KS];
  if (scorer && wave < hgroups) {
    const uint16_t* qrow = a.q + static_cast<int64_t>(t) * a.q_tok_stride + (16 * wave + col) * a.q_head_stride;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qa[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g));
  }

  // Prologue: entries -> slots, two dependent gathers (index, block table;
  // one without a block table) each issued for all of the thread's entries
  // first.  The rows' scales come with the rows.
  int len = a.width;
  if (a.lengths) len = min(max(a.lengths[t], 0), a.width);
  const int e_begin = split * a.per_split;
  const int e_cnt = max(0, min(e_begin + a.per_split, len) - e_begin);
  const int ntiles = (e_cnt + kTile - 1) / kTile;
  const int e_pad = ntiles * kTile;
  // Steps of the main loop: step s finishes tile s-1 and scores tile s, so
  // ntiles + 1 steps, rounded up to even (the data waves take steps in pairs).
  const int steps = (ntiles + 2) & ~1;
  constexpr int kPrologue = kMaxSplitEntries / kThreads;
  int64_t sv[kPrologue];
#pragma unroll
  for (int j = 0; j < kPrologue; ++j) {
    const int e = tid + kThreads * j;
    sv[j] = (e < e_cnt) ? a.indices[static_cast<int64_t>(t) * a.idx_stride + e_begin + e] : -1;
  }
  if (a.block_table != nullptr) {
    const int32_t* bt = a.block_table + static_cast<int64_t>(a.req_ids[t]) * a.bt_stride;
#pragma unroll
    for (int j = 0; j < kPrologue; ++j) {
      const int64_t idx = sv[j];
      const bool ok = idx >= 0 && (idx >> 6) < a.bt_stride;
      const int64_t page = bt[ok ? (idx >> 6) : 0];
      sv[j] = ok ? page * kPageTokens + (idx & 63) : -1;
    }
  }
#pragma unroll
  for (int j = 0; j < kPrologue; ++j) {
    const int e = tid + kThreads * j;
    const int64_t slot = (sv[j] >= 0 && sv[j] < a.num_rows) ? sv[j] : -1;
    if (e < e_pad) sm.slot[e] = static_cast<int32_t>(slot);
  }
  if (tid < 2 * kScoreWaves) sm.grow[tid / kScoreWaves][tid % kScoreWaves] = 0;
  __syncthreads();

  f32x4 o[4][4];
#pragma unroll
  for (int hf = 0; hf < 4; ++hf)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) o[hf][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (!scorer) {
    // ---------------- data waves ----------------
    const int u = wave - kScoreWaves;
    RowRegs<D, BF16> bufA, bufB;  // even tiles in A, odd tiles in B
    fetch_rows<D, BF16>(a, sm, u, 0, ntiles, bufA);
    fetch_rows<D, BF16>(a, sm, u, 1, ntiles, bufB);
    store_rows<D, BF16>(bufA, u, 0, sm, kimg(0));
    fetch_rows<D, BF16>(a, sm, u, 2, ntiles, bufA);
    __syncthreads();  // tile 0 stored
    // Step s finishes tile s-1 (P V from image (s-1) % 3), stores tile s+1 into
    // image (s+1) % 3 and issues the loads of tile s+3.  Every load and
    // store is unconditional (tiles past the end are zero rows nobody
    // reads), so each wait leaves the newer tile in flight.
    store_rows<D, BF16>(bufB, u, 1, sm, kimg(1));  // step 0
    fetch_rows<D, BF16>(a, sm, u, 3, ntiles, bufB);
    __syncthreads();
    int s = 1, kp = 0;  // kp: image of tile s-1
    for (; s + 1 <= ntiles; s += 2) {
      const int k1 = (kp == 2) ? 0 : kp + 1, k2 = (k1 == 2) ? 0 : k1 + 1;
      accumulate_pv<D, BF16>(sm, kimg(kp), (s - 1) & 1, hgroups, o);
      store_rows<D, BF16>(bufA, u, s + 1, sm, kimg(k2));
      fetch_rows<D, BF16>(a, sm, u, s + 3, ntiles, bufA);
      __syncthreads();
      accumulate_pv<D, BF16>(sm, kimg(k1), s & 1, hgroups, o);
      store_rows<D, BF16>(bufB, u, s + 2, sm, kimg(kp));
      fetch_rows<D, BF16>(a, sm, u, s + 4, ntiles, bufB);
      __syncthreads();
      kp = k2;
    }
    // the last (odd) step
    if (s - 1 < ntiles) accumulate_pv<D, BF16>(sm, kimg(kp), (s - 1) & 1, hgroups, o);
    __syncthreads();
  } else {
    // ---------------- score waves ----------------
    SoftmaxState st;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st.m2[i] = -INFINITY;
      st.lsum[i] = 0.0f;
    }
    const float sc2 = a.scale * kLog2e;
    __syncthreads();  // tile 0 stored
    // Step s finishes tile s-1 and scores tile s (image s % 3, P buffer s & 1).
    // Score waves past `hgroups` run on unused heads rather than branching.
    if (ntiles == 0) {
      for (int s = 0; s < steps; ++s) __syncthreads();
    } else {
      score_tile<D, BF16>(sm, kimg(0), 0, 0, sc2, qa, st);
      __syncthreads();
      int kp = 0;  // image of tile s-1
      for (int s = 1; s < ntiles; ++s) {
        const int kr = (kp == 2) ? 0 : kp + 1;
        accumulate_pv<D, BF16>(sm, kimg(kp), (s - 1) & 1, hgroups, o);
        score_tile<D, BF16>(sm, kimg(kr), s & 1, s * kTile, sc2, qa, st);
        __syncthreads();
        kp = kr;
      }
      accumulate_pv<D, BF16>(sm, kimg(kp), (ntiles - 1) & 1, hgroups, o);
      __syncthreads();
      for (int s = ntiles + 1; s < steps; ++s) __syncthreads();
    }
    // final denominators and maxima of this wave's heads
    if (wave < hgroups) {
      const int64_t base = (static_cast<int64_t>(t) * a.splits + split) * a.heads;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float l = row16_sum(st.lsum[i]);
        if (col == 0) {
          const int h = 16 * wave + 4 * g + i;
          sm.row_l[h] = l;
          a.ws_ml[(base + h) * 2 + 0] = st.m2[i];
          a.ws_ml[(base + h) * 2 + 1] = l;
        }
      }
    }
  }
  __syncthreads();

  // Epilogue: O / l of the split in fp32 (the combine sums the splits'
  // partials, which may cancel, so they keep fp32 precision): each store
  // instruction writes 16 consecutive channels (64 bytes) of one head.
  const int64_t base = (static_cast<int64_t>(t) * a.splits + split) * a.heads;
#pragma unroll
  for (int hf = 0; hf < 4; ++hf) {
    if (hf >= hgroups) break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 16 * hf + 4 * g + i;
      const float l = sm.row_l[h];
      const float inv = (l > 0.0f) ? 1.0f / l : 0.0f;
      float* orow = a.ws_o + (base + h) * kDv + 64 * wave + col;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) orow[16 * nt] = o[hf][nt][i] * inv;
    }
  }
}

// 256 threads per (t, 4 heads): wave = head, lane = 8 output channels.
__global__ void __launch_bounds__(256) decode_combine_kernel(
    const float* ws_o, const float* ws_ml, int32_t splits, int32_t heads, const float* sinks,
    uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride, float* lse, int64_t lse_stride) {
  const int t = blockIdx.y;
  const int h = 4 * blockIdx.x + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (h >= heads) return;
  const int64_t b0 = static_cast<int64_t>(t) * splits * heads + h;
  // Splits in batches of 8 with every load of a batch issued before any is
  // used; a running max rescales the partial sums between batches.
  constexpr int kBatch = 8;
  float M = -INFINITY, L = 0.0f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += kBatch) {
    float ms[kBatch], ls[kBatch];
    float4 v[kBatch][2];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const bool ok = s0 + b < splits;
      const int64_t row = b0 + static_cast<int64_t>(ok ? s0 + b : s0) * heads;
      const float2 ml = *reinterpret_cast<const float2*>(ws_ml + row * 2);
      ms[b] = ok ? ml.x : -INFINITY;
      ls[b] = ml.y;
      v[b][0] = *reinterpret_cast<const float4*>(ws_o + row * kDv + 8 * lane);
      v[b][1] = *reinterpret_cast<const float4*>(ws_o + row * kDv + 8 * lane + 4);
    }
    float mb = M;
#pragma unroll
    for (int b = 0; b < kBatch; ++b) mb = fmaxf(mb, ms[b]);
    if (mb == -INFINITY) continue;
    if (M != mb) {
      const float sc = (M == -INFINITY) ? 0.0f : exp2f(M - mb);
      L *= sc;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= sc;
      M = mb;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (ms[b] == -INFINITY) continue;
      const float f = exp2f(ms[b] - M) * ls[b];
      L += f;
      const float x[8] = {v[b][0].x, v[b][0].y, v[b][0].z, v[b][0].w, v[b][1].x, v[b][1].y, v[b][1].z, v[b][1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += x[i] * f;
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
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(f32_to_bf16(acc[2 * i] * inv)) |
           (static_cast<uint32_t>(f32_to_bf16(acc[2 * i + 1] * inv)) << 16);
  uint16_t* orow = out + static_cast<int64_t>(t) * out_tok_stride + h * out_head_stride;
  *reinterpret_cast<uint4*>(orow + 8 * lane) = make_uint4(w[0], w[1], w[2], w[3]);
  if (lane == 0 && lse != nullptr)
    lse[static_cast<int64_t>(t) * lse_stride + h] = (L > 0.0f) ? (M + log2f(L)) * kLn2 : -INFINITY;
}

}  // namespace ekv

using namespace ekv;

static int decode_splits(int32_t num_tokens, int32_t width) {
  const int tiles = (width + kTile - 1) / kTile;
  int splits = (kTargetGroups + num_tokens - 1) / (num_tokens > 0 ? num_tokens : 1);
  const int need = (width + kMaxSplitEntries - 1) / kMaxSplitEntries;
  if (splits < need) splits = need;
  if (splits > tiles) splits = tiles;
  if (splits < 1) splits = 1;
  return splits;
}

extern "C" int64_t ekv_sparse_mla_decode_workspace_size(int32_t num_tokens, int32_t heads, int32_t width) {
  if (num_tokens <= 0 || heads <= 0) return 0;
  const int64_t n = static_cast<int64_t>(num_tokens) * decode_splits(num_tokens, width) * heads;
  return n * kDv * 4 + n * 2 * 4 + 256;
}

template <int D, bool BF16>
static void launch_decode(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  const size_t smem = sizeof(DecodeSmem<D, BF16>);
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(sparse_decode_kernel<D, BF16>),
                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  hipLaunchKernelGGL((sparse_decode_kernel<D, BF16>), grid, dim3(kThreads), smem, s, a);
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
  EKV_CHECK(heads > 0 && heads % 16 == 0 && heads <= 16 * kScoreWaves, "heads must be a multiple of 16, <= 64");
  EKV_CHECK(q && cache && indices && out, "null pointer");
  EKV_CHECK(block_table == nullptr || req_ids != nullptr, "block_table needs req_ids");
  EKV_CHECK(q_tok_stride % 8 == 0 && q_head_stride % 8 == 0 && aligned16(q), "q must be 16-byte aligned rows");
  EKV_CHECK(out_tok_stride % 8 == 0 && out_head_stride % 8 == 0 && aligned16(out),
            "out rows must be 16-byte aligned");
  EKV_CHECK(cache_bf16 || (page_stride >= kPageTokens * (dim + 4) && page_stride % 16 == 0), "bad page_stride");
  EKV_CHECK(aligned16(cache), "cache must be 16-byte aligned");
  EKV_CHECK(num_pages >= 1 && num_pages * kPageTokens < (int64_t{1} << 31), "cache must hold 1 .. 2**31 / 64 pages");
  const int64_t need = ekv_sparse_mla_decode_workspace_size(num_tokens, heads, width);
  EKV_CHECK(workspace != nullptr, "workspace is null");
  EKV_CHECK(aligned16(workspace), "workspace must be 16-byte aligned");
  if (workspace_bytes < need) {
    set_error("workspace too small (see ekv_sparse_mla_decode_workspace_size)");
    return kWorkspaceTooSmall;
  }
  const int splits = decode_splits(num_tokens, width);
  const int tiles = (width + kTile - 1) / kTile;
  const int per_split = ((tiles + splits - 1) / splits) * kTile;
  float* ws_o = static_cast<float*>(workspace);
  float* ws_ml = ws_o + static_cast<int64_t>(num_tokens) * splits * heads * kDv;
  DecodeArgs a{q, q_tok_stride, q_head_stride, cache, page_stride, num_pages * kPageTokens, indices, idx_stride,
               width, lengths, block_table, bt_stride, req_ids, scale, heads, per_split, ws_o, ws_ml, splits};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(splits, num_tokens);
  if (dim == 576) {
    if (cache_bf16) launch_decode<576, true>(a, grid, s);
    else launch_decode<576, false>(a, grid, s);
  } else {
    if (cache_bf16) launch_decode<512, true>(a, grid, s);
    else launch_decode<512, false>(a, grid, s);
  }
  int rc = ekv_launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(heads / 4, num_tokens), dim3(256), 0, s, ws_o, ws_ml, splits,
                     heads, sinks, out, out_tok_stride, out_head_stride, lse, lse_stride);
  return ekv_launch_status();
}
