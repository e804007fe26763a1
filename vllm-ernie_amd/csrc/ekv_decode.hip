// Sparse MLA decode over gathered latent rows (DSA top-k + window, HCA
// compressed + window), with the per-head attention sink in the softmax
// denominator.
//
// Workgroup = (query row t, split s of its index row), 512 threads in two
// roles, one barrier per tile of 32 index entries.  Between two barriers:
//   * score waves 0..3 (q for heads 16w .. 16w+15 held in registers) first
//     finish tile t-1 (below), then compute S = Q K^T of tile t on
//     v_mfma_f32_16x16x32_bf16 from a bf16 K image in LDS, run the online
//     softmax and write P (row scale folded in) for their heads as a pair of
//     bf16 values hi = bf16(P), lo = bf16(P - hi); fp8 K fragments become
//     bf16 in registers (exact conversion);
//   * data waves 4..7 finish tile t-1, store tile t+1 (the rows as cached:
//     e4m3fn bytes, or bf16) into the next of three K images, and issue the
//     loads of tile t+3 (8 rows per wave, row addresses in scalar registers,
//     256-byte coalesced loads into registers, two tiles in flight);
//   * "finish tile t-1" = O[:, 64w .. 64w+63] += P_hi V + P_lo V for all
//     heads, every wave taking its 64 channels.  The B operand (V, entries x
//     channels) is read straight from the row-major K image with a
//     transposing LDS read (ds_read_b64_tr_b8 for fp8 rows, ds_read_b64_tr_b16
//     for bf16); no separate V^T image is built.
// The hi/lo pair carries P to about 2^-16 relative (one bf16 alone is 2^-8,
// which rows of a few entries that nearly cancel expose); V itself is exact
// in bf16 for fp8 and bf16 caches.
// A prologue resolves every index entry of the split to a cache slot (block
// table lookup) and fp32 row scale once.  The softmax reference max only
// moves when a score exceeds it by more than 8 (log2 units), so O is rescaled
// rarely.  Each split leaves O / l in fp32 plus (m, l) in fp32; the combine
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
constexpr int kMaxSplitTiles = kMaxSplitEntries / kTile;
constexpr int kTargetGroups = 256;           // one workgroup per CU
constexpr int kXcds = 8;                     // workgroup b runs on XCD b % 8
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
  int32_t rows;             // T
  int32_t groups;           // G workgroups (a multiple of 8), >= T + T * tiles(width) / 32
  float* ws_o;              // [G, H, 512] fp32, O / l of workgroup g's split
  float* ws_ml;             // [G, H, 2] (m in log2 units, l)
  int2* ws_rows;            // [T] (first workgroup, splits) of each row
  const float* sinks;       // [H] or null
  uint16_t* out;            // [T, H, 512] bf16
  int64_t out_tok_stride, out_head_stride;
  float* lse;               // [T, H] or null
  int64_t lse_stride;
};

// Work split.  Row t has tiles_t = ceil(len_t / 32) tiles and gets
//   splits_t = max(1, min(tiles_t, 1 + floor((G - T) * tiles_t / total_tiles)))
// workgroups (sum <= G), taking equal runs of its tiles: splits follow the
// entries, so a long row gets proportionally more workgroups.  Since
// G - T >= total_tiles / 32, every split holds at most 32 tiles
// (kMaxSplitEntries entries).  Row t's splits are the logical workgroups
// first_t .. first_t + splits_t - 1 (first_t = sum of the splits before it).
__device__ __forceinline__ int row_len(const DecodeArgs& a, int t) {
  return a.lengths ? min(max(a.lengths[t], 0), a.width) : a.width;
}
__device__ __forceinline__ int row_splits(int64_t extra, int tiles, int64_t total) {
  const int ns = 1 + (total > 0 ? static_cast<int>((extra * tiles) / total) : 0);
  return max(1, min(tiles, ns));  // never more splits than tiles
}

// Finds the row and split of logical workgroup l; t = -1 when l is past the
// last split.  All threads of the workgroup call it.
template <int kN>
__device__ void locate_split(const DecodeArgs& a, int l, int* s_red, int& t, int& split, int& nsplit, int& first) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kW = kN / 64;
  const int T = a.rows;
  const int64_t extra = a.groups - T;
  if (a.lengths == nullptr) {  // every row has `width` entries: closed form
    const int tiles = (a.width + kTile - 1) / kTile;
    const int ns = row_splits(extra, tiles, static_cast<int64_t>(T) * tiles);
    t = (l / ns < T) ? l / ns : -1;
    split = l % ns;
    nsplit = ns;
    first = l - split;
    return;
  }
  // total tiles
  int64_t sum = 0;
  for (int r = tid; r < T; r += kN) sum += (row_len(a, r) + kTile - 1) / kTile;
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (lane == 0) reinterpret_cast<int64_t*>(s_red)[wave] = sum;
  __syncthreads();
  int64_t total = 0;
#pragma unroll
  for (int w = 0; w < kW; ++w) total += reinterpret_cast<int64_t*>(s_red)[w];
  __syncthreads();
  // splits of a contiguous run of rows per thread, scanned across the block
  const int per = (T + kN - 1) / kN;
  const int r0 = min(tid * per, T), r1 = min(r0 + per, T);
  int cnt = 0;
  for (int r = r0; r < r1; ++r) cnt += row_splits(extra, (row_len(a, r) + kTile - 1) / kTile, total);
  int x = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_red[2 * kW + wave] = x;
  if (tid == 0) s_red[3 * kW] = -1;
  __syncthreads();
  int before = 0;
#pragma unroll
  for (int w = 0; w < kW; ++w) before += (w < wave) ? s_red[2 * kW + w] : 0;
  int pos = before + x - cnt;  // logical workgroups before row r0
  if (pos <= l && l < pos + cnt) {
    for (int r = r0; r < r1; ++r) {
      const int ns = row_splits(extra, (row_len(a, r) + kTile - 1) / kTile, total);
      if (l < pos + ns) {
        s_red[3 * kW] = r;
        s_red[3 * kW + 1] = l - pos;
        s_red[3 * kW + 2] = ns;
        break;
      }
      pos += ns;
    }
  }
  __syncthreads();
  t = s_red[3 * kW];
  split = s_red[3 * kW + 1];
  nsplit = s_red[3 * kW + 2];
  first = l - split;
  __syncthreads();
}

// K images hold the tile's rows as stored: raw e4m3fn bytes (fp8 cache) or
// bf16.  The fp8 row stride D + 8 bytes is 8 (mod 16) words: the 16 rows a
// QK fragment read touches land on distinct bank pairs.
template <int D, bool BF16>
struct DecodeSmem {
  static constexpr int kKRowB = BF16 ? 2 * (D + 8) : D + 8;  // K row stride (bytes)
  static constexpr int kImgB = kTile * kKRowB;
  static constexpr int kPRow = kTile + 8;   // bf16 P row stride (elements)
  __align__(16) uint8_t img[kKImages * kImgB];
  uint16_t p[2][64 * kPRow];                // bf16(P) of tiles t (written) and t-1 (read)
  uint16_t plo[2][64 * kPRow];              // bf16(P - bf16(P)), same layout
  float alpha[2][64];                       // rescale factor per head (valid when grow[.][head / 16])
  int32_t grow[2][kScoreWaves];
  float row_f[64];                          // epilogue: per-head output factor
  __align__(8) int32_t red[64];             // split location scratch
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
  // the lo parts one head group ahead of their products (register pressure)
  auto p_lo = [&](int hf) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&sm.plo[pb][(16 * hf + col) * SM::kPRow + 8 * g]));
  };
  bf16x8 pl = p_lo(0);
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
  for (int hf = 0; hf < 4; ++hf) {
    const bf16x8 pl_next = p_lo(hf < 3 ? hf + 1 : 3);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      o[hf][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, vb[nt], o[hf][nt], 0, 0, 0);
      o[hf][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[hf], vb[nt], o[hf][nt], 0, 0, 0);
    }
    pl = pl_next;
  }
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
    const int prow = (16 * wave + 4 * g + i) * SM::kPRow;
    const float w0 = p0 * ks0, w1 = p1 * ks1;
    const uint32_t pk = bf16x2_bits(w0, w1);
    const float h0 = __uint_as_float(pk << 16), h1 = __uint_as_float(pk & 0xffff0000u);
    const uint32_t pl = bf16x2_bits(w0 - h0, w1 - h1);  // exact differences
    sm.p[pb][prow + col] = static_cast<uint16_t>(pk & 0xffffu);
    sm.p[pb][prow + 16 + col] = static_cast<uint16_t>(pk >> 16);
    sm.plo[pb][prow + col] = static_cast<uint16_t>(pl & 0xffffu);
    sm.plo[pb][prow + 16 + col] = static_cast<uint16_t>(pl >> 16);
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
  const int hgroups = a.heads / 16;
  const bool scorer = wave < kScoreWaves;
  // Logical workgroup: consecutive ids share an XCD (hardware workgroup b
  // runs on XCD b % 8), so a row's splits read its q through one L2.
  const int b = blockIdx.x;
  const int l = (b % kXcds) * (a.groups / kXcds) + b / kXcds;
  int t, split, nsplit, first;
  locate_split<kThreads>(a, l, sm.red, t, split, nsplit, first);
  if (t < 0) return;
  if (split == 0 && tid == 0) a.ws_rows[t] = make_int2(first, nsplit);

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
  const int len = row_len(a, t);
  const int per_split = ((len + kTile - 1) / kTile + nsplit - 1) / nsplit * kTile;
  const int e_begin = split * per_split;
  const int e_cnt = max(0, min(e_begin + per_split, len) - e_begin);
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
    // final denominators and maxima of this wave's heads: a row of one split
    // is finished here (sink, lse), otherwise its partial goes to the combine
    if (wave < hgroups) {
      const int64_t base = static_cast<int64_t>(l) * a.heads;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lsum = row16_sum(st.lsum[i]);
        if (col == 0) {
          const int h = 16 * wave + 4 * g + i;
          const float m = st.m2[i];
          if (nsplit == 1) {
            float den = lsum, numf = 1.0f;
            if (a.sinks != nullptr) {
              const float sk = a.sinks[h] * kLog2e;
              const float mp = fmaxf(m, sk);
              if (mp != -INFINITY) {
                numf = (m == -INFINITY) ? 0.0f : exp2f(m - mp);
                den = lsum * numf + exp2f(sk - mp);
              }
            }
            sm.row_f[h] = (den > 0.0f) ? numf / den : 0.0f;
            if (a.lse != nullptr)
              a.lse[static_cast<int64_t>(t) * a.lse_stride + h] = (lsum > 0.0f) ? (m + log2f(lsum)) * kLn2 : -INFINITY;
          } else {
            sm.row_f[h] = (lsum > 0.0f) ? 1.0f / lsum : 0.0f;
            a.ws_ml[(base + h) * 2 + 0] = m;
            a.ws_ml[(base + h) * 2 + 1] = lsum;
          }
        }
      }
    }
  }
  __syncthreads();

  if (nsplit == 1) {
    // the finished row in bf16: 16 consecutive channels (32 bytes) of one head
    // per store instruction
#pragma unroll
    for (int hf = 0; hf < 4; ++hf) {
      if (hf >= hgroups) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 16 * hf + 4 * g + i;
        const float f = sm.row_f[h];
        uint16_t* orow = a.out + static_cast<int64_t>(t) * a.out_tok_stride + h * a.out_head_stride + 64 * wave + col;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) orow[16 * nt] = f32_to_bf16(o[hf][nt][i] * f);
      }
    }
    return;
  }
  // O / l of the split in fp32 (the combine sums the splits' partials, which
  // may cancel, so they keep fp32 precision): each store instruction writes
  // 16 consecutive channels (64 bytes) of one head.
  const int64_t base = static_cast<int64_t>(l) * a.heads;
#pragma unroll
  for (int hf = 0; hf < 4; ++hf) {
    if (hf >= hgroups) break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 16 * hf + 4 * g + i;
      const float inv = sm.row_f[h];
      float* orow = a.ws_o + (base + h) * kDv + 64 * wave + col;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) orow[16 * nt] = o[hf][nt][i] * inv;
    }
  }
}

// 256 threads per (t, 4 heads): wave = head, lane = 8 output channels.  Rows
// finished by their only split are skipped.
__global__ void __launch_bounds__(256) decode_combine_kernel(
    const float* ws_o, const float* ws_ml, const int2* ws_rows, int32_t heads, const float* sinks,
    uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride, float* lse, int64_t lse_stride) {
  const int t = blockIdx.y;
  const int h = 4 * blockIdx.x + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int2 rs = ws_rows[t];
  const int splits = rs.y;
  if (h >= heads || splits <= 1) return;
  const int64_t b0 = static_cast<int64_t>(rs.x) * heads + h;
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

// Workgroups of a call: at least one per CU, and enough that every split
// holds at most kMaxSplitTiles tiles (G - T >= T * tiles(width) / 32 bounds
// total_tiles / 32); a multiple of the XCD count.  Monotone in T and width,
// so a workspace sized for (T, H, width) serves every smaller call.
static int64_t decode_groups(int32_t num_tokens, int32_t width) {
  const int64_t tiles = (static_cast<int64_t>(width) + kTile - 1) / kTile;
  int64_t g = num_tokens + (num_tokens * tiles + kMaxSplitTiles - 1) / kMaxSplitTiles;
  if (g < kTargetGroups) g = kTargetGroups;
  return (g + kXcds - 1) / kXcds * kXcds;
}

extern "C" int64_t ekv_sparse_mla_decode_workspace_size(int32_t num_tokens, int32_t heads, int32_t width) {
  if (num_tokens <= 0 || heads <= 0 || width < 0) return 0;
  const int64_t n = decode_groups(num_tokens, width) * heads;
  return n * kDv * 4 + n * 2 * 4 + static_cast<int64_t>(num_tokens) * 8 + 256;
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
  const int64_t groups = decode_groups(num_tokens, width);
  EKV_CHECK(groups < (int64_t{1} << 31), "too many decode workgroups");
  float* ws_o = static_cast<float*>(workspace);
  float* ws_ml = ws_o + groups * heads * kDv;
  int2* ws_rows = reinterpret_cast<int2*>(ws_ml + groups * heads * 2);
  DecodeArgs a{q, q_tok_stride, q_head_stride, cache, page_stride, num_pages * kPageTokens, indices, idx_stride,
               width, lengths, block_table, bt_stride, req_ids, scale, heads, num_tokens,
               static_cast<int32_t>(groups), ws_o, ws_ml, ws_rows, sinks, out, out_tok_stride, out_head_stride,
               lse, lse_stride};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(groups));
  if (dim == 576) {
    if (cache_bf16) launch_decode<576, true>(a, grid, s);
    else launch_decode<576, false>(a, grid, s);
  } else {
    if (cache_bf16) launch_decode<512, true>(a, grid, s);
    else launch_decode<512, false>(a, grid, s);
  }
  int rc = ekv_launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(heads / 4, num_tokens), dim3(256), 0, s, ws_o, ws_ml, ws_rows,
                     heads, sinks, out, out_tok_stride, out_head_stride, lse, lse_stride);
  return ekv_launch_status();
}
