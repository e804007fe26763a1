// Sparse MLA decode over gathered latent rows (DSA top-k + window, HCA
// compressed + window), with the per-head attention sink in the softmax
// denominator.
//
// Workgroup = (query row t, split s of its index row): 8 waves, a scorer and
// a data wave per group of 16 heads, the two waves of a group on one SIMD
// (wave w and w + 4).  The split's entries go through in tiles of 32, one
// barrier per tile.  At step s:
//   * the scorer wave of a group computes S^T = K Q^T for tile s
//     (v_mfma_f32_16x16x32_bf16, A = the tile's rows from LDS, fp8 converted
//     exactly to bf16, B = its 16 heads of q held in registers), runs the
//     online softmax (a lane holds one head's scores of 8 entries; the
//     reference max only moves when a score exceeds it by more than 8 log2
//     units), turns the weights P (row scale folded in) into a pair of bf16
//     B operands hi = bf16(P), lo = bf16(P - hi), publishes them for the data
//     wave and accumulates O^T[0, 256) += V^T P^T of tile s;
//   * the data wave of a group accumulates O^T[256, 512) += V^T P^T of tile
//     s - 1 from the published operands, and issues the direct global->LDS
//     loads of a later tile (coalesced 16-byte loads of whole rows).
// V^T (channels x entries) is read straight from the row-major tile image
// with transposing LDS reads (ds_read_b64_tr_b8 / _b16); S^T's accumulator
// layout is the B-operand layout of P^T, so P never leaves the registers of
// the wave that computed it except for the data wave's copy.  The hi/lo pair
// carries P to about 2^-16 relative (one bf16 alone is 2^-8, which rows of a
// few entries that nearly cancel expose); V is exact in bf16.
// A prologue resolves every index entry of the split to a cache slot (block
// table lookup) and loads the rows' fp32 scales once.  Each split leaves
// O / l in fp32 plus (m, l); the combine kernel merges the splits, adds the
// sink and writes bf16 out and the natural-log lse (log sum_j exp(s_j), sink
// excluded).  A row of one split is finished in place.
#include "ekv_common.h"
#include "ekv_internal.h"

#include <atomic>
#include <mutex>
#include <type_traits>

namespace ekv {

constexpr int kDv = 512;
constexpr int kTile = 32;
constexpr int kGroups = 4;                   // head groups of 16 (up to 64 heads)
constexpr int kThreads = 64 * 2 * kGroups;   // a scorer and a data wave per head group
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

// Finds the row, its length and the split of logical workgroup l; t = -1
// when l is past the last split.  All threads of the workgroup call it.
template <int kN>
__device__ void locate_split(const DecodeArgs& a, int l, int* s_red, int& t, int& len, int& split, int& nsplit,
                             int& first) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kW = kN / 64;
  const int T = a.rows;
  const int64_t extra = a.groups - T;
  if (a.lengths == nullptr) {  // every row has `width` entries: closed form
    const int tiles = (a.width + kTile - 1) / kTile;
    const int ns = row_splits(extra, tiles, static_cast<int64_t>(T) * tiles);
    t = (l / ns < T) ? l / ns : -1;
    len = a.width;
    split = l % ns;
    nsplit = ns;
    first = l - split;
    return;
  }
  // total tiles (with T <= kN thread r reads row r's length once, here)
  const int mylen = (T <= kN && tid < T) ? row_len(a, tid) : 0;
  const int mine = (mylen + kTile - 1) / kTile;
  int64_t sum = 0;
  if (T <= kN) sum = mine;
  else
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
  if (T <= kN) {
    if (r0 < r1) cnt = row_splits(extra, mine, total);  // r0 = tid
  } else {
    for (int r = r0; r < r1; ++r) cnt += row_splits(extra, (row_len(a, r) + kTile - 1) / kTile, total);
  }
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
      const int rl = T <= kN ? mylen : row_len(a, r);
      const int ns = T <= kN ? cnt : row_splits(extra, (rl + kTile - 1) / kTile, total);
      if (l < pos + ns) {
        s_red[3 * kW] = r;
        s_red[3 * kW + 1] = l - pos;
        s_red[3 * kW + 2] = ns;
        s_red[3 * kW + 3] = rl;
        break;
      }
      pos += ns;
    }
  }
  __syncthreads();
  t = s_red[3 * kW];
  len = s_red[3 * kW + 3];
  split = s_red[3 * kW + 1];
  nsplit = s_red[3 * kW + 2];
  first = l - split;
  __syncthreads();
}

// K tile images hold 32 rows as cached (e4m3fn bytes, or bf16), unpadded,
// with each row's 16-byte chunks permuted (chunk j of row r is stored at
// chunk swz(j, r), an XOR within runs of 8 chunks, of 4 for the last 4 of a
// 36-chunk row) so that the 16 rows a fragment read touches spread over the
// LDS banks.  For 576-byte rows (144 dwords, so rows 4 apart start on the
// same bank) the XOR value is parity(r & 6) | parity(r & 9) << 1 |
// parity(r & 16) << 2, which leaves both the QK fragment reads (rows
// 0..15 or 16..31 at one chunk) and the transposed P·V reads (rows
// 4 kg .. 4 kg + 3 and 16 + 4 kg .. at one chunk) free of bank conflicts.  Rows arrive by direct global->LDS loads: lane i of a load
// instruction writes bytes [16 i, 16 i + 16) of the instruction's 1 KB.
template <int D, bool BF16>
struct DecodeSmem {
  // Tile images: fp8 tiles are loaded two steps ahead into 4 images; bf16
  // tiles (twice the bytes) one step ahead into 3.
  static constexpr int kBufs = BF16 ? 3 : 4;
  static constexpr int kAhead = kBufs - 2;
  static constexpr int kRowB = BF16 ? 2 * D : D;     // row bytes
  static constexpr int kChunks = kRowB / 16;          // 16-byte chunks per row
  static constexpr int kImgB = kTile * kRowB;         // bytes of one tile image
  static constexpr int kLoads = kImgB / 1024;         // 1 KB load instructions per tile
  static constexpr int kLoadsPerWave = (kLoads + kGroups - 1) / kGroups;
  __align__(16) uint8_t img[kBufs][kImgB];
  __align__(16) uint8_t spill[1024];                  // target of the padding load instructions
  __align__(16) uint4 p[2][kGroups][2][64];           // P hi / lo B operands of a head group, per lane
  float alpha[2][kGroups][16];                        // O rescale factor per head (when grow)
  int32_t grow[2][kGroups];
  float fin[kGroups][16];                             // epilogue: per-head output factor
  __align__(8) int32_t red[64];                       // split location scratch
  int32_t slot[kMaxSplitEntries];
  __align__(16) float kscale[kMaxSplitEntries];       // row scale, 0 for masked entries
  __align__(8) int64_t roff[kMaxSplitEntries];        // byte offset of the entry's row in the cache (masked: 0)
};

template <int D, bool BF16>
__device__ __forceinline__ int swz_chunk(int j, int r) {
  using SM = DecodeSmem<D, BF16>;
  if constexpr (SM::kChunks % 8 == 0) {
    return j ^ (r & 7);
  } else {
    const int f = (__builtin_popcount(r & 6) & 1) | ((__builtin_popcount(r & 9) & 1) << 1) |
                  ((__builtin_popcount(r & 16) & 1) << 2);
    return j < 32 ? (j ^ f) : (32 + ((j - 32) ^ (f & 3)));
  }
}

// Byte offset in a tile image of bytes [8 h, 8 h + 8) of 16-byte chunk c of row r.
template <int D, bool BF16>
__device__ __forceinline__ int img_off(int r, int c, int h) {
  return r * DecodeSmem<D, BF16>::kRowB + 16 * swz_chunk<D, BF16>(c, r) + 8 * h;
}

// Four e4m3fn bytes -> four bf16 (exact: every e4m3fn value is a bf16 value).
__device__ __forceinline__ uint2 fp8x4_bf16(uint32_t w) {
  const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
  return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}
__device__ __forceinline__ bf16x8 fp8x8_bf16(uint2 w) {
  const uint2 lo = fp8x4_bf16(w.x), hi = fp8x4_bf16(w.y);
  return __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
}

__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};  // round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

// ds_read_b64_tr_b8: in each row of 16 lanes, lane j receives byte j % 8 of
// the 8 bytes addressed by lanes j / 8 + 2m (m = 0..7), as byte m.
typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 lds_read_tr8(const uint8_t* p) {
  const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
      (__attribute__((address_space(3))) i32x2*)((__attribute__((address_space(3))) uint8_t*)(p)));
  return make_uint2(static_cast<uint32_t>(v.x), static_cast<uint32_t>(v.y));
}
// ds_read_b64_tr_b16: lane j receives 16-bit element j % 4 of the 8 bytes
// addressed by lanes j / 4 + 4m (m = 0..3), as element m.
__device__ __forceinline__ i16x4 lds_read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)((__attribute__((address_space(3))) uint8_t*)(p)));
}

// Max of v over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows),
// with VALU lane swaps instead of LDS permutes: after a swap of rows r and
// r ^ 1 (or halves) between two copies of v, the max of the two results is
// the pairwise max in every lane.
__device__ __forceinline__ float max_rows(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t w = __float_as_uint(m);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// s_waitcnt vmcnt(N), other counters untouched.
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Data waves: wait until at most n tiles' loads (n < kAhead) are in flight.
template <int D, bool BF16>
__device__ __forceinline__ void wait_tiles(int n) {
  constexpr int L = DecodeSmem<D, BF16>::kLoadsPerWave;
  if (n <= 0) wait_vm<0>();
  else if (n == 1) wait_vm<L>();
  else wait_vm<2 * L>();
}

// Entry of k-slot m (0..7) of lane group kg in the S^T accumulators / the
// P V operands: S^T rows 4 kg + i of entry halves 0 and 1.
__device__ __forceinline__ int slot_entry(int kg, int m) { return m < 4 ? 4 * kg + m : 16 + 4 * kg + (m - 4); }

// ---------------------------------------------------------------------------
// Tile loads (data waves).  Instruction k of a tile covers image bytes
// [1024 k, 1024 k + 1024); lane i its 16-byte chunk 64 k + i, i.e. row
// (64 k + i) / kChunks, stored chunk j = (64 k + i) % kChunks, which holds
// row chunk swz(j, r).  Masked rows load the first cache row (their image
// rows are zeroed once the tile has landed).  Padding instructions (when the
// tile has fewer than kLoadsPerWave * 4) write the spill area.
// A data wave's share of every tile's loads, fixed for the kernel: load j is
// instruction k = j * kGroups + u, and this lane copies the tile's entry
// `row` from byte `col` of its cached row.
template <int D, bool BF16>
struct TileLanes {
  static constexpr int kN = DecodeSmem<D, BF16>::kLoadsPerWave;
  int row[kN], col[kN];
};

template <int D, bool BF16>
__device__ __forceinline__ TileLanes<D, BF16> tile_lanes(int u) {
  using SM = DecodeSmem<D, BF16>;
  const int lane = threadIdx.x & 63;
  TileLanes<D, BF16> tl;
#pragma unroll
  for (int j = 0; j < SM::kLoadsPerWave; ++j) {
    const int k = j * kGroups + u;
    const int pos = (k < SM::kLoads ? k : 0) * 64 + lane;
    const int r = pos / SM::kChunks, jj = pos % SM::kChunks;
    tl.row[j] = r;
    tl.col[j] = 16 * swz_chunk<D, BF16>(jj, r);
  }
  return tl;
}

// Byte offset of the cached row of a slot (-1: masked, read as row 0).
template <int D, bool BF16>
__device__ __forceinline__ int64_t row_offset(const DecodeArgs& a, int64_t s) {
  if (s < 0) return 0;
  if constexpr (BF16) return s * (2 * D);
  else return (s >> 6) * a.page_stride + (s & 63) * D;
}

template <int D, bool BF16>
__device__ __forceinline__ void issue_tile(const DecodeArgs& a, DecodeSmem<D, BF16>& sm, const TileLanes<D, BF16>& tl,
                                           int u, int tile) {
  using SM = DecodeSmem<D, BF16>;
  int64_t ro[SM::kLoadsPerWave];  // every row offset read issued before the first use
#pragma unroll
  for (int j = 0; j < SM::kLoadsPerWave; ++j) ro[j] = sm.roff[tile * kTile + tl.row[j]];
#pragma unroll
  for (int j = 0; j < SM::kLoadsPerWave; ++j) {
    const int k = j * kGroups + u;
    const uint8_t* src = a.cache + ro[j] + tl.col[j];
    uint8_t* dst = k < SM::kLoads ? sm.img[tile % SM::kBufs] + 1024 * k : sm.spill;
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
  }
}

// Zero the image rows of masked entries of a tile that has landed.
template <int D, bool BF16>
__device__ __forceinline__ void zero_masked(DecodeSmem<D, BF16>& sm, int u, int tile) {
  using SM = DecodeSmem<D, BF16>;
  const int lane = threadIdx.x & 63;
  const bool any = __any(lane < kTile && sm.slot[tile * kTile + lane] < 0);
  if (!any) return;
#pragma unroll
  for (int j = 0; j < SM::kLoadsPerWave; ++j) {
    const int k = j * kGroups + u;
    if (k >= SM::kLoads) break;
    const int pos = k * 64 + lane;
    if (sm.slot[tile * kTile + pos / SM::kChunks] < 0)
      *reinterpret_cast<uint4*>(sm.img[tile % SM::kBufs] + 16 * pos) = make_uint4(0, 0, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// O^T[16 cb + 4 kg + i][head col] += V^T P^T over the tile's 32 entries for
// the channel blocks [cb0, cb1): A = V^T from the image (transposing reads),
// B = the P hi / lo operands.
// This lane's V^T fragment of channel block cb (16 channels x the tile's 32
// entries), read transposed from the row-major image: 8 fp8 bytes (in .x,
// .y) or 8 bf16 values.
template <int D, bool BF16>
__device__ __forceinline__ uint4 pv_read(const uint8_t* img, int cb) {
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 4, col = lane & 15;
  if constexpr (BF16) {
    // element m of read h: row slot_entry(kg, 4h + col / 4), channel 16 cb + 4 (col % 4)
    const int ch = 16 * cb + 4 * (col & 3);
    const int r0 = slot_entry(kg, col >> 2), r1 = slot_entry(kg, 4 + (col >> 2));
    const i16x4 lo = lds_read_tr16(img + img_off<D, BF16>(r0, ch >> 3, (ch >> 2) & 1));
    const i16x4 hi = lds_read_tr16(img + img_off<D, BF16>(r1, ch >> 3, (ch >> 2) & 1));
    const i16x4 both[2] = {lo, hi};
    return __builtin_bit_cast(uint4, both);
  } else {
    // byte m: row slot_entry(kg, m) at channel 16 cb + (lane j of the row group)
    const int r = slot_entry(kg, col >> 1);
    const uint2 w = lds_read_tr8(img + img_off<D, BF16>(r, cb, col & 1));
    return make_uint4(w.x, w.y, 0u, 0u);
  }
}

template <bool BF16>
__device__ __forceinline__ bf16x8 pv_frag(const uint4& raw) {
  if constexpr (BF16) return __builtin_bit_cast(bf16x8, raw);
  else return fp8x8_bf16(make_uint2(raw.x, raw.y));
}

// O^T[16 cb .. ] += V^T P^T over channel blocks [kCb0, kCb1): the V^T
// fragments of a group of kPvGroup blocks are read while the previous group
// multiplies, and a group issues its lo products, then its hi products, so
// the two MFMAs into one accumulator are kPvGroup issues apart.
constexpr int kPvGroup = 4;

template <int D, bool BF16, int kCb0, int kCb1>
__device__ __forceinline__ void pv_tile(const uint8_t* img, const bf16x8& phi, const bf16x8& plo,
                                        f32x4 (&o)[kCb1 - kCb0]) {
  constexpr int kN = kCb1 - kCb0, kG = kPvGroup;
  static_assert(kN % kG == 0, "channel blocks must fill whole groups");
  uint4 raw[2][kG];
#pragma unroll
  for (int j = 0; j < kG; ++j) raw[0][j] = pv_read<D, BF16>(img, kCb0 + j);
#pragma unroll
  for (int g = 0; g < kN / kG; ++g) {
    if (g + 1 < kN / kG) {
#pragma unroll
      for (int j = 0; j < kG; ++j) raw[(g + 1) & 1][j] = pv_read<D, BF16>(img, kCb0 + (g + 1) * kG + j);
    }
    bf16x8 v[kG];
#pragma unroll
    for (int j = 0; j < kG; ++j) v[j] = pv_frag<BF16>(raw[g & 1][j]);
#pragma unroll
    for (int j = 0; j < kG; ++j)
      o[g * kG + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v[j], plo, o[g * kG + j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < kG; ++j)
      o[g * kG + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v[j], phi, o[g * kG + j], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Channels 16 cb + 4 kg .. +3 of head 16 grp + col (this lane's O^T
// values) times f: bf16 output of a row finished in place, else the split's
// fp32 partial.
template <bool kUnused>
__device__ __forceinline__ void store_o(const DecodeArgs& a, int t, int l, int nsplit, int grp, int cb, float f,
                                        const f32x4& v) {
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 4, col = lane & 15;
  const int h = 16 * grp + col;
  const int c0 = 16 * cb + 4 * kg;
  if (nsplit == 1) {
    uint16_t* o = a.out + static_cast<int64_t>(t) * a.out_tok_stride + h * a.out_head_stride + c0;
    *reinterpret_cast<uint2*>(o) = make_uint2(
        static_cast<uint32_t>(f32_to_bf16(v[0] * f)) | (static_cast<uint32_t>(f32_to_bf16(v[1] * f)) << 16),
        static_cast<uint32_t>(f32_to_bf16(v[2] * f)) | (static_cast<uint32_t>(f32_to_bf16(v[3] * f)) << 16));
  } else {
    float* o = a.ws_o + (static_cast<int64_t>(l) * a.heads + h) * kDv + c0;
    *reinterpret_cast<float4*>(o) = make_float4(v[0] * f, v[1] * f, v[2] * f, v[3] * f);
  }
}

// ---------------------------------------------------------------------------
template <int D, bool BF16>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
sparse_decode_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  using SM = DecodeSmem<D, BF16>;
  SM& sm = *reinterpret_cast<SM*>(smem_raw);
  constexpr int KS = D / 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = lane >> 4, col = lane & 15;
  const int hgroups = a.heads / 16;
  const bool scorer = wave < kGroups;
  const int grp = scorer ? wave : wave - kGroups;   // head group; waves w and w + 4 share SIMD w
  const bool active = grp < hgroups;

  const int b = blockIdx.x;
  const int l = (b % kXcds) * (a.groups / kXcds) + b / kXcds;

  // Prologue: entries -> slots (index, then block table), each gather issued
  // for all of the thread's entries before the next.  The entries of the
  // split this workgroup takes when every row has `width` entries (the
  // closed form) are requested before the row lengths are read; they are
  // kept when the lengths give the same row and entry range (uniform rows),
  // and requested again otherwise.
  constexpr int kPrologue = kMaxSplitEntries / kThreads;
  int64_t sv[kPrologue];
  auto split_range = [&](int row, int sp, int ns, int len, int& begin, int& cnt) {
    const int per = ((len + kTile - 1) / kTile + ns - 1) / ns * kTile;
    begin = sp * per;
    cnt = (row >= 0) ? max(0, min(begin + per, len) - begin) : 0;
  };
  auto load_entries = [&](int row, int begin, int cnt) {
#pragma unroll
    for (int j = 0; j < kPrologue; ++j) {
      const int e = tid + kThreads * j;
      sv[j] = (e < cnt) ? a.indices[static_cast<int64_t>(row) * a.idx_stride + begin + e] : -1;
    }
  };
  int g_t, g_begin, g_cnt;
  {
    const int tiles = (a.width + kTile - 1) / kTile;
    const int ns = row_splits(a.groups - a.rows, tiles, static_cast<int64_t>(a.rows) * tiles);
    g_t = (l / ns < a.rows) ? l / ns : -1;
    split_range(g_t, l % ns, ns, a.width, g_begin, g_cnt);
  }
  load_entries(g_t, g_begin, g_cnt);

  int t, len, split, nsplit, first;
  locate_split<kThreads>(a, l, sm.red, t, len, split, nsplit, first);
  if (t < 0) {
    wait_vm<0>();  // (the entries requested above)
    return;
  }
  if (split == 0 && tid == 0) a.ws_rows[t] = make_int2(first, nsplit);

  int e_begin, e_cnt;
  split_range(t, split, nsplit, len, e_begin, e_cnt);
  const int ntiles = (e_cnt + kTile - 1) / kTile;
  const int e_pad = ntiles * kTile;
  if (t != g_t || e_begin != g_begin || e_cnt != g_cnt) load_entries(t, e_begin, e_cnt);  // (workgroup-uniform)
  // The q operands (scorer waves) are requested once the entries are.
  bf16x8 qb[KS];  // B operand of S^T = K Q^T: head 16 grp + col, dims 32 ks + 8 kg .. +7
  if (scorer && active) {
    const uint16_t* qrow = a.q + static_cast<int64_t>(t) * a.q_tok_stride + (16 * grp + col) * a.q_head_stride;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qb[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * kg));
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
    if (e < e_pad) {
      sm.slot[e] = static_cast<int32_t>(slot);
      sm.roff[e] = row_offset<D, BF16>(a, slot);
    }
  }
  __syncthreads();
  // Data waves: the first kAhead tiles in flight (the only vector memory
  // operations they issue, so their load counter counts tiles).  Scorer
  // waves: the row scales.
  const TileLanes<D, BF16> tl = tile_lanes<D, BF16>(grp);
  if (!scorer) {
    for (int i = 0; i < SM::kAhead && i < ntiles; ++i) issue_tile<D, BF16>(a, sm, tl, grp, i);
    wait_tiles<D, BF16>(min(SM::kAhead, ntiles) - 1);  // tile 0 landed
    if (0 < ntiles) zero_masked<D, BF16>(sm, grp, 0);
  } else {
    constexpr int kPer = kMaxSplitEntries / (64 * kGroups);
    float ksv[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 64 * kGroups * j;
      const int s = (e < e_pad) ? sm.slot[e] : -1;
      if constexpr (BF16) ksv[j] = s >= 0 ? 1.0f : 0.0f;
      else ksv[j] = s >= 0 ? *reinterpret_cast<const float*>(a.cache + static_cast<int64_t>(s >> 6) * a.page_stride +
                                                              kPageTokens * D + (s & 63) * 4)
                           : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 64 * kGroups * j;
      if (e < e_pad) sm.kscale[e] = ksv[j];
    }
  }
  __syncthreads();

  // O^T accumulators: the scorer wave of a group holds channels [0, 256), the
  // data wave [256, 512) (an even split: the scorer's QK and softmax and the
  // data wave's tile loads take about the same time).  The two roles run
  // separate loops with the same barriers (one per step, ntiles + 1 steps).
  constexpr int kCbA = 16;
  constexpr int kChains = 4;  // QK accumulation chains per entry half
  if (scorer) {
    f32x4 oa[kCbA];
#pragma unroll
    for (int i = 0; i < kCbA; ++i) oa[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m2 = -INFINITY, lsum = 0.0f;  // reference max (log2 units) and this lane's share of l, head col
    const float sc2 = a.scale * kLog2e;
    for (int s = 0; s <= ntiles; ++s) {
      if (s < ntiles && active) {
        const uint8_t* img = sm.img[s % SM::kBufs];
        const int tb = s * kTile;
        // S^T = K Q^T for entries [16 nt, 16 nt + 16): eight accumulation
        // chains (an MFMA's result is ready ~4 issues later)
        f32x4 st[2][kChains];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int c = 0; c < kChains; ++c) st[nt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        // K fragments of entries col and 16 + col at K step ks, read kKPre
        // steps ahead of their MFMAs; the steps are issued in order so an
        // accumulator's consecutive MFMAs are 2 kChains issues apart
        constexpr int kKPre = BF16 ? 2 : 4;  // bf16 fragments take twice the registers
        uint4 kr[kKPre][BF16 ? 2 : 1];
        auto k_read = [&](int ks, uint4 (&dst)[BF16 ? 2 : 1]) {
          if constexpr (BF16) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
              dst[nt] = *reinterpret_cast<const uint4*>(img + img_off<D, BF16>(16 * nt + col, 4 * ks + kg, 0));
          } else {
            const uint2 a0 = *reinterpret_cast<const uint2*>(img + img_off<D, BF16>(col, 2 * ks + (kg >> 1), kg & 1));
            const uint2 a1 =
                *reinterpret_cast<const uint2*>(img + img_off<D, BF16>(16 + col, 2 * ks + (kg >> 1), kg & 1));
            dst[0] = make_uint4(a0.x, a0.y, a1.x, a1.y);
          }
        };
#pragma unroll
        for (int p = 0; p < kKPre; ++p) k_read(p, kr[p]);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          bf16x8 kf[2];
          if constexpr (BF16) {
            kf[0] = __builtin_bit_cast(bf16x8, kr[ks % kKPre][0]);
            kf[1] = __builtin_bit_cast(bf16x8, kr[ks % kKPre][1]);
          } else {
            kf[0] = fp8x8_bf16(make_uint2(kr[ks % kKPre][0].x, kr[ks % kKPre][0].y));
            kf[1] = fp8x8_bf16(make_uint2(kr[ks % kKPre][0].z, kr[ks % kKPre][0].w));
          }
          if (ks + kKPre < KS) k_read(ks + kKPre, kr[ks % kKPre]);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
            st[nt][ks % kChains] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[nt], qb[ks], st[nt][ks % kChains], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        // this lane: head col, entries slot_entry(kg, m)
        const float4 k0 = *reinterpret_cast<const float4*>(&sm.kscale[tb + 4 * kg]);
        const float4 k1 = *reinterpret_cast<const float4*>(&sm.kscale[tb + 16 + 4 * kg]);
        const float ks8[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        f32x4 s0 = st[0][0], s1 = st[1][0];
#pragma unroll
        for (int c = 1; c < kChains; ++c) {
          s0 += st[0][c];
          s1 += st[1][c];
        }
        const float sv8[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        float x[8];
        float mx = -INFINITY;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          x[m] = ks8[m] > 0.0f ? sv8[m] * (sc2 * ks8[m]) : -INFINITY;
          mx = fmaxf(mx, x[m]);
        }
        mx = max_rows(mx);
        const bool grow = mx > m2 + kRescaleSlack || (m2 == -INFINITY && mx != -INFINITY);
        const bool any = __any(grow);
        if (any) {  // wave-uniform: move every head's reference to its max so far
          const float mnew = fmaxf(m2, mx);
          float al = 1.0f;
          if (mnew != -INFINITY) {
            al = (m2 == -INFINITY) ? 0.0f : exp2f(m2 - mnew);
            lsum *= al;
            m2 = mnew;
          }
#pragma unroll
          for (int i = 0; i < kCbA; ++i) oa[i] *= al;
          if (kg == 0) sm.alpha[s & 1][grp][col] = al;
        }
        if (lane == 0) sm.grow[s & 1][grp] = any ? 1 : 0;
        const bool live = m2 != -INFINITY;
        float w[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const float p = live ? __builtin_amdgcn_exp2f(x[m] - m2) : 0.0f;  // (x - m2 <= 8; tiny weights flush to 0)
          lsum += p;
          w[m] = p * ks8[m];
        }
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          hi[m] = bf16x2_bits(w[2 * m], w[2 * m + 1]);
          const float h0 = __uint_as_float(hi[m] << 16), h1 = __uint_as_float(hi[m] & 0xffff0000u);
          lo[m] = bf16x2_bits(w[2 * m] - h0, w[2 * m + 1] - h1);  // exact differences
        }
        const uint4 phu = make_uint4(hi[0], hi[1], hi[2], hi[3]), plu = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        sm.p[s & 1][grp][0][lane] = phu;
        sm.p[s & 1][grp][1][lane] = plu;
        pv_tile<D, BF16, 0, kCbA>(img, __builtin_bit_cast(bf16x8, phu), __builtin_bit_cast(bf16x8, plu), oa);
      }
      __syncthreads();
    }
    // Epilogue: finish the heads' softmax (a row of one split gets the sink
    // and its lse here, otherwise (m, l) go to the combine), publish the
    // factor for the data wave, scale and store channels [0, 256).
    float f = 0.0f;
    if (active) {
      float lt = lsum + __shfl_xor(lsum, 16);
      lt += __shfl_xor(lt, 32);
      const int h = 16 * grp + col;
      if (nsplit == 1) {
        float den = lt, numf = 1.0f;
        if (a.sinks != nullptr) {
          const float sk = a.sinks[h] * kLog2e;
          const float mp = fmaxf(m2, sk);
          if (mp != -INFINITY) {
            numf = (m2 == -INFINITY) ? 0.0f : exp2f(m2 - mp);
            den = lt * numf + exp2f(sk - mp);
          }
        }
        f = (den > 0.0f) ? numf / den : 0.0f;
        if (kg == 0 && a.lse != nullptr)
          a.lse[static_cast<int64_t>(t) * a.lse_stride + h] = (lt > 0.0f) ? (m2 + log2f(lt)) * kLn2 : -INFINITY;
      } else {
        f = (lt > 0.0f) ? 1.0f / lt : 0.0f;
        if (kg == 0) {
          const int64_t row = static_cast<int64_t>(l) * a.heads + h;
          a.ws_ml[row * 2 + 0] = m2;
          a.ws_ml[row * 2 + 1] = lt;
        }
      }
      if (kg == 0) sm.fin[grp][col] = f;
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int i = 0; i < kCbA; ++i) store_o<false>(a, t, l, nsplit, grp, i, f, oa[i]);
    }
  } else {
    constexpr int kCbB = kDv / 16 - kCbA;
    f32x4 ob[kCbB];
#pragma unroll
    for (int i = 0; i < kCbB; ++i) ob[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s <= ntiles; ++s) {
      if (s + SM::kAhead < ntiles) issue_tile<D, BF16>(a, sm, tl, grp, s + SM::kAhead);
      if (s >= 1 && active) {
        const uint8_t* img = sm.img[(s - 1) % SM::kBufs];
        const int pb = (s - 1) & 1;
        if (sm.grow[pb][grp]) {
          const float al = sm.alpha[pb][grp][col];
#pragma unroll
          for (int i = 0; i < kCbB; ++i) ob[i] *= al;
        }
        const bf16x8 phi = __builtin_bit_cast(bf16x8, sm.p[pb][grp][0][lane]);
        const bf16x8 plo = __builtin_bit_cast(bf16x8, sm.p[pb][grp][1][lane]);
        pv_tile<D, BF16, kCbA, kDv / 16>(img, phi, plo, ob);
      }
      // tile s + 1 must have landed when the step ends; tiles s + 2 ..
      // s + kAhead may stay in flight
      wait_tiles<D, BF16>(min(ntiles - 1, s + SM::kAhead) - (s + 1));
      if (s + 1 < ntiles) zero_masked<D, BF16>(sm, grp, s + 1);
      __syncthreads();
    }
    __syncthreads();  // the scorer wave's factor
    if (active) {
      const float f = sm.fin[grp][col];
#pragma unroll
      for (int i = 0; i < kCbB; ++i) store_o<false>(a, t, l, nsplit, grp, kCbA + i, f, ob[i]);
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
  EKV_CHECK(heads > 0 && heads % 16 == 0 && heads <= 16 * kGroups, "heads must be a multiple of 16, <= 64");
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

// ---------------------------------------------------------------------------
// Allocation-free variant: the split partials live in `scratch`, a
// file-scope device array (one per GPU the library runs on, held until the
// process ends).  Its device address is looked up once per device, with that
// device current, on the first call there; host code passes that address to
// the kernels, never the array's name.  Calls on one GPU share the array, so
// calls that overlap on one GPU (different streams) race; the decode writes
// every partial it reads within the call, so nothing needs clearing.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchBytes = int64_t{64} << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

static void* scratch_address(int device) {
  void* p = g_scratch_ptr[device].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  p = g_scratch_ptr[device].load(std::memory_order_relaxed);
  if (p == nullptr) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    g_scratch_ptr[device].store(p, std::memory_order_release);
  }
  return p;
}

extern "C" int ekv_sparse_mla_decode_noalloc(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                             int32_t num_tokens, int32_t heads, int32_t dim, const uint8_t* cache,
                                             int32_t cache_bf16, int64_t page_stride, int64_t num_pages,
                                             const int32_t* indices, int64_t idx_stride, int32_t width,
                                             const int32_t* lengths, const int32_t* block_table, int64_t bt_stride,
                                             const int32_t* req_ids, const float* sinks, float scale, uint16_t* out,
                                             int64_t out_tok_stride, int64_t out_head_stride, float* lse,
                                             int64_t lse_stride, void* stream) {
  EKV_CHECK(num_tokens >= 0 && width >= 0, "sizes must be >= 0");
  if (num_tokens == 0) return 0;
  const int64_t need = ekv_sparse_mla_decode_workspace_size(num_tokens, heads, width);
  if (need > kNoAllocScratchBytes) {
    set_error("ekv_sparse_mla_decode_noalloc: the call needs more scratch than the 64 MiB the library holds "
              "(see ekv_sparse_mla_decode_workspace_size); use ekv_sparse_mla_decode with a workspace");
    return kInvalidArgument;
  }
  int device = 0;
  EKV_CHECK(hipGetDevice(&device) == hipSuccess && device >= 0 && device < kMaxDevices, "no current device");
  void* ws = scratch_address(device);
  EKV_CHECK(ws != nullptr, "hipGetSymbolAddress of the decode scratch failed");
  return ekv_sparse_mla_decode(q, q_tok_stride, q_head_stride, num_tokens, heads, dim, cache, cache_bf16, page_stride,
                               num_pages, indices, idx_stride, width, lengths, block_table, bt_stride, req_ids, sinks,
                               scale, out, out_tok_stride, out_head_stride, lse, lse_stride, ws, kNoAllocScratchBytes,
                               stream);
}
