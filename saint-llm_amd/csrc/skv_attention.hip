// Decode attention of one layer over the paged cache, with the gather fused in.
//
// Reference (one query token per sequence, MQA: one K/V head, H query heads):
//   CSA.forward   csa.py:324-373  sparse branch over the top-k picks (K = V =
//                                 k_norm(entry), no sink) + window branch
//   HCA.forward   hca.py:126-169  dense branch over the visible entries
//                                 (K = V = k_norm(entry), sink) + window branch
//   SWAttention   swa.py:115-137  window branch only
//   scaled_dot_product / softmax_with_sink / RMSNorm   common.py:12-124
// Each branch is its own softmax (scores q.k / sqrt(D); the window branch
// with the softcap c*tanh(s/c)); the layer's output is their sum.
//
// k_norm is folded in, not applied to the keys: with r_j = rsqrt(mean(k_j^2)
// + eps), q . (w*k_j*r_j) = ((q*w) . k_j) r_j and sum_j p_j w*k_j*r_j =
// w * sum_j (p_j r_j) k_j, so the MFMAs read the raw entries (fp8 entries are
// dequantized to bf16 exactly as the gathers do), q*w is formed once and w
// scales the merged output.
//
// Launch 1 (k_attn_part): one workgroup per (sequence, unit, head group of
// 64); a unit is a contiguous range of 32-key tiles of one branch.  Per tile:
// the key rows go to LDS twice, row-major for S^T = K Q^T (MFMA A = keys,
// B = queries: lane l holds key/head l%16 and dims 8*(l/16)..+7 of a 32-dim
// step) and transposed for O = P V (A = P straight from the S^T accumulators,
// B = V^T: lane l holds dim l%16 and 8 keys).  The transposed tile stores the
// keys in the order the S^T accumulators hold them (slot group g = keys
// 4g..4g+3 and 16+4g..16+4g+3), so P needs no shuffle.  Wave w owns heads
// 16w..16w+15: online softmax per head (log2 domain), O in 36 accumulators.
// The next tile's rows are loaded while the current one is multiplied
// (barriers order LDS only).  The unit writes (max, sum, O) per head.
// Launch 2 (k_attn_merge, or k_attn_merge_q for sequences of at most 8
// units): per (sequence, head) merges the units of each
// branch with the sink, applies 1/sum and w, and writes the sum of branches.
#include <algorithm>
#include <type_traits>

#include "skv_common.h"
#include "skv_entry.h"
#include "skv_step.h"

namespace skv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kAtThreads = 512;
constexpr int kAtWaves = kAtThreads / 64;
constexpr int kAtHeads = 64;  // query heads per workgroup: 16 per pair of waves
constexpr int kAtTile = 32;   // keys per tile
constexpr int kAtMaxD = 576;
constexpr int kAtMaxQueries = 4096;  // query tokens per sequence of one call
constexpr int kAtRun = 512;   // keys whose source rows are resolved at once
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kAhead = 4;  // LDS operand reads in flight ahead of the products
constexpr float kRescaleAt = 8.f;  // log2 headroom of the softmax weights over the reference max

struct AttnArgs {
  const uint8_t* q;  // [B, H, D] bf16
  float* part;       // [B * U * Hp] x (max, sum), then [B * U * Hp][D] O
  const int32_t* lens;
  const uint8_t* pool;
  const int32_t* block_table;
  const int32_t* n_entries;
  const int32_t* picks;
  const float* knorm_w;
  const uint8_t* win_k;
  const uint8_t* win_v;
  int64_t entry_bytes, pick_stride;
  int32_t kind, fp8_main;  // fp8_main > 0: fp8 entries with that many coded dims
  int32_t block_size, n_pages, bt_stride, m, top_k;
  int32_t window, H, D, n_hg, n_cu, n_wu;
  int32_t batch;       // query rows: sequences x n_q
  int32_t n_q;         // query tokens per sequence (row b: sequence b / n_q, token b % n_q)
  int32_t ring;        // window slots per sequence of win_k / win_v
  int64_t win_row;     // bytes from one window slot to the next
  float eps, softcap;  // softcap <= 0: none
  int32_t fused;       // 1: the decode step's last launch (lens are the step's new lengths)
  int32_t xcds;        // the device's XCDs, a power of two (unit placement)
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Key j (0..7) of slot group a (0..3) within a tile: keys 4a..4a+3, 16+4a..16+4a+3.
__device__ __forceinline__ int slot_key(int a, int j) { return (j < 4) ? 4 * a + j : 16 + 4 * a + (j - 4); }

template <int NKS>
struct AtSmem {
  static constexpr int kD = NKS * 32;
  // keys and window values: kAtTile rows of kD elements (32 bytes of pad
  // per row) in swizzled 16-byte chunks (tile_chunk)
  alignas(16) uint16_t kr[kAtTile][kD + 16];
  alignas(16) uint16_t vs[kAtTile][kD + 16];
  int64_t row[kAtRun];                       // byte offset of each key's source row in the run, -1 masked
  f32x4 sx[kAtWaves][2][kWave];              // per wave: its half-dims S^T partial per key block
  float ssx[2][2][16];                       // per half of the dims: the keys' sums of squares
  float w[kAtMaxD];                          // k_norm weight (compressed branch)
};

// A tile row's 16-byte chunk c (dims 8c..8c+7) sits at chunk c ^ ((r/4) % 2)
// of its LDS row; rows are kD + 16 elements apart.  The LDS has 32 banks of 4
// bytes, 8 chunks per bank round, and a row starts 2 chunks further round
// than the one before.  The 8 lanes of one cycle of a 16-byte operand read
// (rows r..r+7, one chunk c) then take chunks c + 2i (rows r + i, i < 4) and
// (c ^ 1) + 2i (the next 4), every position of the round once; the 16 lanes of
// one cycle of a transposing read (rows 4g..4g+3, an aligned pair of chunks
// each) take 4 different pairs.  (Rows of kD + 8 elements, one chunk round
// apart, put two of those rows' pairs on the same banks.)
__device__ __forceinline__ int tile_chunk(int r, int c) { return c ^ ((r >> 2) & 1); }

// Zero bytes that dead chunks (masked keys, dims past D) are read from: no
// select follows a load, so the loaded registers are first used when they are
// stored to LDS, one tile later, and the loads stay in flight meanwhile.
__device__ __align__(16) uint8_t g_zero_row[2 * kAtMaxD];

template <int NKS>
struct TileChunks {
  static constexpr int kChunks = NKS * 4;  // 16-byte chunks of a bf16 row of kD dims
  static constexpr int kTotal = kAtTile * kChunks;
  static constexpr int kPer = (kTotal + kAtThreads - 1) / kAtThreads;
};

// A tile's bf16 rows spread over the threads: chunk q = tid + 512k is dims
// 8(q % chunks).. of key q / chunks (consecutive threads read consecutive
// chunks of a row).
template <int NKS>
struct RawBf16 {
  u32x4 v[TileChunks<NKS>::kPer];
};

template <int NKS>
__device__ __forceinline__ void load_tile(RawBf16<NKS>& r, const int64_t* rows, const uint8_t* base, int D) {
  using TC = TileChunks<NKS>;
#pragma unroll
  for (int k = 0; k < TC::kPer; ++k) {
    const int q = min(static_cast<int>(threadIdx.x) + k * kAtThreads, TC::kTotal - 1);
    const int c = q % TC::kChunks;
    const int64_t off = rows[q / TC::kChunks];
    const bool live = off >= 0 && 8 * c < D;
    const uint8_t* p = live ? base + off + c * 16 : g_zero_row + c * 16;
    r.v[k] = *reinterpret_cast<const u32x4*>(p);
  }
}

template <int NKS>
__device__ __forceinline__ void store_tile(uint16_t* dst, const RawBf16<NKS>& r) {
  using TC = TileChunks<NKS>;
#pragma unroll
  for (int k = 0; k < TC::kPer; ++k) {
    const int q = static_cast<int>(threadIdx.x) + k * kAtThreads;
    if (TC::kTotal % kAtThreads == 0 || q < TC::kTotal) {
      const int row = q / TC::kChunks;
      *reinterpret_cast<u32x4*>(dst + row * (NKS * 32 + 16) + 8 * tile_chunk(row, q % TC::kChunks)) = r.v[k];
    }
  }
}

// A tile's fp8 entries (576 dims: 512 e4m3 codes, 4 fp32 scales, 64 bf16
// rope dims): 8-code chunks with their scale spread over the threads, then
// the rope chunks on threads 0..255; dequantized (fp32 product rounded to
// bf16, as the gathers do) when stored.
constexpr int kFp8Main = kAtMaxD - SKV_FP8_ROPE_DIMS;
constexpr int kFp8CodeChunks = kFp8Main / 8;         // per entry
constexpr int kFp8RopeChunks = SKV_FP8_ROPE_DIMS / 8;  // per entry
constexpr int kFp8CodePer = (kAtTile * kFp8CodeChunks + kAtThreads - 1) / kAtThreads;

struct RawFp8 {
  u32x2 codes[kFp8CodePer];
  float scale[kFp8CodePer];
  u32x4 rope;
};

__device__ __forceinline__ void load_tile(RawFp8& r, const int64_t* rows, const uint8_t* base) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < kFp8CodePer; ++k) {
    const int q = tid + k * kAtThreads;  // kAtTile * kFp8CodeChunks is a multiple of kAtThreads
    const int c = q % kFp8CodeChunks;
    const int64_t off = rows[q / kFp8CodeChunks];
    const uint8_t* p = off >= 0 ? base + off : g_zero_row;
    r.codes[k] = *reinterpret_cast<const u32x2*>(p + c * 8);
    r.scale[k] = *reinterpret_cast<const float*>(p + kFp8Main + (c >> 4) * 4);
  }
  const int qr = min(tid, kAtTile * kFp8RopeChunks - 1);
  const int64_t off = rows[qr / kFp8RopeChunks];
  const uint8_t* p = off >= 0 ? base + off : g_zero_row;
  r.rope = *reinterpret_cast<const u32x4*>(p + kFp8Main + (kFp8Main >> 7) * 4 + (qr % kFp8RopeChunks) * 16);
}

__device__ __forceinline__ void store_tile(uint16_t* dst, const RawFp8& r) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < kFp8CodePer; ++k) {
    const int q = tid + k * kAtThreads;
    float f[8];
    e4m3fn_x4_to_f32(r.codes[k][0], f);
    e4m3fn_x4_to_f32(r.codes[k][1], f + 4);
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) o[h] = bf16_pack2(f[2 * h] * r.scale[k], f[2 * h + 1] * r.scale[k]);
    const int row = q / kFp8CodeChunks;
    *reinterpret_cast<u32x4*>(dst + row * (kAtMaxD + 16) + 8 * tile_chunk(row, q % kFp8CodeChunks)) = o;
  }
  if (tid < kAtTile * kFp8RopeChunks) {
    const int row = tid / kFp8RopeChunks;
    *reinterpret_cast<u32x4*>(dst + row * (kAtMaxD + 16) +
                              8 * tile_chunk(row, kFp8CodeChunks + tid % kFp8RopeChunks)) = r.rope;
  }
}

typedef short short4v __attribute__((ext_vector_type(4)));

// Four keys of one dim from row-major rows, by gfx950's transposing LDS read:
// in each group of 16 lanes, source lane s gives the address of 4 bf16 and
// lane i receives element i%4 of sources i/4, i/4+4, i/4+8, i/4+12.  With
// source lane s pointing at dims c + 4(s%4).. of key row r0 + s/4, lane i gets
// dim c + i of rows r0..r0+3.
__device__ __forceinline__ u32x2 read_tr(const uint16_t* p) {
  const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4v*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// The keys of a unit: the picks of a top-k row (CSA), the visible entries
// (HCA) or the window, split by tiles over the units of the branch.
struct NoRank {
  static constexpr bool kOn = false;
};

// Unit s of ns of one branch (kComp: compressed entries, else the window).
// Waves 2hb and 2hb+1 share heads 16hb..16hb+15 of the group: wave half h
// multiplies key block h (keys 16h..16h+15) for S^T and dims
// [kD/2 * h, kD/2 * (h+1)) for O; the pair exchanges its block maxima and P
// through LDS.  With a ranking Rank (Rank::kOn), a CSA unit's keys are the
// picks Rank finds (its share of the row's top-k, in output order) once the
// query's loads are in flight; they resolve to pool rows through Rank::row.
template <int NKS, bool kFp8, bool kComp, class Rank = NoRank>
__device__ __forceinline__ void attn_unit(AtSmem<NKS>& sm, const AttnArgs& a, int b, int s, int ns, int hg,
                                          int64_t unit, Rank&& rk = Rank{}) {
  constexpr int kD = NKS * 32;
  constexpr int kDbW = kD / 32;  // 16-dim blocks of O per wave
  constexpr bool kRanked = std::remove_reference_t<Rank>::kOn;
  static_assert(!kRanked || kComp, "ranked keys are compressed entries");
  using TC = TileChunks<NKS>;
  const int tid = threadIdx.x;
  // a ranked unit takes the wave's index as a scalar (uniform) value: the
  // values derived from it then stay out of the vector registers, which its
  // tile loop fills (spill stores ahead of the loop would hold its first
  // wait on the vector memory count); the other units keep the allocation
  // that spills least for them
  const int wave = (kRanked ? __builtin_amdgcn_readfirstlane(tid) : tid) / kWave, lane = tid % kWave;
  const int hb = wave >> 1, half = wave & 1;
  const int col = lane & 15, grp = lane >> 4;
  // query row b is token t of sequence cb, position L - n_q + t of its L
  // tokens: it sees the first L - n_q + t + 1 of them
  const int cb = b / a.n_q, t_q = b - cb * a.n_q;
  const int L = min(max(a.lens[cb] - (a.n_q - 1 - t_q), 0), (1 << 24) - 1);
  // keys of this branch for query row b (ranked: known after the ranking)
  int n_keys = 0;
  if constexpr (!kComp) {
    n_keys = min(L, a.window);
  } else if constexpr (!kRanked) {
    if (a.kind == SKV_LAYER_CSA) {
      n_keys = a.top_k;
    } else {
      // in the step's launch the visible count (L-1)/m is what the entry
      // count committed beside it bounds it by
      const int q_pos = max(L - 1, 0);
      n_keys = a.fused ? static_cast<int>(udiv24(q_pos, a.m))
                       : min(static_cast<int>(udiv24(q_pos, a.m)), max(a.n_entries[cb], 0));
    }
  }
  int n_tiles = (n_keys + kAtTile - 1) / kAtTile;
  int t_lo = static_cast<int>((static_cast<int64_t>(s) * n_tiles) / ns);
  int t_hi = static_cast<int>((static_cast<int64_t>(s + 1) * n_tiles) / ns);
  const int head0 = hg * kAtHeads + hb * 16;  // the pair's first head
  float* part_ml = a.part + unit * kAtHeads * 2;
  const int64_t n_units = static_cast<int64_t>(a.batch) * (a.n_cu + a.n_wu) * a.n_hg;
  uint16_t* part_o =  // bf16 outputs after every unit's (max, sum)
      reinterpret_cast<uint16_t*>(a.part + n_units * kAtHeads * 2) + unit * kAtHeads * a.D;
  const int D = a.D;
  // query (times w for the compressed branch) as B operands for this wave's
  // half of the dims: head head0+col, dims 32(ks0 + ks) + 8grp..+7, zero past
  // H and D
  constexpr int kHalfKs = NKS / 2;
  const int ks0 = half * kHalfKs;
  // The prologue's loads, in this order (vector loads complete in order):
  // a CSA unit's first pick and the entry count; the k_norm weight, one or
  // two elements per thread, for LDS (per-lane loads of each 32-dim step's 8
  // weights would add 18 load instructions per wave, which the CU's address
  // unit works through one after another); the query; then the pick's
  // block-table entry, which waits for the pick only.  The pick -> block
  // table chain overlaps the query's round trip, and q * w waits for the
  // query.  Every load is unconditional (a branch around a load waits for it
  // where the branch ends); lanes without a key read the zero row.
  // A ranked unit's first loads are its ranking's (they return first).
  int32_t pick0 = 0, ne0 = 0;
  float w_lo = 0.f, w_hi = 0.f;
  using Raw = std::conditional_t<kFp8, RawFp8, RawBf16<NKS>>;
  Raw raw;                 // a compressed tile's rows in flight
  bool raw_early = false;  // the first tile's loads were issued by the ranking
  auto load_raw = [&](Raw& r, const int64_t* rows, const uint8_t* base) {
    if constexpr (kFp8) {
      load_tile(r, rows, base);
    } else {
      load_tile<NKS>(r, rows, base, D);
    }
  };

  if constexpr (kRanked) {
    rk.load();
    w_lo = a.knorm_w[min(tid, D - 1)];
    w_hi = a.knorm_w[min(tid + kAtThreads, D - 1)];
  } else if constexpr (kComp) {
    const bool csa = a.kind == SKV_LAYER_CSA && n_keys > 0;
    pick0 = *(csa ? a.picks + static_cast<int64_t>(b) * a.pick_stride + min(t_lo * kAtTile + tid, n_keys - 1)
                  : reinterpret_cast<const int32_t*>(g_zero_row));
    ne0 = a.n_entries[cb];
    w_lo = a.knorm_w[min(tid, D - 1)];
    w_hi = a.knorm_w[min(tid + kAtThreads, D - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 qreg[kHalfKs];
  {
    const int h = head0 + col;
    const uint8_t* qrow = a.q + (static_cast<int64_t>(b) * a.H + min(h, a.H - 1)) * D * 2;
#pragma unroll
    for (int ks = 0; ks < kHalfKs; ++ks) {
      const int d0 = (ks0 + ks) * 32 + grp * 8;
      const bool live = h < a.H && d0 < D;
      // dead lanes read zeros: no select after the load, which would make
      // the window branch wait for the query before its row lookups
      qreg[ks] = *reinterpret_cast<const u32x4*>(live ? qrow + d0 * 2 : g_zero_row);
    }
  }
  if constexpr (kRanked) rk.load_bt();
  __builtin_amdgcn_sched_barrier(0);
  int e0 = -1, pi0 = 0;
  int32_t page0 = -1;
  if constexpr (kComp && !kRanked) {
    e0 = (pick0 < max(ne0, 0)) ? pick0 : -1;
    pi0 = e0 >= 0 ? static_cast<int>(udiv24(e0, a.block_size)) : 0;
    if (pi0 >= a.bt_stride) e0 = -1;
    page0 = *(e0 >= 0 ? a.block_table + static_cast<int64_t>(cb) * a.bt_stride + pi0
                      : reinterpret_cast<const int32_t*>(g_zero_row));
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kComp) {
    if (tid < D) sm.w[tid] = w_lo;
    if (tid + kAtThreads < D) sm.w[tid + kAtThreads] = w_hi;
    lds_barrier();
    if constexpr (kRanked) {
      // the ranking waits for its own loads only; q * w below waits for the query.
      // Where the unit's first tile is all sure keys, the ranking resolves
      // their rows and issues the tile's loads before it ranks the ties.
      n_keys = rk.rank(sm, [&]() {
        for (int j = tid; j < kAtTile; j += kAtThreads) {
          const int64_t r = rk.row(j);
          sm.row[j] = r >= 0 ? r * a.entry_bytes : -1;
        }
        lds_barrier();
        load_raw(raw, sm.row, a.pool);
        raw_early = true;
      });
      n_tiles = (n_keys + kAtTile - 1) / kAtTile;
      t_lo = 0;
      t_hi = n_tiles;
    }
    const int h = head0 + col;
#pragma unroll
    for (int ks = 0; ks < kHalfKs; ++ks) {
      const int d0 = (ks0 + ks) * 32 + grp * 8;
      const bool live = h < a.H && d0 < D;
      const float* wp = sm.w + (live ? d0 : 0);
      u32x4 v = qreg[ks];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[t] = bf16_pack2(__uint_as_float(v[t] << 16) * wp[2 * t], __uint_as_float(v[t] & 0xffff0000u) * wp[2 * t + 1]);
      }
      qreg[ks] = v;
    }
  }
  const float inv_sqrt_d = rsqrtf(static_cast<float>(D));
  const float inv_d = 1.f / static_cast<float>(D);
  const float scale2 = inv_sqrt_d * kLog2e;
  const bool capped = !kComp && a.softcap > 0.f;
  const float inv_cap = capped ? 1.f / a.softcap : 0.f;
  const float cap_log2e = a.softcap * kLog2e;
  const int64_t row_bytes = kComp ? a.entry_bytes : a.win_row;
  const uint8_t* kbase = kComp ? a.pool : a.win_k;
  float m_run = -__builtin_huge_valf(), l_run = 0.f;
  f32x4 acc_o[kDbW];
#pragma unroll
  for (int db = 0; db < kDbW; ++db) acc_o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // LDS element offsets of the tile operands (tile_chunk's layout; the swizzle
  // flips bit 0 of the chunk index, so chunk 4m + grp and pair 2X move by
  // whole steps of m and X).  K (S^T's A operand): lane (col, grp) reads
  // chunk 4m + grp, m = ks0 + ks, of rows col and 16 + col.  V (O's B operand,
  // transposing reads): lane (col, grp) reads dims 4(col % 4).. of 16-dim
  // block X = half * kDbW + db in rows 4grp + col/4 and 16 more, chunk
  // 2X + (col % 4) / 2.
  constexpr int kRow = kD + 16;
  const int koff = col * kRow + 8 * tile_chunk(col, grp) + 32 * ks0;
  const int voff = (4 * grp + (col >> 2)) * kRow + 8 * tile_chunk(4 * grp + (col >> 2), (col & 3) >> 1) +
                   4 * (col & 1) + 16 * half * kDbW;
  for (int k_lo = t_lo * kAtTile; k_lo < t_hi * kAtTile; k_lo += kAtRun) {
    const int k_hi = min(t_hi * kAtTile, k_lo + kAtRun);
    lds_barrier();  // the previous run's rows are no longer read
    // source rows of keys [k_lo, k_hi): -1 for masked keys
    for (int j = k_lo + tid; j < k_hi; j += kAtThreads) {
      int64_t row = -1;
      if (j < n_keys) {
        if constexpr (!kComp) {
          const int pos = L - n_keys + j;
          row = (static_cast<int64_t>(cb) * a.ring + static_cast<int>(umod24(pos, a.ring))) * row_bytes;
        } else if constexpr (kRanked) {
          const int64_t r = rk.row(j);
          row = r >= 0 ? r * row_bytes : -1;
        } else {
          int e = j;
          if (a.kind == SKV_LAYER_CSA) {
            if (k_lo == t_lo * kAtTile) {  // uniform: the first run's rows come from the prologue
              e = -1;
              if (e0 >= 0 && page0 >= 0 && page0 < a.n_pages) {
                row = (static_cast<int64_t>(page0) * a.block_size + (e0 - pi0 * a.block_size)) * row_bytes;
              }
            } else {
              e = a.picks[static_cast<int64_t>(b) * a.pick_stride + j];
              if (e >= max(a.n_entries[cb], 0)) e = -1;
            }
          }
          if (e >= 0) {
            const int pi = static_cast<int>(udiv24(e, a.block_size));
            if (pi < a.bt_stride) {
              const int32_t page = a.block_table[static_cast<int64_t>(cb) * a.bt_stride + pi];
              if (page >= 0 && page < a.n_pages) {
                row = (static_cast<int64_t>(page) * a.block_size + (e - pi * a.block_size)) * row_bytes;
              }
            }
          }
        }
      }
      sm.row[j - k_lo] = row;
    }
    lds_barrier();
    const int n_run_tiles = (k_hi - k_lo) / kAtTile;
    if constexpr (kComp) {
      if (!(raw_early && k_lo == 0)) load_raw(raw, sm.row, kbase);  // uniform
    }
    for (int t = 0; t < n_run_tiles; ++t) {
      const int64_t* rows = sm.row + t * kAtTile;
      lds_barrier();  // the previous tile's LDS reads are done
      if constexpr (kComp) {
        if constexpr (kFp8) {
          store_tile(&sm.kr[0][0], raw);
        } else {
          store_tile<NKS>(&sm.kr[0][0], raw);
        }
        // the next tile's rows are in flight while this one is multiplied
        if (t + 1 < n_run_tiles) load_raw(raw, rows + kAtTile, kbase);
      } else {
        RawBf16<NKS> rk, rv;
        load_tile<NKS>(rk, rows, kbase, D);  // keys and values in flight together
        load_tile<NKS>(rv, rows, a.win_v, D);
        store_tile<NKS>(&sm.kr[0][0], rk);
        store_tile<NKS>(&sm.vs[0][0], rv);
      }
      lds_barrier();
      // which keys of the tile are live (bits 0..31)
      const uint64_t live = __ballot(lane < kAtTile && rows[lane & (kAtTile - 1)] >= 0);
      // S^T = K (Q w)^T over this wave's half of the dims, both key blocks:
      // keys 16kb + 4grp + i, head head0 + col
      // operand o = 2ks + kb: reads run kAhead operands ahead of the
      // products, and the two key blocks' products alternate (independent
      // accumulators)
      constexpr int kOps = 2 * kHalfKs;
      u32x4 kv[kOps];
      auto read_k = [&](int o) {
        kv[o] = *reinterpret_cast<const u32x4*>(&sm.kr[0][0] + koff + 32 * (o >> 1) + (o & 1) * 16 * kRow);
      };
#pragma unroll
      for (int o = 0; o < kAhead; ++o) read_k(o);
      f32x4 st[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      // the keys' sums of squares for k_norm: diag(K K^T) over this wave's
      // half of the dims, on the pair of head block 0 only
      f32x4 sq[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      if (kComp && hb == 0) {
#pragma unroll
        for (int o = 0; o < kOps; ++o) {
          if (o + kAhead < kOps) read_k(o + kAhead);
          const int kb = o & 1;
          st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kv[o]), as_bf16x8(qreg[o >> 1]), st[kb], 0, 0, 0);
          sq[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kv[o]), as_bf16x8(kv[o]), sq[kb], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        // lane (col, grp) holds the diagonal element of key col when col - 4grp is in [0, 4)
        const int i = col - 4 * grp;
        if (i >= 0 && i < 4) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) sm.ssx[half][kb][col] = i == 0 ? sq[kb][0] : i == 1 ? sq[kb][1] : i == 2 ? sq[kb][2] : sq[kb][3];
        }
      } else {
#pragma unroll
        for (int o = 0; o < kOps; ++o) {
          if (o + kAhead < kOps) read_k(o + kAhead);
          const int kb = o & 1;
          st[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kv[o]), as_bf16x8(qreg[o >> 1]), st[kb], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) sm.sx[wave][kb][lane] = st[kb];
      lds_barrier();  // the pair's partials
      // full scores: own half + the pair's half; norm factors of the keys
      // this lane's accumulators hold (16kb + 4grp + i)
      float sc[2][4], rk[2][4];
      float mx = -__builtin_huge_valf();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const f32x4 other = sm.sx[wave ^ 1][kb][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = 16 * kb + 4 * grp + i;
          if constexpr (kComp) {
            const float ssum = sm.ssx[0][kb][4 * grp + i] + sm.ssx[1][kb][4 * grp + i];
            rk[kb][i] = rsqrtf(fmaf(ssum, inv_d, a.eps));
          } else {
            rk[kb][i] = 1.f;
          }
          float v;
          if (capped) {
            v = (st[kb][i] + other[i]) * inv_sqrt_d;
            v = cap_log2e * tanhf(v * inv_cap);
          } else {
            v = (st[kb][i] + other[i]) * (rk[kb][i] * scale2);
          }
          v = ((live >> key) & 1) ? v : -__builtin_huge_valf();
          sc[kb][i] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // the reference max moves only when the tile's max passes it by more
      // than kRescaleAt (log2): weights stay below 2^kRescaleAt otherwise, and
      // O and the sum are rescaled rarely
      const bool move = mx > m_run + kRescaleAt;
      const float alpha = move ? __builtin_amdgcn_exp2f(m_run - mx) : 1.f;
      if (move) m_run = mx;
      const bool none = m_run == -__builtin_huge_valf();
      float psum = 0.f;
      u32x4 pa;  // P as A operand: slots 8grp..+3 = key block 0, +4..+7 = key block 1
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = none ? 0.f : __builtin_amdgcn_exp2f(sc[kb][i] - m_run);
          psum += p[i];
          p[i] *= rk[kb][i];
        }
        pa[2 * kb] = bf16_pack2(p[0], p[1]);
        pa[2 * kb + 1] = bf16_pack2(p[2], p[3]);
      }
      l_run = l_run * alpha + psum;
      // rescale O rows (heads head0 + 4grp + i) by their alpha
      if (__ballot(alpha != 1.f)) {
        float al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * grp + i);
#pragma unroll
        for (int db = 0; db < kDbW; ++db) {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc_o[db][i] *= al[i];
        }
      }
      // O += P V over this wave's dims, reads kAhead operands ahead.  The B
      // operand of lane (n, grp) is dim 16db + n of the slot group's keys
      // 4grp..4grp+3 and 16+4grp..16+4grp+3, read transposed from the rows
      u32x4 vv[kDbW];
      const uint16_t* vrows = kComp ? &sm.kr[0][0] : &sm.vs[0][0];
      auto read_v = [&](int db) {
        const uint16_t* v = vrows + voff + 16 * db;
        const u32x2 lo = read_tr(v);
        const u32x2 hi = read_tr(v + 16 * kRow);
        vv[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
#pragma unroll
      for (int db = 0; db < kAhead; ++db) read_v(db);
#pragma unroll
      for (int db = 0; db < kDbW; ++db) {
        if (db + kAhead < kDbW) read_v(db + kAhead);
        acc_o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pa), as_bf16x8(vv[db]), acc_o[db], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  // the unit's (max, sum) per head and, when it saw a live key, its O
  // both waves of the pair hold the same (max, sum): the sum over the lane
  // groups of the per-lane partial sums
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (half == 0 && grp == 0) {
    const int hl = hb * 16 + col;  // head within the group
    part_ml[2 * hl] = m_run;
    part_ml[2 * hl + 1] = l_run;
  }
  if constexpr (kRanked) rk.finish(sm);
  if (!__ballot(m_run != -__builtin_huge_valf())) return;  // no live key: O is not read
#pragma unroll
  for (int db = 0; db < kDbW; ++db) {
    const int d = 16 * (half * kDbW + db) + col;
    if (d < D) {
#pragma unroll
      for (int i = 0; i < 4; ++i) part_o[static_cast<int64_t>(hb * 16 + 4 * grp + i) * D + d] = static_cast<uint16_t>(bf16_pack2(acc_o[db][i], 0.f));
    }
  }
}

// Blocks go to the XCDs in turn (block i to XCD i % X on a device of X =
// a.xcds XCDs); the units of sequence b take the blocks of XCD b % X, so the
// query that every unit of b reads comes from far memory once per sequence
// and the partial outputs stay in the L2 of the XCD whose merge blocks read
// them (merge block b runs there too when the batch is a multiple of X).
// The grid holds X * ceil(batch / X) * (units per sequence) blocks; blocks
// past the batch exit.

template <int NKS, bool kFp8>
__global__ __launch_bounds__(kAtThreads, 1) void k_attn_part(AttnArgs a) {
  __shared__ AtSmem<NKS> sm;
  const int U = a.n_cu + a.n_wu;
  const int per_seq = U * a.n_hg;
  const int xs = __builtin_ctz(static_cast<uint32_t>(a.xcds));  // a.xcds is a power of two
  const int k = static_cast<int>(blockIdx.x) >> xs;             // this block's turn on its XCD
  const int sb = k / per_seq;
  const int b = (static_cast<int>(blockIdx.x) & (a.xcds - 1)) + (sb << xs);
  if (b >= a.batch) return;  // uniform
  const int r = k - sb * per_seq;
  const int u = r / a.n_hg, hg = r - u * a.n_hg;
  const int64_t unit = (static_cast<int64_t>(b) * U + u) * a.n_hg + hg;
  if (u < a.n_cu) {
    attn_unit<NKS, kFp8, true>(sm, a, b, u, a.n_cu, hg, unit);
  } else {
    attn_unit<NKS, false, false>(sm, a, b, u - a.n_cu, a.n_wu, hg, unit);
  }
}

struct MergeArgs {
  const float* part;
  float* out;  // [B, H, D]
  const float* knorm_w;
  const float* sink;  // [H] or nullptr
  int32_t H, D, n_hg, n_cu, n_wu;
  int32_t sink_comp;  // the compressed branch takes the sink (HCA)
};

// One workgroup per (sequence, 4 heads, half of the dims), one wave per
// head.  Two memory round trips: lane t loads the (max, sum) of unit t (units
// of both branches), the wave reduces them per branch; then every lane loads
// its dims of 16 units' outputs at a time and sums them with the weights.
constexpr int kMergeUnits = 64;  // units per sequence the merge takes (one per lane)
constexpr int kMergeChunk = 16;  // units whose outputs are loaded at once

__global__ __launch_bounds__(256) void k_attn_merge(MergeArgs a) {
  const int b = blockIdx.x;
  const int h = blockIdx.y * 4 + static_cast<int>(threadIdx.x) / kWave;
  const int t = threadIdx.x % kWave;
  if (h >= a.H) return;
  const int U = a.n_cu + a.n_wu;
  const int hg = h / kAtHeads, hl = h % kAtHeads;
  const int64_t n_units = static_cast<int64_t>(gridDim.x) * U * a.n_hg;
  auto unit_of = [&](int u) { return (static_cast<int64_t>(b) * U + u) * a.n_hg + hg; };
  const uint16_t* po = reinterpret_cast<const uint16_t*>(a.part + n_units * kAtHeads * 2);
  const float ninf = -__builtin_huge_valf();
  // this lane's dims: d0 + t + 64j, j < kJ, within this half
  const int dh = (a.D + 1) / 2;
  const int d0 = blockIdx.z * dh, d1 = min(a.D, d0 + dh);
  constexpr int kJ = (kAtMaxD / 2 + kWave - 1) / kWave;
  float kw[kJ];
#pragma unroll
  for (int j = 0; j < kJ; ++j) kw[j] = a.knorm_w ? a.knorm_w[min(d0 + t + kWave * j, a.D - 1)] : 0.f;
  // lane t: unit t's (max, sum)
  const int64_t mi = unit_of(min(t, U - 1)) * kAtHeads * 2 + 2 * hl;
  const float m_t = t < U ? a.part[mi] : ninf;
  const float l_t = t < U ? a.part[mi + 1] : 0.f;
  const bool comp_t = t < a.n_cu;
  const float sink2 = a.sink ? a.sink[h] * kLog2e : ninf;
  // per branch: max over the units (and the sink), the denominator
  float mc = comp_t ? m_t : ninf, mw = comp_t ? ninf : m_t;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mc = fmaxf(mc, __shfl_xor(mc, off));
    mw = fmaxf(mw, __shfl_xor(mw, off));
  }
  const bool live_c = mc != ninf, live_w = mw != ninf;  // the branch saw a live key
  if (a.sink_comp) mc = fmaxf(mc, sink2);
  mw = fmaxf(mw, sink2);
  const float mb = comp_t ? mc : mw;
  const float w_t = m_t != ninf ? __builtin_amdgcn_exp2f(m_t - mb) : 0.f;
  float dc = comp_t ? w_t * l_t : 0.f, dw = comp_t ? 0.f : w_t * l_t;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    dc += __shfl_xor(dc, off);
    dw += __shfl_xor(dw, off);
  }
  if (a.sink_comp && sink2 != ninf) dc += __builtin_amdgcn_exp2f(sink2 - mc);
  if (sink2 != ninf) dw += __builtin_amdgcn_exp2f(sink2 - mw);
  // unit t's weight in the output: its branch's 1/denominator folded in (0
  // for a branch without a live key)
  const float f_t = comp_t ? (live_c ? w_t / dc : 0.f) : (live_w ? w_t / dw : 0.f);
  float rc[kJ], rw[kJ];
#pragma unroll
  for (int j = 0; j < kJ; ++j) rc[j] = rw[j] = 0.f;
  for (int u0 = 0; u0 < U; u0 += kMergeChunk) {
    float o[kMergeChunk][kJ];
#pragma unroll
    for (int q = 0; q < kMergeChunk; ++q) {
      const uint16_t* ou = po + (unit_of(min(u0 + q, U - 1)) * kAtHeads + hl) * a.D;
#pragma unroll
      for (int j = 0; j < kJ; ++j) o[q][j] = bf16_to_f32(ou[min(d0 + t + kWave * j, a.D - 1)]);
    }
#pragma unroll
    for (int q = 0; q < kMergeChunk; ++q) {
      const float f = __shfl(f_t, min(u0 + q, kWave - 1));
      if (u0 + q < U && f > 0.f) {  // units without a live key wrote no output
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
          if (u0 + q < a.n_cu) {
            rc[j] = fmaf(f, o[q][j], rc[j]);
          } else {
            rw[j] = fmaf(f, o[q][j], rw[j]);
          }
        }
      }
    }
  }
  float* out = a.out + (static_cast<int64_t>(b) * a.H + h) * a.D;
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const int d = d0 + t + kWave * j;
    if (d < d1) out[d] = (live_c ? rc[j] * kw[j] : 0.f) + rw[j];
  }
}

// The merge for sequences of at most kMergeChunkQ units: one wave per (head,
// third of the dims), lane t takes the 4-dim quad t + 64z, so that every load
// and store of the wave covers consecutive bytes; one memory round trip
// brings lane t's (max, sum) of unit t and its quad of every unit's output.
constexpr int kMergeChunkQ = 8;
constexpr int kQLane = 1;  // quads per lane

__global__ __launch_bounds__(256) void k_attn_merge_q(MergeArgs a) {
  const int b = blockIdx.x;
  const int h = blockIdx.y * 4 + static_cast<int>(threadIdx.x) / kWave;
  const int t = threadIdx.x % kWave;
  if (h >= a.H) return;  // whole waves
  const int U = a.n_cu + a.n_wu;
  const int hg = h / kAtHeads, hl = h % kAtHeads;
  const int64_t n_units = static_cast<int64_t>(gridDim.x) * U * a.n_hg;
  auto unit_of = [&](int u) { return (static_cast<int64_t>(b) * U + u) * a.n_hg + hg; };
  const uint16_t* po = reinterpret_cast<const uint16_t*>(a.part + n_units * kAtHeads * 2);
  const float ninf = -__builtin_huge_valf();
  const int n_quads = a.D / 4;  // D is a multiple of 32
  int qj[kQLane];  // this lane's quads (clamped; stores check the bound)
#pragma unroll
  for (int j = 0; j < kQLane; ++j) qj[j] = min(t + kWave * (blockIdx.z + gridDim.z * j), n_quads - 1);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  auto load_units = [&](u32x2 (&o)[kMergeChunkQ][kQLane], int u0) {
#pragma unroll
    for (int q = 0; q < kMergeChunkQ; ++q) {
      const u32x2* ou = reinterpret_cast<const u32x2*>(po + (unit_of(min(u0 + q, U - 1)) * kAtHeads + hl) * a.D);
#pragma unroll
      for (int j = 0; j < kQLane; ++j) o[q][j] = ou[qj[j]];
    }
  };
  // every load of the round trip before any use
  const int64_t mi = unit_of(min(t, U - 1)) * kAtHeads * 2 + 2 * hl;
  const float m_raw = a.part[mi];
  const float l_raw = a.part[mi + 1];
  u32x2 o[kMergeChunkQ][kQLane];
  load_units(o, 0);
  float kw[kQLane][4];  // knorm_w and out may be only 4-byte aligned
#pragma unroll
  for (int j = 0; j < kQLane; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) kw[j][e] = a.knorm_w ? a.knorm_w[4 * qj[j] + e] : 0.f;
  }
  const float m_t = t < U ? m_raw : ninf;
  const float l_t = t < U ? l_raw : 0.f;
  const bool comp_t = t < a.n_cu;
  const float sink2 = a.sink ? a.sink[h] * kLog2e : ninf;
  // per branch: max over the units (and the sink), the denominator
  float mc = comp_t ? m_t : ninf, mw = comp_t ? ninf : m_t;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mc = fmaxf(mc, __shfl_xor(mc, off));
    mw = fmaxf(mw, __shfl_xor(mw, off));
  }
  const bool live_c = mc != ninf, live_w = mw != ninf;  // the branch saw a live key
  if (a.sink_comp) mc = fmaxf(mc, sink2);
  mw = fmaxf(mw, sink2);
  const float mb = comp_t ? mc : mw;
  const float w_t = m_t != ninf ? __builtin_amdgcn_exp2f(m_t - mb) : 0.f;
  float dc = comp_t ? w_t * l_t : 0.f, dw = comp_t ? 0.f : w_t * l_t;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    dc += __shfl_xor(dc, off);
    dw += __shfl_xor(dw, off);
  }
  if (a.sink_comp && sink2 != ninf) dc += __builtin_amdgcn_exp2f(sink2 - mc);
  if (sink2 != ninf) dw += __builtin_amdgcn_exp2f(sink2 - mw);
  // unit t's weight in the output: its branch's 1/denominator folded in (0
  // for a branch without a live key)
  const float f_t = comp_t ? (live_c ? w_t / dc : 0.f) : (live_w ? w_t / dw : 0.f);
  float rc[kQLane][4], rw[kQLane][4];
#pragma unroll
  for (int j = 0; j < kQLane; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) rc[j][e] = rw[j][e] = 0.f;
  }
  for (int u0 = 0; u0 < U; u0 += kMergeChunkQ) {
    if (u0 > 0) load_units(o, u0);
#pragma unroll
    for (int q = 0; q < kMergeChunkQ; ++q) {
      const float f = __shfl(f_t, min(u0 + q, kWave - 1));
      if (u0 + q < U && f > 0.f) {  // units without a live key wrote no output
        const bool comp = u0 + q < a.n_cu;
#pragma unroll
        for (int j = 0; j < kQLane; ++j) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const uint32_t w2 = o[q][j][e];
            const float lo = __uint_as_float(w2 << 16), hi = __uint_as_float(w2 & 0xffff0000u);
            if (comp) {
              rc[j][2 * e] = fmaf(f, lo, rc[j][2 * e]);
              rc[j][2 * e + 1] = fmaf(f, hi, rc[j][2 * e + 1]);
            } else {
              rw[j][2 * e] = fmaf(f, lo, rw[j][2 * e]);
              rw[j][2 * e + 1] = fmaf(f, hi, rw[j][2 * e + 1]);
            }
          }
        }
      }
    }
  }
  float* out = a.out + (static_cast<int64_t>(b) * a.H + h) * a.D;
  const bool al16 = (reinterpret_cast<uintptr_t>(out) & 15) == 0;  // uniform
#pragma unroll
  for (int j = 0; j < kQLane; ++j) {
    const int c = t + kWave * (blockIdx.z + gridDim.z * j);
    if (c >= n_quads) continue;
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (live_c ? rc[j][e] * kw[j][e] : 0.f) + rw[j][e];
    if (al16) {
      reinterpret_cast<f32x4*>(out)[c] = v;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) out[4 * c + e] = v[e];
    }
  }
}

struct AttnPlan {
  int n_cu, n_wu, n_hg, nks;
  int64_t rows;  // query rows: batch x query tokens per sequence
  int64_t nq, ring, win_row;
  int64_t ws_bytes;
};

int attn_plan(const skv_attention_desc* d, AttnPlan& p) {
  const char* what = "skv_decode_attention";
  if (!d) return set_error(SKV_EINVAL, "%s: NULL descriptor", what);
  if (d->batch < 0) return set_error(SKV_EINVAL, "%s: negative batch", what);
  if (d->kind != SKV_LAYER_SWA && d->kind != SKV_LAYER_HCA && d->kind != SKV_LAYER_CSA) {
    return set_error(SKV_EINVAL, "%s: unknown layer kind %d", what, d->kind);
  }
  if (d->n_heads < 1 || d->n_heads > 4 * kAtHeads) {
    return set_error(SKV_EINVAL, "%s: n_heads must be in [1, %d]", what, 4 * kAtHeads);
  }
  if (d->head_dim < 32 || d->head_dim > kAtMaxD || d->head_dim % 32) {
    return set_error(SKV_EINVAL, "%s: head_dim must be a multiple of 32 in [32, %d]", what, kAtMaxD);
  }
  if (d->window < 1 || d->window >= (1 << 24)) return set_error(SKV_EINVAL, "%s: window must be in [1, 2^24)", what);
  p.nq = d->n_queries > 0 ? d->n_queries : 1;
  p.ring = d->ring > 0 ? d->ring : d->window;
  if (d->n_queries < 0 || p.nq > kAtMaxQueries) {
    return set_error(SKV_EINVAL, "%s: n_queries must be in [0, %d]", what, kAtMaxQueries);
  }
  if (d->ring < 0 || p.ring >= (1 << 24) || p.ring < d->window) {
    return set_error(SKV_EINVAL, "%s: ring must be in [window, 2^24)", what);
  }
  p.win_row = d->win_stride > 0 ? d->win_stride : d->head_dim * 2;
  if (d->win_stride < 0 || (d->win_stride > 0 && (d->win_stride < d->head_dim * 2 || d->win_stride % 16))) {
    return set_error(SKV_EINVAL, "%s: win_stride must be 0 or a multiple of 16 of at least head_dim * 2", what);
  }
  p.rows = d->batch * p.nq;
  if (p.rows >= (1 << 24)) return set_error(SKV_EINVAL, "%s: batch x n_queries must be < 2^24", what);
  const bool comp = d->kind != SKV_LAYER_SWA;
  int64_t comp_keys = 0;
  if (comp) {
    if (d->block_size <= 0 || d->n_pages <= 0 || d->n_pages > 0x7fffffff || d->bt_stride <= 0 ||
        d->bt_stride * d->block_size >= (1 << 24)) {
      return set_error(SKV_EINVAL, "%s: bad page geometry (bt_stride * block_size must be < 2^24)", what);
    }
    const int main = entry_layout(d->format, d->head_dim, d->entry_bytes);
    if (main < 0) return set_error(SKV_EINVAL, "%s: entry_bytes/format do not match head_dim", what);
    if (d->format == SKV_FMT_FP8 && d->head_dim != kAtMaxD) {
      return set_error(SKV_EINVAL, "%s: fp8 entries need head_dim %d", what, kAtMaxD);
    }
    if (d->kind == SKV_LAYER_CSA) {
      if (d->top_k < 0 || d->top_k >= (1 << 20) || d->pick_stride < d->top_k) {
        return set_error(SKV_EINVAL, "%s: CSA needs 0 <= top_k <= pick_stride", what);
      }
      comp_keys = d->top_k;
    } else {
      if (d->m < 1 || d->m >= (1 << 24)) return set_error(SKV_EINVAL, "%s: HCA needs m >= 1", what);
      comp_keys = d->max_entries > 0 ? d->max_entries : d->bt_stride * d->block_size;
      if (comp_keys > d->bt_stride * d->block_size) comp_keys = d->bt_stride * d->block_size;
    }
  }
  p.n_hg = static_cast<int>(ceil_div(d->n_heads, kAtHeads));
  p.nks = d->head_dim <= 128 ? 4 : (d->head_dim <= 512 ? 16 : 18);
  const int64_t tiles_c = ceil_div(comp_keys, kAtTile);
  const int64_t tiles_w = ceil_div(d->window, kAtTile);
  int64_t n_cu = tiles_c > 0 ? 1 : 0, n_wu = 1;
  if (d->splits > 0) {
    const int64_t cap_c = kMergeUnits - 1;
    n_cu = tiles_c > 0 ? std::min(std::min<int64_t>(d->splits, tiles_c), cap_c) : 0;
    const int64_t w = n_cu > 0 ? ceil_div(d->splits * 2 * tiles_w, tiles_c + 2 * tiles_w) : d->splits;
    n_wu = std::max<int64_t>(1, std::min(std::min(w, tiles_w), kMergeUnits - n_cu));
  } else {
    // split the branch with the most tiles per unit (a window tile reads K
    // and V) while the grid is short of one workgroup per CU of the device
    // (a CU holds one) and units keep at least 2 tiles' worth of reads
    const int cus = device_cus();
    while (p.rows * p.n_hg * (n_cu + n_wu) < cus && n_cu + n_wu < kMergeUnits) {
      const double pc = n_cu ? static_cast<double>(tiles_c) / n_cu : 0.0;
      const double pw = 2.0 * tiles_w / n_wu;
      if (pc >= pw && pc >= 2.0) {
        ++n_cu;
      } else if (pw >= 2.0 && n_wu < tiles_w) {
        ++n_wu;
      } else {
        break;
      }
    }
  }
  if (d->splits <= 0 && d->kind == SKV_LAYER_CSA && n_wu > 1) {
    // a CSA unit resolves its picks (or ranks them) before its tiles, so
    // window units of two tiles still end before it; fewer units leave the
    // merge fewer partial outputs
    n_wu = std::max<int64_t>(1, std::min<int64_t>(n_wu, ceil_div(tiles_w, 2)));
  }
  if (n_cu + n_wu > kMergeUnits) {
    return set_error(SKV_EINVAL, "%s: at most %d splits per sequence", what, kMergeUnits);
  }
  p.n_cu = static_cast<int>(n_cu);
  p.n_wu = static_cast<int>(n_wu);
  const int64_t units = p.rows * (n_cu + n_wu) * p.n_hg;
  if (units >= (1 << 30)) return set_error(SKV_EINVAL, "%s: too many workgroups", what);
  p.ws_bytes = units * kAtHeads * (2 * static_cast<int64_t>(sizeof(float)) + d->head_dim * 2);  // (max, sum) fp32, O bf16
  return SKV_OK;
}

// The merge launch of a part launch's units (k_attn_merge_q for sequences
// of at most kMergeChunkQ units).
int launch_merge(const AttnArgs& a, const AttnPlan& p, int kind, const float* knorm_w, const float* sink,
                 float* out, hipStream_t s, const char* what) {
  MergeArgs mg;
  mg.part = a.part;
  mg.out = out;
  mg.knorm_w = knorm_w;
  mg.sink = sink;
  mg.H = a.H;
  mg.D = a.D;
  mg.n_hg = p.n_hg;
  mg.n_cu = p.n_cu;
  mg.n_wu = p.n_wu;
  mg.sink_comp = kind == SKV_LAYER_HCA;
  if (p.n_cu + p.n_wu <= kMergeChunkQ) {
    hipLaunchKernelGGL(k_attn_merge_q,
                       dim3(static_cast<unsigned>(a.batch), static_cast<unsigned>(ceil_div(a.H, 4)),
                            static_cast<unsigned>(ceil_div(a.D / 4, kWave))),
                       dim3(256), 0, s, mg);
  } else {
    hipLaunchKernelGGL(k_attn_merge,
                       dim3(static_cast<unsigned>(a.batch), static_cast<unsigned>(ceil_div(a.H, 4)), 2),
                       dim3(256), 0, s, mg);
  }
  return check_launch(what);
}


// ---------------------------------------------------------------------------
// The decode step's last launch with the attention fused in
// (skv_decode_step_attend, one layer).  It takes the place of the step's
// gather launch: a CSA unit ranks its share of the row's top-k candidates
// (the lists the step's filter chunks wrote), writes those positions of the
// top-k row and attends over its picks, read in place through the block
// table; HCA and window units are the attention's own, and a CSA layer has
// one positions unit per sequence besides.  The gather launch's other work
// happens here as well: the first window unit of a sequence commits the
// step (lengths, entry counts, free-stack tops) and the positions unit
// clears the row's top-k histogram for the next step.  No unit reads what
// the commit writes: lengths come from the step's scratch (a.lens is
// step_lens) and an HCA unit's visible count from the length alone.
// ---------------------------------------------------------------------------

// A CSA unit's ranking works in the LDS of the key tiles, which it is done
// with before the first tile is stored: kr holds the candidates' order keys
// (or the full-select fallback's state); vs, which compressed units do not
// use otherwise, holds the compaction's per-wave counts, the unit's picks by
// output position, its keys in output order and the block-table row.
template <int NKS>
struct RankLds {
  static constexpr int kKr = sizeof(AtSmem<NKS>::kr);
  static constexpr int kVs = sizeof(AtSmem<NKS>::vs);
  static constexpr int kCkCap = kKr / 8;  // order keys held in LDS
  static constexpr int kScan = 16;
  static constexpr int kBtCap = (kVs - 4 * (kScan + 2 * kMaxTopK)) / 4;  // block-table entries held in LDS
  static_assert(sizeof(TopkSmemT<kAtThreads>) <= kKr, "full-select fallback state fits the key tile");
  static_assert(kBtCap >= 1024, "block-table row in LDS");
};

constexpr int kPosEmpty = -2147483647 - 1;  // an output position another unit owns

// Ranking of CSA unit `part` of `parts` of sequence b, over the one layer of
// a step: its candidates are the entries at positions part, part + parts,
// ... of each list in canonical order, the list's entries sorted by entry
// index (restored through the run table the filter chunks write), so that
// which picks a unit attends over, and with them its partial output, do not
// depend on the order in which the filter chunks appended to the lists, and
// every unit holds the same share of the sure candidates.  With more filter
// chunks than the run table holds, its candidates are the entries e with
// e % parts == part; with lists longer than LDS holds, the lists' positions
// part, part + parts, ... as written (not reproducible).  Positions
// [part * out, (part + 1) * out), out = ceil(k / parts), are its share of
// the fills (and of the fallback's positions).  On the canonical path a
// unit ranks only its ties (every sure candidate wins); the sure
// candidates' positions come from the sequence's positions unit (positions_unit).
template <int NKS>
struct StepRank {
  static constexpr bool kOn = true;
  using RL = RankLds<NKS>;
  static constexpr int kBtPer = (RL::kBtCap + kAtThreads - 1) / kAtThreads;
  const StepMap& map;
  int32_t* topk_idx;
  int b, part, parts;
  bool lead;  // head group 0: writes the top-k row and clears the histogram
  // the first round trip
  int status = 0, L = 0, cnt0 = 0, cnt1 = 0, flag = 0, n_bt = 0;
  int word = 0;  // lane 0: status, 1: length, 2-4: the lists' counters and tie-overflow flag
  int2 sh, th;
  int4 run;  // the row's run table entry of filter chunk `lane`
  int32_t btv[kBtPer];
  const int32_t* bt_row = nullptr;
  int32_t* ws = nullptr;
  // LDS, from rank()
  const int* keys = nullptr;
  const int32_t* bt_lds = nullptr;
  // sure candidates among the unit's keys whose positions the positions
  // unit writes (the canonical path), ahead of the ranked ones
  int n_sure_keys = 0;
  bool early_bt = false;  // the block-table row went to LDS before the ranking

  // the row's block-table slices (load_bt) into LDS
  __device__ __forceinline__ void put_bt(int32_t* bt) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < kBtPer; ++u) {
      if (u * kAtThreads >= n_bt) break;
      if (tid + u * kAtThreads < n_bt) bt[tid + u * kAtThreads] = btv[u];
    }
  }

  // the layer's group fields, read from the kernel arguments once, at the
  // unit's start (read where they are used, a computed index into the
  // arguments makes them dependent scalar loads on the unit's path)
  int k = 0, m = 1, bs = 1, bt_stride = 1, n_pages = 1;

  __device__ StepRank(const StepMap& m_, int32_t* idx, int b_, int part_, int parts_, bool lead_)
      : map(m_), topk_idx(idx), b(b_), part(part_), parts(parts_), lead(lead_) {
    const int gi = map.group[0];
    k = map.top_k[0];
    m = map.m[gi];
    bs = map.block_size[gi];
    bt_stride = map.bt_stride[gi];
    n_pages = map.n_pages[gi];
  }

  // The ranking's loads, unconditional (clamped indices), ahead of the
  // query's: the heads of both lists, and the status, length and list
  // counters as one load whose lanes read different words.  Loaded as
  // uniform values they would go to scalar registers right after their
  // loads, behind a wait that would hold back the query's loads; read out of
  // lanes in rank(), they are waited for there.
  __device__ __forceinline__ void load() {
    const int tid = threadIdx.x;
    const int gi = map.group[0];
    ws = map.topk_ws[0] + static_cast<int64_t>(b) * kTkWsWords;
    bt_row = map.block_table[gi] + static_cast<int64_t>(b) * bt_stride;
    n_bt = min(bt_stride, RL::kBtCap);
    static_assert(kAtThreads <= kMaxTopK && kAtThreads <= kTkTieCap, "list heads within the lists");
    sh = reinterpret_cast<const int2*>(ws + kTkWsSure)[tid];
    th = reinterpret_cast<const int2*>(ws + kTkWsTie)[tid];
    const int lane = tid % kWave;
    static_assert(kTkRunCap == kWave, "one run table entry per lane");
    run = reinterpret_cast<const int4*>(ws + kTkWsRuns)[lane];
    word = *(lane == 1 ? map.step_lens + b : (lane >= 2 && lane <= 4) ? ws + kTkWsCnt + (lane - 2) : map.status);
  }

  // The row's block-table slices, after the query's loads: they are first
  // needed when the ranking is done, and registers held from the start
  // would be reused (and waited for) by the query's address arithmetic.
  __device__ __forceinline__ void load_bt() {
    const int tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < kBtPer; ++u) {
      if (u * kAtThreads >= n_bt) break;  // uniform: the row's slices only
      btv[u] = bt_row[min(tid + u * kAtThreads, n_bt - 1)];
    }
  }

  // Ranks the unit's candidates and writes its positions of the top-k row
  // (on the canonical path its tie winners' only); returns its key count
  // (its sure candidates first on that path, then its picks >= 0 in output
  // order).  Every thread calls it; the result is uniform.  Its barriers
  // order LDS only, so the query's loads stay in flight through the ranking.
  // On the canonical path, when the unit has a tile's worth of sure
  // candidates and the canonical map fits in the key tile beside the keys,
  // every thread calls early() once the block-table row and the sure
  // candidates are in LDS, before the ties are ranked: the caller resolves
  // the first tile's rows (row()) and issues its loads, which then overlap
  // the ranking.
  template <class Early>
  __device__ __forceinline__ int rank(AtSmem<NKS>& sm, Early&& early) {
    const int tid = threadIdx.x;
    int* scan = reinterpret_cast<int*>(&sm.vs[0][0]);
    int* at_pos = scan + RL::kScan;
    int* key_list = at_pos + kMaxTopK;
    int32_t* bt = key_list + kMaxTopK;
    keys = key_list;
    bt_lds = bt;
    uint64_t* ck = reinterpret_cast<uint64_t*>(&sm.kr[0][0]);
    // Every value of the first round trip is used here, by every wave: a
    // load whose only use sits in a branch that some waves skip stays
    // pending in the compiler's count, and the next write of its register
    // then waits for every load in flight, the query's among them.
    const uint64_t key_sh = order_key(sh), key_th = order_key(th);
    status = __builtin_amdgcn_readlane(word, 0);
    L = __builtin_amdgcn_readlane(word, 1);
    cnt0 = __builtin_amdgcn_readlane(word, 2);
    cnt1 = __builtin_amdgcn_readlane(word, 3);
    flag = __builtin_amdgcn_readlane(word, 4);
    for (int i = tid; i < k; i += kAtThreads) at_pos[i] = kPosEmpty;
    if (__builtin_expect(status != 0, 0)) return 0;  // refused step
    int n_cols, n_valid;
    score_cols(map.score_stride[0], m, L, n_cols, n_valid);
    const int sel = topk_sel(k, n_cols, n_valid);
    const int out = static_cast<int>(ceil_div24(k, parts));
    const int o0 = min(k, part * out), o1 = min(k, o0 + out);
    lds_barrier();
    if (__builtin_expect(sel > 0 && flag, 0)) {
      // tie bin over the list capacity: full select of the row, keeping this
      // unit's positions
      auto& fb = *reinterpret_cast<TopkSmemT<kAtThreads>*>(ck);
      topk_row_emit<kAtThreads>(fb, nullptr, map.scores[0] + static_cast<int64_t>(b) * map.score_stride[0], n_cols,
                                n_valid, k, [&](int j, int v) {
                                  if (j >= o0 && j < o1) at_pos[j] = v;
                                });
    } else if (sel > 0) {
      const int S = min(cnt0, kMaxTopK);
      const int T = min(cnt1, kTkTieCap);
      const int C = S + T;
      const int2* sure_list = reinterpret_cast<const int2*>(ws + kTkWsSure);
      const int2* tie_list = reinterpret_cast<const int2*>(ws + kTkWsTie);
      const bool in_lds = C <= RL::kCkCap;  // uniform
      // Canonical order of a list: its entries sorted by entry index.  Filter
      // chunk c (entries [c * kTkChunk, (c + 1) * kTkChunk)) writes its
      // candidates to one run of slots of each list, sorted by entry index,
      // and records the run's first slot and length in the row's run table;
      // the runs follow each other in the order the chunks reserved them.
      // Slot p of chunk c's run is therefore at canonical position p - first(c)
      // + (the list's entries in the chunks before c); every wave holds that
      // difference of chunk `lane` for both lists, as two 16-bit halves (a
      // scan of the run lengths, both lists' in one word: a list holds fewer
      // than 2^15 entries).
      const int n_ch = static_cast<int>(ceil_div24(static_cast<uint32_t>(n_valid), kTkChunk));
      const bool canon = in_lds && n_ch <= kTkRunCap;  // uniform
      static_assert(kMaxTopK < (1 << 15) && kTkTieCap < (1 << 15), "16-bit run sums and differences");
      int d_pack = 0;
      if (canon) {
        const int lane = tid % kWave;
        const int n2 = lane < n_ch ? (run.y | (run.w << 16)) : 0;
        const int before = wave_prefix_sum(n2) - n2;
        const int d_sure = (before & 0xffff) - run.x, d_tie = (before >> 16) - run.z;
        d_pack = static_cast<int>((static_cast<uint32_t>(d_sure) & 0xffffu) | (static_cast<uint32_t>(d_tie) << 16));
      }
      // canonical position -> slot, each class at its own offset (sure
      // [0, S), ties [S, C)): in the key tile after the keys where it fits
      // (the block-table row then goes to LDS before the ranking, and the
      // first tile of sure keys can be loaded while the ties are ranked),
      // else in the (not yet filled) block-table area
      static_assert(RL::kBtCap >= RL::kCkCap, "canonical map fits the block-table area");
      early_bt = canon && C * 12 <= static_cast<int>(sizeof(sm.kr));  // uniform
      int* slot_at = early_bt ? reinterpret_cast<int*>(ck + C) : bt;
      // the canonical position of slot c holding `key`; every lane of the
      // wave takes part (the lookup reads other lanes' registers)
      const auto canon_pos = [&](int c, uint64_t key) {
        const int ch = static_cast<int>((~static_cast<uint32_t>(key)) / kTkChunk) & (kWave - 1);
        const int d = __shfl(d_pack, ch);
        return c + (c < S ? static_cast<int>(static_cast<int16_t>(d & 0xffff)) : (d >> 16));
      };
      const auto put_slot = [&](int c, int q) {
        if (c < S ? static_cast<unsigned>(q) < static_cast<unsigned>(S)
                  : static_cast<unsigned>(q - S) < static_cast<unsigned>(T)) {
          slot_at[q] = c;
        }
      };
      if (in_lds) {
        if (tid < S) ck[tid] = key_sh;
        if (tid < T) ck[S + tid] = key_th;
        if (canon) {
          const int qs = canon_pos(tid, key_sh), qt = canon_pos(S + tid, key_th);
          if (tid < S) put_slot(tid, qs);
          if (tid < T) put_slot(S + tid, qt);
        }
        if (__builtin_expect(S > kAtThreads || T > kAtThreads, 0)) {  // uniform: the rest of the lists
          constexpr int kLoad = 4;  // list loads in flight per thread
          const int lane = tid % kWave;
          // the trip count is the wave's: canon_pos needs the whole wave
          for (int w0 = tid - lane; w0 < C; w0 += kAtThreads * kLoad) {
            const int c0 = w0 + lane;
            int2 v[kLoad];
#pragma unroll
            for (int u = 0; u < kLoad; ++u) {
              const int c = min(c0 + u * kAtThreads, C - 1);  // unconditional: C >= sel > 0
              v[u] = (c < S ? sure_list : tie_list - S)[c];
            }
#pragma unroll
            for (int u = 0; u < kLoad; ++u) {
              const int c = c0 + u * kAtThreads;
              const bool in_head = c < S ? c < kAtThreads : c - S < kAtThreads;
              // keyed unconditionally: a load used only under a branch that a
              // wave may skip stays pending in the compiler's count, and later
              // register reuse would then wait for every load in flight
              const uint64_t key = order_key(v[u]);
              asm volatile("" ::"v"(key));
              const int q = canon ? canon_pos(c, key) : 0;
              if (c < C && !in_head) {
                ck[c] = key;
                if (canon) put_slot(c, q);
              }
            }
          }
        }
      }
      if (early_bt) put_bt(bt);
      lds_barrier();
      const auto put = [&](int pos, int idx) { at_pos[pos] = idx; };
      if (__builtin_expect(canon, 1)) {
        // canonical positions part, part + parts, ... of each list: the same
        // share of the sure candidates for every unit.  A sure candidate
        // always wins, so only the ties are ranked here; the sure candidates
        // are the unit's first keys, in canonical order, and the positions unit
        // writes their positions of the top-k row (positions_unit).
        const int n_os = part < S ? static_cast<int>(ceil_div24(S - part, parts)) : 0;
        const int n_ot = part < T ? static_cast<int>(ceil_div24(T - part, parts)) : 0;
        const auto own_slot = [&](int cls, int j) {
          return min(max(slot_at[(cls ? S : 0) + part + j * parts], 0), C - 1);
        };
        for (int j = tid; j < n_os; j += kAtThreads) {
          const uint64_t key = ck[own_slot(0, j)];
          key_list[j] = key_finite(static_cast<uint32_t>(key >> 32)) ? static_cast<int>(~static_cast<uint32_t>(key)) : -1;
        }
        n_sure_keys = n_os;
        if (early_bt && n_os >= kAtTile) early();  // uniform; key j of the first tile is this thread's own write
        rank_candidates_of<kAtThreads, 4>(put, [&](int q) { return ck[q]; }, own_slot, 0, n_ot, S, C, sel);
      } else if (in_lds) {
        // more filter chunks than the run table holds: the unit's candidates
        // are the entries e with e % parts == part (its share of the sure
        // candidates then varies), sure ones from the front of the block-table
        // area, ties from its back; their order there is immaterial: each
        // one's position is its rank
        int* own = bt;
        int* own_cnt = scan;  // [0] sure, [1] ties
        if (tid < 2) own_cnt[tid] = 0;
        lds_barrier();
        for (int c = tid; c < C; c += kAtThreads) {
          const uint32_t e = ~static_cast<uint32_t>(ck[c]);
          if (umod24(e, parts) == static_cast<uint32_t>(part)) {
            if (c < S) own[atomicAdd(&own_cnt[0], 1)] = c;
            else own[RL::kBtCap - 1 - atomicAdd(&own_cnt[1], 1)] = c;
          }
        }
        lds_barrier();
        const int n_os = own_cnt[0], n_ot = own_cnt[1];
        rank_candidates_of<kAtThreads, 4>(
            put, [&](int q) { return ck[q]; },
            [&](int cls, int j) { return cls ? own[RL::kBtCap - 1 - j] : own[j]; }, n_os, n_ot, S, C, sel);
      } else {
        rank_candidates<kAtThreads>(put, [&](int q) { return order_key(q < S ? sure_list[q] : tie_list[q - S]); },
                                    S, C, sel, part, parts);
      }
    }
    for (int j = max(o0, sel) + tid; j < o1; j += kAtThreads) at_pos[j] = -1;  // the fills
    lds_barrier();
    // its picks >= 0 become the unit's keys, in output order, after its sure
    // candidates on the canonical path (4 consecutive positions per thread,
    // counts summed over the wave, then over the waves)
    static_assert(4 * kAtThreads >= kMaxTopK, "positions per thread");
    int v[4], cnt = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pos = 4 * tid + i;
      v[i] = pos < k ? at_pos[pos] : kPosEmpty;
      cnt += v[i] >= 0;
    }
    const int lane = tid % kWave, wave = tid / kWave;
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int o = __shfl_up(incl, off);
      if (lane >= off) incl += o;
    }
    if (lane == kWave - 1) scan[wave] = incl;
    lds_barrier();
    int base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kAtWaves; ++w) {
      const int c = scan[w];
      base += w < wave ? c : 0;
      total += c;
    }
    int at = n_sure_keys + base + incl - cnt;  // after the sure keys the ranking left in place
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (v[i] >= 0) key_list[at++] = v[i];
    }
    if (!early_bt) put_bt(bt);
    lds_barrier();
    return n_sure_keys + total;
  }

  // The unit's global stores, after its last loads: every position it owns
  // goes to the top-k row.  Stores issued while loads are in flight would
  // make every later wait for a load wait for all of them (the compiler
  // cannot count on a mix of loads and stores completing in order).
  __device__ __forceinline__ void finish(AtSmem<NKS>& sm) {
    if (!lead) return;
    const int tid = threadIdx.x;
    if (status) return;
    const int* at_pos = reinterpret_cast<const int*>(&sm.vs[0][0]) + RL::kScan;
    for (int pos = tid; pos < k; pos += kAtThreads) {
      const int v = at_pos[pos];
      if (v != kPosEmpty) topk_idx[static_cast<int64_t>(b) * k + pos] = v;
    }
  }

  // Pool row (page * block_size + slot) of key j, or -1.
  __device__ __forceinline__ int64_t row(int j) const {
    const int e = keys[j];
    if (e < 0 || e >= static_cast<int>(udiv24(static_cast<uint32_t>(max(L, 0)), m))) return -1;
    const int pi = static_cast<int>(udiv24(e, bs));
    if (pi >= bt_stride) return -1;
    const int32_t page = pi < n_bt ? bt_lds[pi] : bt_row[pi];
    if (page < 0 || page >= n_pages) return -1;
    return static_cast<int64_t>(page) * bs + (e - pi * bs);
  }
};

// The positions of a CSA row's sure candidates in its top-k row, written by
// positions unit w of n_w of sequence b (one block per sequence beside the
// layer's units, on a CU the attention leaves free; the lists are complete
// when the launch starts): its share is the sure list's slots w, w + n_w,
// ...; a sure candidate's position is the count of sure keys above it.  Only
// where StepRank::rank takes its canonical path (the same conditions from
// the same loads), on which the CSA units rank their ties alone.
template <int NKS>
__device__ __forceinline__ void sure_positions_of(AtSmem<NKS>& sm, const StepMap& map, int32_t* topk_idx, int b,
                                                  int w, int n_w) {
  using RL = RankLds<NKS>;
  const int tid = threadIdx.x;
  const int32_t* ws = map.topk_ws[0] + static_cast<int64_t>(b) * kTkWsWords;
  const int status = *map.status;
  const int L = map.step_lens[b];
  const int cnt0 = ws[kTkWsCnt], cnt1 = ws[kTkWsCnt + 1], flag = ws[kTkWsCnt + 2];
  const int k = map.top_k[0];
  const int m = map.m[map.group[0]];
  if (status != 0 || flag != 0) return;
  int n_cols, n_valid;
  score_cols(map.score_stride[0], m, L, n_cols, n_valid);
  const int sel = topk_sel(k, n_cols, n_valid);
  if (sel == 0) return;
  const int S = min(cnt0, kMaxTopK), T = min(cnt1, kTkTieCap);
  const int n_ch = static_cast<int>(ceil_div24(static_cast<uint32_t>(n_valid), kTkChunk));
  if (S + T > RL::kCkCap || n_ch > kTkRunCap) return;  // the CSA units rank every candidate
  uint64_t* ck = reinterpret_cast<uint64_t*>(&sm.kr[0][0]);
  const int2* sure_list = reinterpret_cast<const int2*>(ws + kTkWsSure);
  for (int c = tid; c < S; c += kAtThreads) ck[c] = order_key(sure_list[c]);
  lds_barrier();
  const int n_own = w < S ? static_cast<int>(ceil_div24(S - w, n_w)) : 0;
  int32_t* row = topk_idx + static_cast<int64_t>(b) * k;
  rank_candidates_of<kAtThreads, 4>([&](int pos, int idx) { row[pos] = idx; }, [&](int q) { return ck[q]; },
                                     [&](int, int j) { return w + j * n_w; }, n_own, 0, S, S, sel);
}

// The positions unit of sequence b: the sure candidates' positions, then
// (also after a refusal, and after its last loads) the row's histogram
// cleared for the next step; nothing in the launch reads the histogram.
template <int NKS>
__device__ __forceinline__ void positions_unit(AtSmem<NKS>& sm, const StepMap& map, int32_t* topk_idx, int b) {
  sure_positions_of<NKS>(sm, map, topk_idx, b, 0, 1);
  int32_t* ws = map.topk_ws[0] + static_cast<int64_t>(b) * kTkWsWords;
  for (int i = threadIdx.x; i < kTkBins; i += kAtThreads) ws[kTkWsHist + i] = 0;
}

// The step's commit for sequence b (after a refusal: nothing).
__device__ __forceinline__ void step_commit(const StepMap& map, int b) {
  if (*map.status) return;
  const int L = map.step_lens[b];
  map.tok_lens[b] = L;
  for (int g = 0; g < map.n_groups; ++g) map.n_entries[g][b] = udiv24(static_cast<uint32_t>(L), map.m[g]);
  if (b == 0) {
    for (int g = 0; g < map.n_groups; ++g) *map.free_top[g] = map.step_top[g];
  }
}

// Units as k_attn_part places them.
template <int NKS, bool kFp8>
__global__ __launch_bounds__(kAtThreads, 1) void k_decode_attend(AttnArgs a, StepMap map, int32_t* topk_idx) {
  __shared__ AtSmem<NKS> sm;
  const int U = a.n_cu + a.n_wu;
  // a CSA layer's sequences have one more block: the positions unit
  const int per_seq = U * a.n_hg + (a.kind == SKV_LAYER_CSA ? 1 : 0);
  const int xs = __builtin_ctz(static_cast<uint32_t>(a.xcds));  // a.xcds is a power of two
  const int k = static_cast<int>(blockIdx.x) >> xs;
  const int sb = k / per_seq;
  const int b = (static_cast<int>(blockIdx.x) & (a.xcds - 1)) + (sb << xs);
  if (b >= a.batch) return;  // uniform
  const int r = k - sb * per_seq;
  if constexpr (NKS >= 16) {
    if (r == U * a.n_hg) {  // the positions unit (CSA layers only)
      positions_unit<NKS>(sm, map, topk_idx, b);
      return;
    }
  }
  const int u = r / a.n_hg, hg = r - u * a.n_hg;
  const int64_t unit = (static_cast<int64_t>(b) * U + u) * a.n_hg + hg;
  if (u < a.n_cu) {
    if constexpr (NKS >= 16) {  // the host refuses a CSA layer of head_dim <= 128
      if (a.kind == SKV_LAYER_CSA) {
        attn_unit<NKS, kFp8, true>(sm, a, b, 0, 1, hg, unit, StepRank<NKS>(map, topk_idx, b, u, a.n_cu, hg == 0));
        return;
      }
    }
    attn_unit<NKS, kFp8, true>(sm, a, b, u, a.n_cu, hg, unit);
  } else {
    if (u == a.n_cu && hg == 0 && threadIdx.x == 0) step_commit(map, b);
    attn_unit<NKS, false, false>(sm, a, b, u - a.n_cu, a.n_wu, hg, unit);
  }
}

int decode_attend(const skv_attention_desc* d, const skv_decode_desc* h, const StepMap* map, void* workspace,
                  int64_t ws_bytes, hipStream_t s, int64_t* ws_need, bool call) {
  const char* what = "skv_decode_step_attend";
  if (!d) return set_error(SKV_EINVAL, "%s: NULL attention descriptor", what);
  if (h->n_layers != 1) return set_error(SKV_EINVAL, "%s: the step must have exactly one layer", what);
  const skv_decode_layer& Ly = h->layers[0];
  if (Ly.out_entries || Ly.out_window) {
    return set_error(SKV_EINVAL, "%s: the layer must not write gathered copies (out_entries / out_window)", what);
  }
  if (d->head_dim != h->latent || d->batch != h->batch) {
    return set_error(SKV_EINVAL, "%s: head_dim must equal the step's latent and batch its batch", what);
  }
  const bool comp = Ly.kind != SKV_LAYER_SWA;
  if (comp && (Ly.group < 0 || Ly.group >= h->n_groups)) return set_error(SKV_EINVAL, "%s: layer group out of range", what);
  if (Ly.kind == SKV_LAYER_CSA && d->head_dim <= 128) {
    return set_error(SKV_EINVAL, "%s: a CSA layer needs head_dim > 128", what);
  }
  // the attention over the step's own cache
  skv_attention_desc x = *d;
  x.kind = Ly.kind;
  x.format = Ly.format;
  x.lens = h->step_lens;
  x.win_k = Ly.ring;
  if (!x.win_v) x.win_v = Ly.ring;
  x.window = h->window;
  if (d->n_queries > 1 || d->ring > 0 || d->win_stride > 0) {
    return set_error(SKV_EINVAL, "%s: one query token per sequence over the layer's ring (n_queries 0 or 1, "
                     "ring and win_stride 0)", what);
  }
  x.n_queries = 1;
  x.ring = h->window;
  if (comp) {
    const skv_page_group& G = h->groups[Ly.group];
    x.pool = Ly.pool;
    x.entry_bytes = Ly.entry_bytes;
    x.block_size = G.block_size;
    x.n_pages = G.n_pages;
    x.block_table = G.block_table;
    x.bt_stride = G.bt_stride;
    x.n_entries = G.n_entries;
    x.m = G.m;
    if (Ly.kind == SKV_LAYER_CSA) {
      x.picks = Ly.topk_idx;
      x.pick_stride = Ly.top_k;
      x.top_k = Ly.top_k;
    }
  }
  AttnPlan p;
  int rc = attn_plan(&x, p);
  if (rc != SKV_OK) return rc;
  if (ws_need) *ws_need = p.ws_bytes;
  if (!call) return SKV_OK;
  if (!x.q || !x.out || (comp && !x.knorm_w)) return set_error(SKV_EINVAL, "%s: NULL q/out/knorm_w", what);
  if (!workspace || ws_bytes < p.ws_bytes) {
    return set_error(SKV_EINVAL, "%s: workspace of %lld bytes needed", what, (long long)p.ws_bytes);
  }
  if (reinterpret_cast<uintptr_t>(workspace) & 15) {
    return set_error(SKV_EINVAL, "%s: workspace must be 16-byte aligned", what);
  }
  if (!map) return SKV_OK;
  AttnArgs a;
  a.q = static_cast<const uint8_t*>(x.q);
  a.part = static_cast<float*>(workspace);
  a.lens = x.lens;
  a.pool = static_cast<const uint8_t*>(x.pool);
  a.block_table = x.block_table;
  a.n_entries = x.n_entries;
  a.picks = x.picks;
  a.knorm_w = x.knorm_w;
  a.win_k = static_cast<const uint8_t*>(x.win_k);
  a.win_v = static_cast<const uint8_t*>(x.win_v);
  a.entry_bytes = comp ? x.entry_bytes : 0;
  a.pick_stride = x.pick_stride;
  a.kind = x.kind;
  a.fp8_main = comp && x.format == SKV_FMT_FP8 ? entry_layout(x.format, x.head_dim, x.entry_bytes) : 0;
  a.block_size = static_cast<int32_t>(comp ? x.block_size : 1);
  a.n_pages = static_cast<int32_t>(comp ? x.n_pages : 1);
  a.bt_stride = static_cast<int32_t>(comp ? x.bt_stride : 1);
  a.m = static_cast<int32_t>(x.kind == SKV_LAYER_HCA ? x.m : 1);
  a.top_k = static_cast<int32_t>(x.kind == SKV_LAYER_CSA ? x.top_k : 0);
  a.window = static_cast<int32_t>(x.window);
  a.H = static_cast<int32_t>(x.n_heads);
  a.D = static_cast<int32_t>(x.head_dim);
  a.n_hg = p.n_hg;
  a.n_cu = p.n_cu;
  a.n_wu = p.n_wu;
  a.batch = static_cast<int32_t>(x.batch);
  a.n_q = 1;
  a.ring = static_cast<int32_t>(x.window);
  a.win_row = x.head_dim * 2;
  a.eps = x.eps;
  a.softcap = x.softcap;
  a.fused = 1;
  a.xcds = device_xcds();
  const dim3 grid(static_cast<unsigned>(a.xcds * ceil_div(x.batch, a.xcds) *
                                        ((p.n_cu + p.n_wu) * p.n_hg + (x.kind == SKV_LAYER_CSA ? 1 : 0))));
  int32_t* idx = Ly.kind == SKV_LAYER_CSA ? Ly.topk_idx : nullptr;
  if (a.fp8_main > 0) {
    hipLaunchKernelGGL((k_decode_attend<18, true>), grid, dim3(kAtThreads), 0, s, a, *map, idx);
  } else if (p.nks == 4) {
    hipLaunchKernelGGL((k_decode_attend<4, false>), grid, dim3(kAtThreads), 0, s, a, *map, idx);
  } else if (p.nks == 16) {
    hipLaunchKernelGGL((k_decode_attend<16, false>), grid, dim3(kAtThreads), 0, s, a, *map, idx);
  } else {
    hipLaunchKernelGGL((k_decode_attend<18, false>), grid, dim3(kAtThreads), 0, s, a, *map, idx);
  }
  if ((rc = check_launch(what))) return rc;
  return launch_merge(a, p, x.kind, comp ? x.knorm_w : nullptr, x.sink, x.out, s, what);
}
}  // namespace skv

using namespace skv;

extern "C" int64_t skv_attention_desc_size(void) { return static_cast<int64_t>(sizeof(skv_attention_desc)); }

extern "C" int64_t skv_attention_workspace(const skv_attention_desc* d) {
  AttnPlan p;
  if (attn_plan(d, p) != SKV_OK) return -1;
  return p.ws_bytes;
}

extern "C" int skv_decode_attention(const skv_attention_desc* d, void* workspace, int64_t ws_bytes,
                                    void* stream) {
  const char* what = "skv_decode_attention";
  AttnPlan p;
  int rc = attn_plan(d, p);
  if (rc != SKV_OK) return rc;
  if (d->batch == 0) return SKV_OK;
  const bool comp = d->kind != SKV_LAYER_SWA;
  if (!d->q || !d->out || !d->lens || !d->win_k || !d->win_v ||
      (comp && (!d->pool || !d->block_table || !d->n_entries || !d->knorm_w)) ||
      (d->kind == SKV_LAYER_CSA && !d->picks)) {
    return set_error(SKV_EINVAL, "%s: NULL pointer", what);
  }
  if (!workspace || ws_bytes < p.ws_bytes) {
    return set_error(SKV_EINVAL, "%s: workspace of %lld bytes needed", what, (long long)p.ws_bytes);
  }
  if (reinterpret_cast<uintptr_t>(workspace) & 15) {
    return set_error(SKV_EINVAL, "%s: workspace must be 16-byte aligned (the merge reads it in vectors)", what);
  }
  AttnArgs a;
  a.q = static_cast<const uint8_t*>(d->q);
  a.part = static_cast<float*>(workspace);
  a.lens = d->lens;
  a.pool = static_cast<const uint8_t*>(d->pool);
  a.block_table = d->block_table;
  a.n_entries = d->n_entries;
  a.picks = d->picks;
  a.knorm_w = d->knorm_w;
  a.win_k = static_cast<const uint8_t*>(d->win_k);
  a.win_v = static_cast<const uint8_t*>(d->win_v);
  a.entry_bytes = comp ? d->entry_bytes : 0;
  a.pick_stride = d->pick_stride;
  a.kind = d->kind;
  a.fp8_main = comp && d->format == SKV_FMT_FP8 ? entry_layout(d->format, d->head_dim, d->entry_bytes) : 0;
  a.block_size = static_cast<int32_t>(comp ? d->block_size : 1);
  a.n_pages = static_cast<int32_t>(comp ? d->n_pages : 1);
  a.bt_stride = static_cast<int32_t>(comp ? d->bt_stride : 1);
  a.m = static_cast<int32_t>(d->kind == SKV_LAYER_HCA ? d->m : 1);
  a.top_k = static_cast<int32_t>(d->kind == SKV_LAYER_CSA ? d->top_k : 0);
  a.window = static_cast<int32_t>(d->window);
  a.H = static_cast<int32_t>(d->n_heads);
  a.D = static_cast<int32_t>(d->head_dim);
  a.n_hg = p.n_hg;
  a.n_cu = p.n_cu;
  a.n_wu = p.n_wu;
  a.batch = static_cast<int32_t>(p.rows);
  a.n_q = static_cast<int32_t>(p.nq);
  a.ring = static_cast<int32_t>(p.ring);
  a.win_row = p.win_row;
  a.eps = d->eps;
  a.softcap = d->softcap;
  a.fused = 0;
  a.xcds = device_xcds();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(a.xcds * ceil_div(p.rows, a.xcds) * (p.n_cu + p.n_wu) * p.n_hg));
  if (a.fp8_main > 0) {
    hipLaunchKernelGGL((k_attn_part<18, true>), grid, dim3(kAtThreads), 0, s, a);
  } else if (p.nks == 4) {
    hipLaunchKernelGGL((k_attn_part<4, false>), grid, dim3(kAtThreads), 0, s, a);
  } else if (p.nks == 16) {
    hipLaunchKernelGGL((k_attn_part<16, false>), grid, dim3(kAtThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((k_attn_part<18, false>), grid, dim3(kAtThreads), 0, s, a);
  }
  if ((rc = check_launch(what))) return rc;
  return launch_merge(a, p, d->kind, comp ? d->knorm_w : nullptr, d->sink, d->out, s, what);
}
