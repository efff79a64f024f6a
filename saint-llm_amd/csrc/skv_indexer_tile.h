// One workgroup's tile of lightning-indexer scores: kIdxTile consecutive
// compressed entries of one query row.  Shared by skv_indexer_scores and the
// decode step, whose first launch computes each CSA layer's scores fused
// with the top-k histogram.
//
// Reference: lightning_indexer_scores_reference (kernels/attention.py:33-50)
// and CSA._indexer_topk_cached (csa.py:405-409):
//   scores[s] = sum_h w[h] * ReLU(q[h, :] . k[s, :]).
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, D[16 x 16] += A[16 x 32] B[32 x 16]):
// A = 16 heads x 32 channels of the query, B = 32 channels x 16 entries, D =
// 16 heads x 16 entries.  Lane l holds A row l%16, channels 8*(l/16)..+7;
// B column l%16, channels 8*(l/16)..+7; D rows 4*(l/16)+i, column l%16.
// The query row sits in LDS and is read as A operands; each lane loads its
// entries' 16-byte channel chunks straight from the pool into B operands
// (all of a wave's keys in flight at once), so the keys are read once.  The
// epilogue applies ReLU and the head weights to D and sums the heads across
// the four lane groups.
#pragma once

#include "skv_common.h"

namespace skv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kIdxThreads = 256;
constexpr int kIdxWaves = kIdxThreads / kWave;
constexpr int kIdxCols = 8;                           // 16-entry column blocks per wave
constexpr int kIdxTile = kIdxWaves * kIdxCols * 16;  // entries per workgroup
constexpr int kIdxMaxHB = 4;                          // head blocks of 16 (up to 64 heads)
constexpr int kIdxMaxKS = 4;                          // k-steps of 32 channels (up to 128 channels)
constexpr int kIdxQRow = 32 * kIdxMaxKS + 8;          // LDS row of a query head, bf16 (16 bytes of pad)

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// The query row in LDS, heads padded to 64 and channels to 128 with zeros;
// rows of 272 bytes put the 16 lanes that read one A operand on distinct banks.
struct IndexerSmem {
  alignas(16) uint16_t q[16 * kIdxMaxHB][kIdxQRow];
};

// One query row's operands.
struct IndexerRow {
  const uint8_t* q;       // [n_heads, c] bf16
  const float* w;         // [n_heads]
  const uint8_t* pool;    // [n_pages, block_size, c] bf16
  const int32_t* bt_row;  // the sequence's block-table row
  int bt_stride, block_size, n_pages, n_heads, c;
};

// Scores of entries [tile * kIdxTile, +kIdxTile) below count(): out(e, v) is
// called once per entry e < count() (by lane group 0 of the wave holding
// it), v = -inf for an entry whose page is not mapped.  count() is called
// after the first memory round trip's loads are issued (the block-table
// slots, the query and the weights), so that its own loads overlap them.
// Returns false (uniformly, before any barrier) when the tile lies past the
// count; otherwise every thread passes one __syncthreads.
template <class Count, class Out>
__device__ __forceinline__ bool indexer_tile(IndexerSmem& sm, const IndexerRow& r, int tile, Count count,
                                             Out out) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int col = lane & 15, grp = lane >> 4;
  const int e0 = tile * kIdxTile + (tid / kWave) * (kIdxCols * 16) + col;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  // first round trip (unconditional loads, clamped addresses)
  int pi[kIdxCols], page[kIdxCols];
#pragma unroll
  for (int j = 0; j < kIdxCols; ++j) {
    pi[j] = static_cast<int>(udiv24(e0 + 16 * j, r.block_size));
    page[j] = r.bt_row[min(pi[j], r.bt_stride - 1)];
  }
  constexpr int kQChunks = 16 * kIdxMaxHB * (32 * kIdxMaxKS / 8);  // 16-byte pieces of the padded query
  u32x4 qv[kQChunks / kIdxThreads];
#pragma unroll
  for (int u = 0; u < kQChunks / kIdxThreads; ++u) {
    const int piece = tid + u * kIdxThreads;
    const int h = piece / (32 * kIdxMaxKS / 8), ch = (piece % (32 * kIdxMaxKS / 8)) * 8;
    const bool live = h < r.n_heads && ch < r.c;
    const u32x4 v = *reinterpret_cast<const u32x4*>(live ? r.q + (static_cast<int64_t>(h) * r.c + ch) * 2 : r.q);
    qv[u] = live ? v : zero4;
  }
  float wv[kIdxMaxHB][4];
#pragma unroll
  for (int hb = 0; hb < kIdxMaxHB; ++hb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = hb * 16 + grp * 4 + i;
      const float v = r.w[min(h, r.n_heads - 1)];
      wv[hb][i] = h < r.n_heads ? v : 0.f;
    }
  }
  const int n_ent = count();
  if (tile * kIdxTile >= n_ent) return false;  // uniform: the tile lies past the entries
  // the query to LDS before the keys are requested: the barrier waits for
  // every load issued before it
#pragma unroll
  for (int u = 0; u < kQChunks / kIdxThreads; ++u) {
    const int piece = tid + u * kIdxThreads;
    const int h = piece / (32 * kIdxMaxKS / 8), ch = (piece % (32 * kIdxMaxKS / 8)) * 8;
    *reinterpret_cast<u32x4*>(&sm.q[h][ch]) = qv[u];
  }
  __syncthreads();
  // second round trip: every key of the wave's entries (zero for entries past
  // the count or unmapped, and past the channels); each block is multiplied
  // as soon as its keys arrive
  bool ok[kIdxCols];
  u32x4 kb[kIdxCols][kIdxMaxKS];
#pragma unroll
  for (int j = 0; j < kIdxCols; ++j) {
    const int e = e0 + 16 * j;
    ok[j] = e < n_ent && pi[j] < r.bt_stride && page[j] >= 0 && page[j] < r.n_pages;
    const uint8_t* src =
        r.pool + ((static_cast<int64_t>(ok[j] ? page[j] : 0) * r.block_size + (e - pi[j] * r.block_size)) * r.c) * 2;
#pragma unroll
    for (int ks = 0; ks < kIdxMaxKS; ++ks) {
      const int ch = ks * 32 + grp * 8;
      const bool live = ok[j] && ch < r.c;
      const u32x4 v = *reinterpret_cast<const u32x4*>(live ? src + ch * 2 : r.pool);
      kb[j][ks] = live ? v : zero4;
    }
  }
#pragma unroll
  for (int j = 0; j < kIdxCols; ++j) {
    f32x4 acc[kIdxMaxHB];
#pragma unroll
    for (int hb = 0; hb < kIdxMaxHB; ++hb) acc[hb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // heads and channels past the row's are zero in both operands: the full
    // 64 x 128 product is computed, branch-free
#pragma unroll
    for (int ks = 0; ks < kIdxMaxKS; ++ks) {
      const bf16x8 kv = as_bf16x8(kb[j][ks]);
#pragma unroll
      for (int hb = 0; hb < kIdxMaxHB; ++hb) {
        const bf16x8 qa = as_bf16x8(*reinterpret_cast<const u32x4*>(&sm.q[hb * 16 + col][ks * 32 + grp * 8]));
        acc[hb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa, kv, acc[hb], 0, 0, 0);
      }
    }
    float v = 0.f;
#pragma unroll
    for (int hb = 0; hb < kIdxMaxHB; ++hb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v += wv[hb][i] * fmaxf(acc[hb][i], 0.f);
    }
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    const int e = e0 + 16 * j;
    if (grp == 0 && e < n_ent) out(e, ok[j] ? v : -__builtin_huge_valf());
  }
  return true;
}

}  // namespace skv
