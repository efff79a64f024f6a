// Lightning-indexer block scores over the paged compressed indexer keys.
//
// Reference: lightning_indexer_scores_reference (kernels/attention.py:33-50)
// and the cached decode path CSA._indexer_topk_cached (csa.py:405-409):
//   head_scores[b,t,h,s] = ReLU(q[b,t,h,:] . k[b,s,:])
//   scores[b,t,s]        = sum_h w[b,t,h] * head_scores[b,t,h,s]
// The head axis is reduced on the fly; no (B, T, H, S) tensor is formed.  The
// scores are unmasked (the top-k applies the causal block mask); the cached
// path takes no visual bias (csa.py:396-399) and neither does this kernel.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, D[16 x 16] += A[16 x 32] B[32 x 16]):
// A = 16 heads x 32 channels of the query, B = 32 channels x 16 entries, D =
// 16 heads x 16 entries.  Lane l holds A row l%16, channels 8*(l/16)..+7;
// B column l%16, channels 8*(l/16)..+7; D rows 4*(l/16)+i, column l%16.
// The workgroup's query row sits in LDS and is read as A operands; each
// lane loads its entries' 16-byte channel chunks straight from the pool into
// B operands (all of a wave's keys in flight at once), so the keys are read
// once, 64 bytes per entry per load.  The epilogue applies ReLU and the head
// weights to D and sums the heads across the four lane groups.
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

struct IndexerArgs {
  const uint8_t* q;  // [rows, H, c] bf16, rows = batch * t_per_seq
  const float* w;    // [rows, H]
  const uint8_t* pool;  // [n_pages, block_size, c] bf16
  const int32_t* block_table;
  const int32_t* n_entries;
  float* scores;  // [rows, score_stride]
  int64_t score_stride;
  int32_t bt_stride;
  int32_t n_heads, c, block_size, n_pages, t_per_seq, max_entries;
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// The query row in LDS, heads padded to 64 and channels to 128 with zeros;
// rows of 272 bytes put the 16 lanes that read one A operand on distinct banks.
struct IndexerSmem {
  alignas(16) uint16_t q[16 * kIdxMaxHB][kIdxQRow];
};

// Each wave scores kIdxCols blocks of 16 entries.  All of their keys are
// loaded at once into registers (32 KB of loads in flight per wave), the
// query comes from LDS as A operands.
__global__ __launch_bounds__(kIdxThreads, 2) void k_indexer_scores(IndexerArgs a) {
  __shared__ IndexerSmem sm;
  const int row = blockIdx.y;  // query row
  const int b = static_cast<int>(udiv24(row, a.t_per_seq));
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int col = lane & 15, grp = lane >> 4;
  const int e0 = blockIdx.x * kIdxTile + (tid / kWave) * (kIdxCols * 16) + col;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  // first round trip: the entry count, the entries' block-table slots, the
  // query row (to LDS) and the head weights (unconditional loads, clamped
  // addresses)
  const int n_ent = min(a.n_entries[b], a.max_entries);  // the grid covers max_entries
  const int32_t* bt_row = a.block_table + static_cast<int64_t>(b) * a.bt_stride;
  int pi[kIdxCols], page[kIdxCols];
#pragma unroll
  for (int j = 0; j < kIdxCols; ++j) {
    pi[j] = static_cast<int>(udiv24(e0 + 16 * j, a.block_size));
    page[j] = bt_row[min(pi[j], a.bt_stride - 1)];
  }
  const uint8_t* qrow = a.q + static_cast<int64_t>(row) * a.n_heads * a.c * 2;
  constexpr int kQChunks = 16 * kIdxMaxHB * (32 * kIdxMaxKS / 8);  // 16-byte pieces of the padded query
  u32x4 qv[kQChunks / kIdxThreads];
#pragma unroll
  for (int u = 0; u < kQChunks / kIdxThreads; ++u) {
    const int piece = tid + u * kIdxThreads;
    const int h = piece / (32 * kIdxMaxKS / 8), ch = (piece % (32 * kIdxMaxKS / 8)) * 8;
    const bool live = h < a.n_heads && ch < a.c;
    const u32x4 v = *reinterpret_cast<const u32x4*>(live ? qrow + (static_cast<int64_t>(h) * a.c + ch) * 2 : qrow);
    qv[u] = live ? v : zero4;
  }
  float wv[kIdxMaxHB][4];
#pragma unroll
  for (int hb = 0; hb < kIdxMaxHB; ++hb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = hb * 16 + grp * 4 + i;
      const float v = a.w[static_cast<int64_t>(row) * a.n_heads + min(h, a.n_heads - 1)];
      wv[hb][i] = h < a.n_heads ? v : 0.f;
    }
  }
  if (blockIdx.x * kIdxTile >= n_ent) return;  // uniform: the tile lies past the entries
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
    ok[j] = e < n_ent && pi[j] < a.bt_stride && page[j] >= 0 && page[j] < a.n_pages;
    const uint8_t* src =
        a.pool + ((static_cast<int64_t>(ok[j] ? page[j] : 0) * a.block_size + (e - pi[j] * a.block_size)) * a.c) * 2;
#pragma unroll
    for (int ks = 0; ks < kIdxMaxKS; ++ks) {
      const int ch = ks * 32 + grp * 8;
      const bool live = ok[j] && ch < a.c;
      const u32x4 v = *reinterpret_cast<const u32x4*>(live ? src + ch * 2 : a.pool);
      kb[j][ks] = live ? v : zero4;
    }
  }
  float* out = a.scores + static_cast<int64_t>(row) * a.score_stride;
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
    if (grp == 0 && e < n_ent) out[e] = ok[j] ? v : -__builtin_huge_valf();
  }
}

}  // namespace skv

using namespace skv;

extern "C" int skv_indexer_scores(const void* q, const float* w, const void* idx_pool, int64_t block_size,
                                  int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                                  const int32_t* n_entries, float* scores, int64_t score_stride,
                                  int64_t batch, int64_t t_per_seq, int64_t n_heads, int64_t channels,
                                  int64_t max_entries, void* stream) {
  const char* what = "skv_indexer_scores";
  if (batch < 0 || t_per_seq < 0 || max_entries < 0) return set_error(SKV_EINVAL, "%s: negative size", what);
  if (batch == 0 || t_per_seq == 0 || max_entries == 0) return SKV_OK;
  if (!q || !w || !idx_pool || !block_table || !n_entries || !scores) {
    return set_error(SKV_EINVAL, "%s: NULL pointer", what);
  }
  if (n_heads < 1 || n_heads > 16 * kIdxMaxHB) {
    return set_error(SKV_EINVAL, "%s: n_heads must be in [1, %d]; got %lld", what, 16 * kIdxMaxHB,
                     (long long)n_heads);
  }
  if (channels < 8 || channels > 32 * kIdxMaxKS || channels % 8) {
    return set_error(SKV_EINVAL, "%s: channels must be a multiple of 8 in [8, %d]; got %lld", what,
                     32 * kIdxMaxKS, (long long)channels);
  }
  if (block_size <= 0 || n_pages <= 0 || n_pages > 0x7fffffff || bt_stride <= 0 || bt_stride >= (1 << 24)) {
    return set_error(SKV_EINVAL, "%s: bad page geometry", what);
  }
  if (max_entries > score_stride || max_entries >= (1 << 24) - kIdxTile) {
    return set_error(SKV_EINVAL, "%s: max_entries must be <= score_stride and < 2^24", what);
  }
  const int64_t rows = batch * t_per_seq;
  if (rows > 65535 || batch >= (1 << 24)) return set_error(SKV_EINVAL, "%s: at most 65535 query rows", what);
  IndexerArgs a;
  a.q = static_cast<const uint8_t*>(q);
  a.w = w;
  a.pool = static_cast<const uint8_t*>(idx_pool);
  a.block_table = block_table;
  a.n_entries = n_entries;
  a.scores = scores;
  a.score_stride = score_stride;
  a.bt_stride = static_cast<int32_t>(bt_stride);
  a.n_heads = static_cast<int32_t>(n_heads);
  a.c = static_cast<int32_t>(channels);
  a.block_size = static_cast<int32_t>(block_size);
  a.n_pages = static_cast<int32_t>(n_pages);
  a.t_per_seq = static_cast<int32_t>(t_per_seq);
  a.max_entries = static_cast<int32_t>(max_entries);
  const dim3 grid(static_cast<unsigned>(ceil_div(max_entries, kIdxTile)), static_cast<unsigned>(rows));
  hipLaunchKernelGGL(k_indexer_scores, grid, dim3(kIdxThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch(what);
}
