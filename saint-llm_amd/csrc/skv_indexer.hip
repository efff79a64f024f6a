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
// The tile (MFMA mapping, operand staging) is in skv_indexer_tile.h.
#include "skv_common.h"
#include "skv_indexer_tile.h"

namespace skv {

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

// One workgroup per (tile of kIdxTile entries, query row).
__global__ __launch_bounds__(kIdxThreads, 2) void k_indexer_scores(IndexerArgs a) {
  __shared__ IndexerSmem sm;
  const int row = blockIdx.y;  // query row
  const int b = static_cast<int>(udiv24(row, a.t_per_seq));
  const IndexerRow r{a.q + static_cast<int64_t>(row) * a.n_heads * a.c * 2,
                     a.w + static_cast<int64_t>(row) * a.n_heads,
                     a.pool,
                     a.block_table + static_cast<int64_t>(b) * a.bt_stride,
                     a.bt_stride,
                     a.block_size,
                     a.n_pages,
                     a.n_heads,
                     a.c};
  float* out = a.scores + static_cast<int64_t>(row) * a.score_stride;
  indexer_tile(
      sm, r, static_cast<int>(blockIdx.x),
      [&] { return min(a.n_entries[b], a.max_entries); },  // the grid covers max_entries
      [&](int e, float v) { out[e] = v; });
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
