// Top-k block selection over fp32 indexer scores and the block-table gather
// of the selected compressed entries (with optional FP8 -> bf16 dequant).
//
// Reference semantics:
//   CSA._indexer_topk_cached (csa.py:411-422), kernels/attention.py:53-89:
//     scores[s] = -inf where s*m + m - 1 >= q_pos (causal block mask)
//     k_eff = min(top_k, n_blocks); topk(k_eff) sorted descending;
//     picks whose score is not finite become -1.
//   Sparse gather (csa.py:326-331): idx.clamp(min=0) then torch.gather, so a
//   -1 pick copies entry 0 (masked later by the consumer).
//   dequant_from_fp8 (quant/reference.py:114-116): code * scale, then bf16.
// Order of equal scores: ascending index (a total order; torch leaves ties
// unspecified).
#include "skv_topk.h"

namespace skv {

struct TopkArgs {
  const float* scores;
  int64_t stride;
  const int32_t* n_valid;
  const int32_t* n_cols;
  int n_cols_uni;
  const int32_t* lens;  // decode mode: n_cols = L/m, n_valid = (L-1)/m
  int m;
  int k;
  int32_t* out;
  int64_t out_stride;
};

__global__ __launch_bounds__(kTopkThreads) void k_topk_select(TopkArgs a) {
  __shared__ TopkSmem sm;
  __shared__ uint32_t keys[kLdsKeys];
  const int r = blockIdx.x;
  int n_cols, n_valid;
  if (a.lens) {
    const int L = max(a.lens[r], 0);
    n_cols = L / a.m;
    n_valid = L > 0 ? (L - 1) / a.m : 0;
  } else {
    n_cols = a.n_cols ? a.n_cols[r] : a.n_cols_uni;
    n_valid = a.n_valid[r];
  }
  topk_row(sm, keys, a.scores + r * a.stride, n_cols, n_valid, a.k, a.out + r * a.out_stride);
}

// Multi-workgroup form: hist and filter over grid (chunks, rows), final over
// grid (rows); workspace kTkWsWords int32 per row.
struct TopkMultiArgs {
  TopkArgs a;
  int32_t* ws;
};

__device__ __forceinline__ void topk_row_dims(const TopkArgs& a, int r, int& n_cols, int& n_valid) {
  if (a.lens) {
    const int L = max(a.lens[r], 0);
    n_cols = L / a.m;
    n_valid = L > 0 ? (L - 1) / a.m : 0;
  } else {
    n_cols = a.n_cols ? a.n_cols[r] : a.n_cols_uni;
    n_valid = a.n_valid[r];
  }
}

__global__ __launch_bounds__(kTkPartThreads) void k_topk_hist(TopkMultiArgs m) {
  __shared__ TopkHistSmem sm;
  const int r = blockIdx.y;
  int n_cols, n_valid;
  topk_row_dims(m.a, r, n_cols, n_valid);
  topk_hist_chunk(sm, m.a.scores + r * m.a.stride, n_cols, n_valid, m.a.k, blockIdx.x,
                  m.ws + static_cast<int64_t>(r) * kTkWsWords);
}

__global__ __launch_bounds__(kTkPartThreads) void k_topk_filter(TopkMultiArgs m) {
  __shared__ TopkFilterSmem sm;
  const int r = blockIdx.y;
  int n_cols, n_valid;
  topk_row_dims(m.a, r, n_cols, n_valid);
  topk_filter_chunk(sm, m.a.scores + r * m.a.stride, n_cols, n_valid, m.a.k, blockIdx.x,
                    m.ws + static_cast<int64_t>(r) * kTkWsWords);
}

__global__ __launch_bounds__(kTopkThreads) void k_topk_final(TopkMultiArgs m) {
  __shared__ TopkFinalSmem sm;
  const int r = blockIdx.x;
  int n_cols, n_valid;
  topk_row_dims(m.a, r, n_cols, n_valid);
  topk_final_row(sm, m.a.scores + r * m.a.stride, n_cols, n_valid, m.a.k,
                 m.ws + static_cast<int64_t>(r) * kTkWsWords, m.a.out + r * m.a.out_stride);
}

// ---------------------------------------------------------------------------
// Gather of selected entries through the block table.
// ---------------------------------------------------------------------------
constexpr int kGatherThreads = 256;
constexpr int kGatherEntries = 8;

struct TopkGatherArgs {
  uint8_t* dst;
  const uint8_t* pool;
  int64_t entry_bytes;
  int bs;
  int64_t n_pages;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* n_entries;
  const int32_t* idx;
  int64_t idx_stride;
  int k;
  const int32_t* row_seq;
  int channels;
  int format;
  int fp8_main;
  int64_t out_row_bytes;
};

// Entry address of pick j of row r, or nullptr when no entry exists.
__device__ __forceinline__ const uint8_t* pick_entry(const TopkGatherArgs& a, int r, int j) {
  const int b = a.row_seq ? a.row_seq[r] : r;
  int e = a.idx[r * a.idx_stride + j];
  if (e < 0) e = 0;  // clamp(min=0): a -1 pick reads entry 0
  const int n_ent = a.n_entries[b];
  if (e >= n_ent) return nullptr;
  const int64_t p = e / a.bs;
  if (p >= a.bt_stride) return nullptr;
  const int32_t page = a.bt[b * a.bt_stride + p];
  if (page < 0 || page >= a.n_pages) return nullptr;
  return a.pool + (static_cast<int64_t>(page) * a.bs + e % a.bs) * a.entry_bytes;
}

// grid: (ceil(k / kGatherEntries), rows)
__global__ __launch_bounds__(kGatherThreads) void k_topk_gather(TopkGatherArgs a) {
  const int r = blockIdx.y;
  const int j0 = blockIdx.x * kGatherEntries;
  const int nj = min(kGatherEntries, a.k - j0);
  if (nj <= 0) return;
  uint8_t* out_base = a.dst + (static_cast<int64_t>(r) * a.k + j0) * a.out_row_bytes;
  if (a.format == SKV_FMT_BF16) {
    const int chunks = static_cast<int>(a.entry_bytes >> 4);
    const int total = nj * chunks;
    for (int t = threadIdx.x; t < total; t += kGatherThreads) {
      const int jj = t / chunks;
      const int c = t - jj * chunks;
      const uint8_t* src = pick_entry(a, r, j0 + jj);
      u32x4 v = {0u, 0u, 0u, 0u};
      if (src) v = *(reinterpret_cast<const u32x4*>(src) + c);
      st_stream(reinterpret_cast<u32x4*>(out_base + jj * a.out_row_bytes) + c, v);
    }
    return;
  }
  // FP8 entry: [fp8_main codes][fp8_main/128 fp32 scales][rope bf16]
  const int code_chunks = a.fp8_main >> 4;             // 16 codes each -> 2 output chunks
  const int rope_chunks = (a.channels - a.fp8_main) >> 3;  // 8 bf16 each
  const int per_entry = code_chunks + rope_chunks;
  const int total = nj * per_entry;
  for (int t = threadIdx.x; t < total; t += kGatherThreads) {
    const int jj = t / per_entry;
    const int c = t - jj * per_entry;
    const uint8_t* src = pick_entry(a, r, j0 + jj);
    uint8_t* orow = out_base + jj * a.out_row_bytes;
    if (c < code_chunks) {
      u32x4 o0 = {0u, 0u, 0u, 0u}, o1 = {0u, 0u, 0u, 0u};
      if (src) {
        const u32x4 codes = *(reinterpret_cast<const u32x4*>(src) + c);
        const float scale = *reinterpret_cast<const float*>(src + a.fp8_main + (c >> 3) * 4);
        float f[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) e4m3fn_x4_to_f32(codes[q], f + 4 * q);
#pragma unroll
        for (int q = 0; q < 16; ++q) f[q] *= scale;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          o0[q] = bf16_pack2(f[2 * q], f[2 * q + 1]);
          o1[q] = bf16_pack2(f[8 + 2 * q], f[8 + 2 * q + 1]);
        }
      }
      st_stream(reinterpret_cast<u32x4*>(orow) + 2 * c, o0);
      st_stream(reinterpret_cast<u32x4*>(orow) + 2 * c + 1, o1);
    } else {
      const int rc = c - code_chunks;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (src) {
        v = *reinterpret_cast<const u32x4*>(src + a.fp8_main + (a.fp8_main >> 7) * 4 + rc * 16);
      }
      st_stream(reinterpret_cast<u32x4*>(orow + a.fp8_main * 2) + rc, v);
    }
  }
}

}  // namespace skv

using namespace skv;

static int launch_topk(const TopkArgs& a, int64_t rows, int32_t* workspace, void* stream,
                       const char* what) {
  if (a.k < 0 || a.k > kMaxTopK) {
    return set_error(SKV_EINVAL, "%s: k must be in [0, %d]; got %d", what, kMaxTopK, a.k);
  }
  if (rows < 0 || rows > 65535) return set_error(SKV_EINVAL, "%s: rows must be in [0, 65535]", what);
  if (!a.out || a.out_stride < a.k) return set_error(SKV_EINVAL, "%s: out_stride must be >= k", what);
  if (a.stride <= 0) return set_error(SKV_EINVAL, "%s: score_stride must be positive", what);
  if (rows == 0 || a.k == 0) return SKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!workspace) {
    hipLaunchKernelGGL(k_topk_select, dim3(static_cast<unsigned>(rows)), dim3(kTopkThreads), 0, s, a);
    return check_launch(what);
  }
  TopkMultiArgs m{a, workspace};
  const dim3 grid(static_cast<unsigned>(ceil_div(a.stride, kTkChunk)), static_cast<unsigned>(rows));
  hipLaunchKernelGGL(k_topk_hist, grid, dim3(kTkPartThreads), 0, s, m);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(k_topk_filter, grid, dim3(kTkPartThreads), 0, s, m);
  if ((rc = check_launch(what))) return rc;
  hipLaunchKernelGGL(k_topk_final, dim3(static_cast<unsigned>(rows)), dim3(kTopkThreads), 0, s, m);
  return check_launch(what);
}

extern "C" int64_t skv_topk_workspace_words(void) { return kTkWsWords; }

extern "C" int skv_topk_select(const float* scores, int64_t score_stride, int64_t rows,
                               const int32_t* n_valid, const int32_t* n_cols,
                               int32_t n_cols_uniform, int64_t k, int32_t* out_idx,
                               int64_t out_stride, int32_t* workspace, void* stream) {
  if (!n_valid) return set_error(SKV_EINVAL, "skv_topk_select: n_valid is NULL");
  TopkArgs a{};
  a.scores = scores;
  a.stride = score_stride;
  a.n_valid = n_valid;
  a.n_cols = n_cols;
  a.n_cols_uni = n_cols_uniform;
  a.k = static_cast<int>(k);
  a.out = out_idx;
  a.out_stride = out_stride;
  return launch_topk(a, rows, workspace, stream, "skv_topk_select");
}

extern "C" int skv_topk_select_decode(const float* scores, int64_t score_stride, int64_t batch,
                                      const int32_t* seq_lens, int64_t m, int64_t k,
                                      int32_t* out_idx, int64_t out_stride, int32_t* workspace,
                                      void* stream) {
  if (m <= 0) return set_error(SKV_EINVAL, "skv_topk_select_decode: compression_rate must be positive; got %lld", (long long)m);
  if (!seq_lens) return set_error(SKV_EINVAL, "skv_topk_select_decode: seq_lens is NULL");
  TopkArgs a{};
  a.scores = scores;
  a.stride = score_stride;
  a.lens = seq_lens;
  a.m = static_cast<int>(m);
  a.k = static_cast<int>(k);
  a.out = out_idx;
  a.out_stride = out_stride;
  return launch_topk(a, batch, workspace, stream, "skv_topk_select_decode");
}

extern "C" int skv_topk_gather(void* dst, const void* pool, int64_t entry_bytes, int64_t block_size,
                               int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                               const int32_t* n_entries, const int32_t* idx, int64_t idx_stride,
                               int64_t k, int64_t rows, const int32_t* row_seq, int64_t channels,
                               int32_t format, void* stream) {
  const char* what = "skv_topk_gather";
  if (entry_bytes <= 0 || (entry_bytes & 15) || block_size <= 0 || bt_stride <= 0) {
    return set_error(SKV_EINVAL, "%s: bad entry_bytes/block_size/bt_stride", what);
  }
  if (k < 0 || k > INT32_MAX || rows < 0 || rows > 65535 || idx_stride < k) {
    return set_error(SKV_EINVAL, "%s: need 0 <= k <= idx_stride and rows <= 65535", what);
  }
  if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(pool)) & 15) {
    return set_error(SKV_EINVAL, "%s: dst and pool must be 16-byte aligned", what);
  }
  TopkGatherArgs a{};
  a.dst = static_cast<uint8_t*>(dst);
  a.pool = static_cast<const uint8_t*>(pool);
  a.entry_bytes = entry_bytes;
  a.bs = static_cast<int>(block_size);
  a.n_pages = n_pages;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.n_entries = n_entries;
  a.idx = idx;
  a.idx_stride = idx_stride;
  a.k = static_cast<int>(k);
  a.row_seq = row_seq;
  a.channels = static_cast<int>(channels);
  a.format = format;
  if (format == SKV_FMT_BF16) {
    a.out_row_bytes = entry_bytes;
  } else if (format == SKV_FMT_FP8) {
    a.fp8_main = static_cast<int>(channels - SKV_FP8_ROPE_DIMS);
    if (a.fp8_main <= 0 || (a.fp8_main % 128) || entry_bytes != SKV_FP8_ENTRY_BYTES(channels)) {
      return set_error(SKV_EINVAL, "%s: fp8 entries need channels = 128*q + %d and entry_bytes = %lld",
                       what, SKV_FP8_ROPE_DIMS, (long long)SKV_FP8_ENTRY_BYTES(channels));
    }
    a.out_row_bytes = channels * 2;
  } else {
    return set_error(SKV_EINVAL, "%s: unknown format %d", what, format);
  }
  if (rows == 0 || k == 0) return SKV_OK;
  const dim3 grid(static_cast<unsigned>(ceil_div(k, kGatherEntries)), static_cast<unsigned>(rows));
  hipLaunchKernelGGL(k_topk_gather, grid, dim3(kGatherThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch(what);
}
