// Eviction (release of finished sequences to the free list) and compaction
// (defragmenting copy of live pages + block-table rewrite).
//
// No reference counterpart: the reference keeps contiguous per-layer tensors
// (kv_cache.py:59-60) and plans a block layout and state cache only
// (saint_llm_inference/__init__.py:5-9).  Policies, fixed here and restated by
// the CPU oracle:
//   release : push order ascending sequence, within a sequence from its last
//             logical page to its first; released tables become -1, lengths 0.
//   compact : with n_live live pages, the live pages whose id is >= n_live
//             ("movers", ascending) move into the free ids < n_live ("holes",
//             ascending); other pages keep their ids.  Afterwards the live set
//             is exactly [0, n_live) and pops return n_live, n_live+1, ...
//             Sources are all >= n_live and destinations all < n_live, so the
//             page copies are independent and run fully in parallel.
#include "skv_common.h"

namespace skv {

constexpr int kEvictThreads = 1024;
constexpr int kEvictMaxBatch = 4096;
constexpr int kMaxPools = 16;

__device__ __forceinline__ int owner_of(const int* off, int batch, int t) {
  int lo = 0, hi = batch;  // off[lo] <= t < off[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (off[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kEvictThreads) void k_release(
    int32_t* __restrict__ stack, int32_t* __restrict__ top_ptr, int64_t n_pages,
    int32_t* __restrict__ bt, int64_t bt_stride, int32_t* __restrict__ lens,
    const uint8_t* __restrict__ mask, int batch, int bs, int32_t* __restrict__ status) {
  __shared__ int off[kEvictMaxBatch + 1];
  __shared__ int cnt[kEvictMaxBatch];
  __shared__ int scan_lds[17];
  __shared__ int bad_all;
  const int tid = threadIdx.x;
  if (tid == 0) bad_all = 0;
  int carry = 0;
  for (int base = 0; base < batch; base += kEvictThreads) {
    const int b = base + tid;
    int c = 0;
    if (b < batch && mask[b]) {
      c = static_cast<int>(min<int64_t>(ceil_div(max(lens[b], 0), bs), bt_stride));
    }
    int tot;
    const int ex = block_exclusive_scan(c, scan_lds, &tot);
    if (b < batch) {
      off[b] = carry + ex;
      cnt[b] = c;
    }
    carry += tot;
  }
  if (tid == 0) off[batch] = carry;
  __syncthreads();
  const int top = *top_ptr;
  int bad = (top < 0 || static_cast<int64_t>(top) + carry > n_pages) ? SKV_STATUS_STACK : 0;
  for (int t = tid; t < carry && !bad; t += kEvictThreads) {
    const int b = owner_of(off, batch, t);
    const int32_t page = bt[static_cast<int64_t>(b) * bt_stride + (t - off[b])];
    if (page < 0 || page >= n_pages) bad = SKV_STATUS_BADARG;
  }
  if (bad) atomicOr(&bad_all, bad);
  __syncthreads();
  if (bad_all) {
    if (tid == 0 && status) *status = bad_all;
    return;
  }
  for (int t = tid; t < carry; t += kEvictThreads) {
    const int b = owner_of(off, batch, t);
    const int j = t - off[b];
    stack[top + off[b] + (cnt[b] - 1 - j)] = bt[static_cast<int64_t>(b) * bt_stride + j];
  }
  __syncthreads();  // every page id is read before the tables are cleared
  for (int t = tid; t < carry; t += kEvictThreads) {
    const int b = owner_of(off, batch, t);
    bt[static_cast<int64_t>(b) * bt_stride + (t - off[b])] = -1;
  }
  for (int b = tid; b < batch; b += kEvictThreads) {
    if (mask[b]) lens[b] = 0;
  }
  if (tid == 0) {
    *top_ptr = top + carry;
    if (status) *status = 0;
  }
}

// ---- compaction -------------------------------------------------------------
struct PoolRefs {
  uint8_t* base[kMaxPools];
  int64_t page_bytes[kMaxPools];
  int n;
};

__global__ void k_fill_i32(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    p[i] = v;
  }
}

// grid: (ceil(bt_stride / 256), batch)
__global__ void k_mark_live(const int32_t* __restrict__ bt, int64_t bt_stride,
                            const int32_t* __restrict__ lens, int bs, int64_t n_pages,
                            int32_t* __restrict__ mark) {
  const int b = blockIdx.y;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t np = min<int64_t>(ceil_div(max(lens[b], 0), bs), bt_stride);
  if (j >= np) return;
  const int32_t p = bt[b * bt_stride + j];
  if (p >= 0 && p < n_pages) mark[p] = 1;
}

// One workgroup: n_live, hole and mover lists, remap, new free stack.
// ws: [0, n) mark -> remap, [n, 2n) holes, [2n, 3n) movers.  info = {n_live, n_moved}.
__global__ __launch_bounds__(kEvictThreads) void k_compact_plan(int32_t* __restrict__ ws, int64_t n,
                                                                int32_t* __restrict__ stack,
                                                                int32_t* __restrict__ top_ptr,
                                                                int32_t* __restrict__ info) {
  __shared__ int scan_lds[17];
  const int tid = threadIdx.x;
  int32_t* mark = ws;
  int32_t* holes = ws + n;
  int32_t* movers = ws + 2 * n;
  int n_live = 0;
  for (int64_t base = 0; base < n; base += kEvictThreads) {
    const int64_t i = base + tid;
    n_live += block_reduce_sum(i < n ? mark[i] : 0, scan_lds);
  }
  int carry = 0;
  for (int64_t base = 0; base < n_live; base += kEvictThreads) {
    const int64_t i = base + tid;
    const int is_hole = (i < n_live && mark[i] == 0) ? 1 : 0;
    int tot;
    const int r = carry + block_exclusive_scan(is_hole, scan_lds, &tot);
    if (is_hole) holes[r] = static_cast<int32_t>(i);
    carry += tot;
  }
  __syncthreads();  // holes[] complete before the movers read it
  const int n_moved = carry;
  carry = 0;
  for (int64_t base = n_live; base < n; base += kEvictThreads) {
    const int64_t i = base + tid;
    const int is_mover = (i < n && mark[i] != 0) ? 1 : 0;
    int tot;
    const int r = carry + block_exclusive_scan(is_mover, scan_lds, &tot);
    if (i < n) mark[i] = is_mover ? holes[r] : -1;  // remap for ids >= n_live
    if (is_mover) movers[r] = static_cast<int32_t>(i);
    carry += tot;
  }
  const int64_t n_free = n - n_live;
  for (int64_t i = tid; i < n_free; i += kEvictThreads) stack[i] = static_cast<int32_t>(n - 1 - i);
  if (tid == 0) {
    *top_ptr = static_cast<int32_t>(n_free);
    info[0] = n_live;
    info[1] = n_moved;
  }
}

constexpr int kCompactCopyThreads = 256;

// Persistent grid over (mover rank, pool); each unit copies one page.
__global__ __launch_bounds__(kCompactCopyThreads) void k_compact_copy(PoolRefs pools,
                                                                     const int32_t* __restrict__ ws,
                                                                     int64_t n,
                                                                     const int32_t* __restrict__ info) {
  const int n_moved = info[1];
  const int32_t* holes = ws + n;
  const int32_t* movers = ws + 2 * n;
  const int64_t units = static_cast<int64_t>(n_moved) * pools.n;
  for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
    const int r = static_cast<int>(u / pools.n);
    const int q = static_cast<int>(u % pools.n);
    const int64_t pb = pools.page_bytes[q];
    const u32x4* src = reinterpret_cast<const u32x4*>(pools.base[q] + movers[r] * pb);
    u32x4* dst = reinterpret_cast<u32x4*>(pools.base[q] + holes[r] * pb);
    const int chunks = static_cast<int>(pb >> 4);
    constexpr int U = 8;
    for (int base = 0; base < chunks; base += kCompactCopyThreads * U) {
      u32x4 v[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int c = base + k * kCompactCopyThreads + threadIdx.x;
        if (c < chunks) v[k] = ld_stream(src + c);
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int c = base + k * kCompactCopyThreads + threadIdx.x;
        if (c < chunks) st_stream(dst + c, v[k]);
      }
    }
  }
}

// grid: (ceil(bt_stride / 256), batch)
__global__ void k_compact_rewrite(int32_t* __restrict__ bt, int64_t bt_stride,
                                  const int32_t* __restrict__ lens, int bs,
                                  const int32_t* __restrict__ remap,
                                  const int32_t* __restrict__ info) {
  const int b = blockIdx.y;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t np = min<int64_t>(ceil_div(max(lens[b], 0), bs), bt_stride);
  if (j >= np) return;
  const int n_live = info[0];
  const int32_t p = bt[b * bt_stride + j];
  if (p >= n_live) bt[b * bt_stride + j] = remap[p];
}

}  // namespace skv

using namespace skv;

extern "C" int skv_release(int32_t* free_stack, int32_t* free_top, int64_t n_pages,
                           int32_t* block_table, int64_t bt_stride, int32_t* seq_lens,
                           const uint8_t* release_mask, int64_t batch, int64_t block_size,
                           int32_t* status, void* stream) {
  if (batch < 0 || batch > kEvictMaxBatch) {
    return set_error(SKV_EINVAL, "skv_release: batch must be in [0, %d]; got %lld", kEvictMaxBatch,
                     (long long)batch);
  }
  if (block_size <= 0 || bt_stride <= 0 || n_pages <= 0 || n_pages > INT32_MAX) {
    return set_error(SKV_EINVAL, "skv_release: bad block_size/bt_stride/n_pages");
  }
  if (!release_mask) return set_error(SKV_EINVAL, "skv_release: release_mask is NULL");
  if (batch == 0) return SKV_OK;
  hipLaunchKernelGGL(k_release, dim3(1), dim3(kEvictThreads), 0, static_cast<hipStream_t>(stream),
                     free_stack, free_top, n_pages, block_table, bt_stride, seq_lens, release_mask,
                     static_cast<int>(batch), static_cast<int>(block_size), status);
  return check_launch("skv_release");
}

extern "C" int skv_compact(const skv_pool_ref* pools, int32_t n_pools, int32_t* block_table,
                           int64_t bt_stride, const int32_t* seq_lens, int64_t batch,
                           int64_t block_size, int64_t n_pages, int32_t* free_stack,
                           int32_t* free_top, int32_t* workspace, int32_t* info, void* stream) {
  const char* what = "skv_compact";
  if (n_pools < 1 || n_pools > kMaxPools || !pools) {
    return set_error(SKV_EINVAL, "%s: n_pools must be in [1, %d]; got %d", what, kMaxPools, n_pools);
  }
  if (batch < 0 || batch > 65535 || block_size <= 0 || bt_stride <= 0 || n_pages <= 0 ||
      n_pages > INT32_MAX) {
    return set_error(SKV_EINVAL, "%s: bad batch/block_size/bt_stride/n_pages", what);
  }
  if (!workspace || !info || !free_stack || !free_top) {
    return set_error(SKV_EINVAL, "%s: NULL workspace/info/free list", what);
  }
  PoolRefs refs{};
  refs.n = n_pools;
  for (int q = 0; q < n_pools; ++q) {
    if (!pools[q].base || pools[q].page_bytes <= 0 || (pools[q].page_bytes & 15) ||
        (reinterpret_cast<uintptr_t>(pools[q].base) & 15)) {
      return set_error(SKV_EINVAL, "%s: pool %d needs a 16-byte aligned base and page_bytes", what, q);
    }
    refs.base[q] = static_cast<uint8_t*>(pools[q].base);
    refs.page_bytes[q] = pools[q].page_bytes;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t fill_blocks = ceil_div(n_pages, 256) < 4096 ? ceil_div(n_pages, 256) : 4096;
  hipLaunchKernelGGL(k_fill_i32, dim3(static_cast<unsigned>(fill_blocks)), dim3(256), 0, s, workspace,
                     n_pages, 0);
  int rc = check_launch(what);
  if (rc) return rc;
  const dim3 tgrid(static_cast<unsigned>(ceil_div(bt_stride, 256)), static_cast<unsigned>(batch));
  if (batch > 0) {
    hipLaunchKernelGGL(k_mark_live, tgrid, dim3(256), 0, s, block_table, bt_stride, seq_lens,
                       static_cast<int>(block_size), n_pages, workspace);
    if ((rc = check_launch(what))) return rc;
  }
  hipLaunchKernelGGL(k_compact_plan, dim3(1), dim3(kEvictThreads), 0, s, workspace, n_pages,
                     free_stack, free_top, info);
  if ((rc = check_launch(what))) return rc;
  hipLaunchKernelGGL(k_compact_copy, dim3(kPersistentBlocks), dim3(kCompactCopyThreads), 0, s, refs,
                     workspace, n_pages, info);
  if ((rc = check_launch(what))) return rc;
  if (batch > 0) {
    hipLaunchKernelGGL(k_compact_rewrite, tgrid, dim3(256), 0, s, block_table, bt_stride, seq_lens,
                       static_cast<int>(block_size), workspace, info);
    if ((rc = check_launch(what))) return rc;
  }
  return SKV_OK;
}
