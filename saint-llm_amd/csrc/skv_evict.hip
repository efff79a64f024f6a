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

// The plan runs one workgroup per block of kPlanSpan page ids.  A count
// launch before it writes the live pages of every block (counts: the last
// n_blocks words of the workspace, which the movers' list never reaches:
// n_moved <= n / 2), so that each plan workgroup knows how many live pages
// precede its block without waiting for another workgroup.
constexpr int kPlanPer = 4;                          // ids per thread: one 16-byte load of marks
constexpr int kPlanShift = 12;
constexpr int kPlanSpan = 1 << kPlanShift;           // ids per plan workgroup
static_assert(kPlanSpan == kEvictThreads * kPlanPer, "a plan workgroup covers its block in one pass");

__host__ __device__ __forceinline__ int64_t plan_blocks(int64_t n) { return (n + kPlanSpan - 1) >> kPlanShift; }

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

// The marks of ids [i0, i0 + kPlanPer) (0 past n).
__device__ __forceinline__ void load_run(const int32_t* mark, int64_t i0, int64_t n, int* v) {
  if (i0 + kPlanPer <= n) {  // whole run in range: one 16-byte load (i0 is a multiple of 4)
    const int4 w = *reinterpret_cast<const int4*>(mark + i0);
    v[0] = w.x;
    v[1] = w.y;
    v[2] = w.z;
    v[3] = w.w;
  } else {
#pragma unroll
    for (int k = 0; k < kPlanPer; ++k) v[k] = (i0 + k < n) ? mark[i0 + k] : 0;
  }
}

// Workgroup g writes the live pages of ids [g * kPlanSpan, (g + 1) * kPlanSpan).
__global__ __launch_bounds__(kEvictThreads) void k_count_live(const int32_t* __restrict__ mark, int64_t n,
                                                              int32_t* __restrict__ counts) {
  __shared__ int scan_lds[17];
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kPlanSpan + static_cast<int64_t>(threadIdx.x) * kPlanPer;
  int v[kPlanPer];
  load_run(mark, i0, n, v);
  int c = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) c += (v[k] != 0) ? 1 : 0;
  c = block_reduce_sum(c, scan_lds);
  if (threadIdx.x == 0) counts[blockIdx.x] = c;
}

// Workgroup g: ids [g * kPlanSpan, (g + 1) * kPlanSpan).
// ws: [0, n) marks -> movers' ranks, [n, 2n) holes, [2n, 3n) movers; counts
// as above.  A hole's rank is the number of holes before it (its id less the
// live pages before it); a mover's rank is the number of live pages in
// [n_live, id), i.e. the live pages before it less those before n_live.
// A mover's mark becomes its rank, which the copy launch's table rewrite
// reads and clears; the copy launch also clears the marks below n_live (other
// plan workgroups read them here), so words [0, n) are zero again after the
// compaction.  The free stack is rebuilt so that pops return
// n_live, n_live + 1, ...; info = {n_live, n_moved} (workgroup 0).
__global__ __launch_bounds__(kEvictThreads) void k_compact_plan(int32_t* __restrict__ ws, int64_t n,
                                                                int32_t* __restrict__ stack,
                                                                int32_t* __restrict__ top_ptr,
                                                                int32_t* __restrict__ info) {
  __shared__ int scan_lds[17];
  const int tid = threadIdx.x;
  const int g = blockIdx.x;
  const int n_blocks = static_cast<int>(plan_blocks(n));
  int32_t* mark = ws;
  int32_t* holes = ws + n;
  int32_t* movers = ws + 2 * n;
  const int32_t* counts = ws + 3 * n - n_blocks;
  // every load of the first round trip: the block counts and this block's marks
  constexpr int kCntPer = (1 << 24) / kPlanSpan / kEvictThreads;  // n < 2^24 pages
  int cnt[kCntPer];
#pragma unroll
  for (int k = 0; k < kCntPer; ++k) {
    const int i = tid + k * kEvictThreads;
    cnt[k] = (i < n_blocks) ? counts[i] : 0;
  }
  const int64_t i0 = static_cast<int64_t>(g) * kPlanSpan + static_cast<int64_t>(tid) * kPlanPer;
  int v[kPlanPer];
  load_run(mark, i0, n, v);
  int total = 0, before = 0;
#pragma unroll
  for (int k = 0; k < kCntPer; ++k) {
    total += cnt[k];
    before += (tid + k * kEvictThreads < g) ? cnt[k] : 0;
  }
  const int64_t n_live = block_reduce_sum(total, scan_lds);
  before = block_reduce_sum(before, scan_lds);
  // live pages before n_live: the blocks before its block, then that block up to n_live
  const int gs = static_cast<int>(n_live >> kPlanShift);
  int pre = 0;
#pragma unroll
  for (int k = 0; k < kCntPer; ++k) pre += (tid + k * kEvictThreads < gs) ? cnt[k] : 0;
  int w[kPlanPer];
  const int64_t j0 = static_cast<int64_t>(gs) * kPlanSpan + static_cast<int64_t>(tid) * kPlanPer;
  load_run(mark, j0, n_live, w);
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) pre += (w[k] != 0) ? 1 : 0;
  const int live_below = block_reduce_sum(pre, scan_lds);  // live pages with id < n_live
  const int n_moved = static_cast<int>(n_live) - live_below;
  // this block's ids
  int c = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) c += (v[k] != 0) ? 1 : 0;
  int tot;
  int lb = before + block_exclusive_scan(c, scan_lds, &tot);  // live pages before id i0
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int64_t i = i0 + k;
    if (i >= n) break;
    const bool live = v[k] != 0;
    if (i < n_live) {
      if (!live) holes[i - lb] = static_cast<int32_t>(i);
    } else {
      if (live) {
        const int r = lb - live_below;
        movers[r] = static_cast<int32_t>(i);
        mark[i] = r;
      }
      stack[n - 1 - i] = static_cast<int32_t>(i);
    }
    lb += live ? 1 : 0;
  }
  if (g == 0 && tid == 0) {
    *top_ptr = static_cast<int32_t>(n - n_live);
    info[0] = static_cast<int32_t>(n_live);
    info[1] = n_moved;
  }
}

constexpr int kCompactCopyThreads = 256;
constexpr int kCopySlice = kCompactCopyThreads * 16;  // bytes per copy slice: 16 per thread
constexpr int kCopySlices = 8;                        // slices per workgroup per iteration

// Slices of the page copies: mover rank r owns slices [r * per_mover, (r+1) *
// per_mover); slices [first[q], first[q+1]) of a mover are pool q's page.
struct CopySlices {
  int32_t first[kMaxPools + 1];
  int32_t per_mover;
};

// Persistent grid over 4 KB slices of (mover, pool) pages.  A workgroup takes
// kCopySlices slices per iteration, all loads issued before any store; the
// hole / mover ids of its next iteration are loaded before this iteration's
// stores, so only the first iteration waits for them.  The same grid first
// rewrites the block tables (every table entry of a live page at or above
// n_live takes the hole of its rank, which it then clears) and clears the
// plan's marks below n_live.
struct TableRef {
  int32_t* bt;
  const int32_t* lens;
  int32_t bt_stride;
  int32_t batch;
  int32_t block_size;
};

__device__ __forceinline__ void slice_ids(const CopySlices& cs, const int32_t* movers, const int32_t* holes,
                                          int s0, int total, int32_t* src_id, int32_t* dst_id) {
#pragma unroll
  for (int k = 0; k < kCopySlices; ++k) {
    const int s = min(s0 + k, total - 1);
    const int r = static_cast<int>(udiv24(s, cs.per_mover));
    src_id[k] = movers[r];
    dst_id[k] = holes[r];
  }
}

__global__ __launch_bounds__(kCompactCopyThreads) void k_compact_copy(PoolRefs pools, CopySlices cs, TableRef tr,
                                                                     int32_t* __restrict__ ws, int64_t n,
                                                                     const int32_t* __restrict__ info) {
  const int n_live = info[0];
  const int n_moved = info[1];
  int32_t* remap = ws;
  const int32_t* holes = ws + n;
  const int32_t* movers = ws + 2 * n;
  const int total = n_moved * cs.per_mover;  // < 2^24 (checked on the host)
  // the moved pages' stores: plain (allocating) stores when the move writes
  // 96-256 MiB, where the written pages stay in the 256 MiB last-level
  // cache (fp8 1M-token pools: 227 MiB moved, 115 -> 104 us per release +
  // compaction on MI355X), nontemporal stores otherwise (the same limits as
  // the decode gather's rows)
  const int64_t moved_bytes = static_cast<int64_t>(total) * kCopySlice;
  const bool wb = moved_bytes >= (static_cast<int64_t>(96) << 20) && moved_bytes <= (static_cast<int64_t>(256) << 20);
  const int tid = threadIdx.x;
  const int gtid = blockIdx.x * kCompactCopyThreads + tid;
  const int gsize = gridDim.x * kCompactCopyThreads;
  int s0 = blockIdx.x * kCopySlices;
  int32_t src_id[kCopySlices], dst_id[kCopySlices];
  if (s0 < total) slice_ids(cs, movers, holes, s0, total, src_id, dst_id);  // in flight during the rewrite
  const int entries = tr.batch * tr.bt_stride;  // < 2^24 (checked on the host)
  for (int t = gtid; t < entries; t += gsize) {
    const int b = static_cast<int>(udiv24(t, tr.bt_stride));
    const int j = t - b * tr.bt_stride;
    const int np = static_cast<int>(min<int64_t>(ceil_div24(max(tr.lens[b], 0), tr.block_size), tr.bt_stride));
    if (j < np) {
      const int32_t p = tr.bt[t];
      if (p >= n_live && p < n) {
        tr.bt[t] = holes[remap[p]];
        remap[p] = 0;
      }
    }
  }
  for (int i = gtid; i < n_live; i += gsize) remap[i] = 0;
  for (; s0 < total; s0 += gridDim.x * kCopySlices) {
    int q_of[kCopySlices], off[kCopySlices];
#pragma unroll
    for (int k = 0; k < kCopySlices; ++k) {
      const int s = min(s0 + k, total - 1);
      const int r = static_cast<int>(udiv24(s, cs.per_mover));
      const int j = s - r * cs.per_mover;
      int q = 0;
      for (int qq = 1; qq < pools.n; ++qq) q += (j >= cs.first[qq]) ? 1 : 0;
      q_of[k] = q;
      off[k] = (j - cs.first[q]) * kCopySlice + tid * 16;
    }
    u32x4 v[kCopySlices];
#pragma unroll
    for (int k = 0; k < kCopySlices; ++k) {
      const int64_t pb = pools.page_bytes[q_of[k]];
      const bool live = s0 + k < total && off[k] < pb;
      const uint8_t* src = pools.base[q_of[k]] + static_cast<int64_t>(src_id[k]) * pb + (live ? off[k] : 0);
      v[k] = ld_stream(reinterpret_cast<const u32x4*>(src));
    }
    int32_t next_src[kCopySlices], next_dst[kCopySlices];
    const int s1 = s0 + gridDim.x * kCopySlices;
    if (s1 < total) slice_ids(cs, movers, holes, s1, total, next_src, next_dst);
#pragma unroll
    for (int k = 0; k < kCopySlices; ++k) {
      const int64_t pb = pools.page_bytes[q_of[k]];
      if (s0 + k < total && off[k] < pb) {
        u32x4* dst = reinterpret_cast<u32x4*>(pools.base[q_of[k]] + static_cast<int64_t>(dst_id[k]) * pb + off[k]);
        if (wb) {
          *dst = v[k];
        } else {
          st_stream(dst, v[k]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kCopySlices; ++k) {
      src_id[k] = next_src[k];
      dst_id[k] = next_dst[k];
    }
  }
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
  int64_t slices_per_mover = 0;
  for (int q = 0; q < n_pools; ++q) {
    if (!pools[q].base || pools[q].page_bytes <= 0 || (pools[q].page_bytes & 15) ||
        (reinterpret_cast<uintptr_t>(pools[q].base) & 15)) {
      return set_error(SKV_EINVAL, "%s: pool %d needs a 16-byte aligned base and page_bytes", what, q);
    }
    refs.base[q] = static_cast<uint8_t*>(pools[q].base);
    refs.page_bytes[q] = pools[q].page_bytes;
    slices_per_mover += ceil_div(pools[q].page_bytes, kCopySlice);
  }
  if (n_pages >= (1 << 24) || n_pages * slices_per_mover >= (1 << 24)) {
    return set_error(SKV_EINVAL, "%s: n_pages x 4 KB slices per page must stay below 2^24", what);
  }
  if (batch * bt_stride >= (1 << 24)) {
    return set_error(SKV_EINVAL, "%s: batch x bt_stride must stay below 2^24", what);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
  const dim3 tgrid(static_cast<unsigned>(ceil_div(bt_stride, 256)), static_cast<unsigned>(batch));
  if (batch > 0) {
    hipLaunchKernelGGL(k_mark_live, tgrid, dim3(256), 0, s, block_table, bt_stride, seq_lens,
                       static_cast<int>(block_size), n_pages, workspace);
    if ((rc = check_launch(what))) return rc;
  }
  const dim3 pgrid(static_cast<unsigned>(plan_blocks(n_pages)));
  hipLaunchKernelGGL(k_count_live, pgrid, dim3(kEvictThreads), 0, s, workspace, n_pages,
                     workspace + 3 * n_pages - plan_blocks(n_pages));
  if ((rc = check_launch(what))) return rc;
  hipLaunchKernelGGL(k_compact_plan, pgrid, dim3(kEvictThreads), 0, s, workspace, n_pages,
                     free_stack, free_top, info);
  if ((rc = check_launch(what))) return rc;
  CopySlices cs{};
  for (int q = 0; q < n_pools; ++q) cs.first[q + 1] = cs.first[q] + static_cast<int32_t>(ceil_div(refs.page_bytes[q], kCopySlice));
  cs.per_mover = cs.first[n_pools];
  const TableRef tr{block_table, seq_lens, static_cast<int32_t>(bt_stride), static_cast<int32_t>(batch),
                    static_cast<int32_t>(block_size)};
  hipLaunchKernelGGL(k_compact_copy, dim3(kPersistentBlocks), dim3(kCompactCopyThreads), 0, s, refs, cs, tr,
                     workspace, n_pages, info);
  return check_launch(what);
}
