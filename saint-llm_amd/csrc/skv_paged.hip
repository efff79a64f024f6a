// Paged KV storage: free-stack initialisation, page reservation, paged
// append, full block-table gather and the fused decode-step append+gather.
//
// Reference semantics (packages/inference/src/saint_llm_inference/kv_cache.py):
//   append  self.k[:, L:L+n] = k_new; L += n          (:80-82)
//   view    self.k[:, :L]                             (:83)
// Here the rows live in fixed-size pages reached through an int32 block table,
// and each sequence has its own length.
#include <mutex>

#include "skv_common.h"

namespace skv {

constexpr int kMaxBatch = 4096;
constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 8;
constexpr int kReserveThreads = 1024;
constexpr int kAppendRowsPerUnit = 16;

// ---------------------------------------------------------------------------
// Free stack
// ---------------------------------------------------------------------------
__global__ void k_free_stack_init(int32_t* __restrict__ stack, int32_t* __restrict__ top,
                                  const int32_t* __restrict__ order, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) {
    // pop order: stack[n-1], stack[n-2], ...  => element popped k-th sits at n-1-k.
    stack[n - 1 - i] = order ? order[i] : static_cast<int32_t>(i);
  }
  if (i == 0) *top = static_cast<int32_t>(n);
}

// ---------------------------------------------------------------------------
// Reservation: one workgroup, prefix scan over per-sequence page demand.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kReserveThreads) void k_reserve(
    int32_t* __restrict__ stack, int32_t* __restrict__ top_ptr, int64_t n_pages,
    int32_t* __restrict__ bt, int64_t bt_stride, int64_t max_pages, int32_t* __restrict__ lens,
    const int32_t* __restrict__ n_new, int32_t n_uni, int batch, int bs,
    int32_t* __restrict__ status) {
  __shared__ int off[kMaxBatch + 1];
  __shared__ int first[kMaxBatch];
  __shared__ int scan_lds[17];
  const int tid = threadIdx.x;
  int bad = 0;
  int carry = 0;
  for (int base = 0; base < batch; base += kReserveThreads) {
    const int b = base + tid;
    int need = 0;
    if (b < batch) {
      const int L = lens[b];
      const int n = n_new ? n_new[b] : n_uni;
      if (n < 0 || L < 0) {
        bad |= SKV_STATUS_BADARG;
      } else {
        const int64_t p0 = ceil_div(L, bs);
        const int64_t p1 = ceil_div(static_cast<int64_t>(L) + n, bs);
        if (p1 > max_pages) bad |= SKV_STATUS_MAX_PAGES;
        need = static_cast<int>(p1 - p0);
        first[b] = static_cast<int>(p0);
      }
    }
    int tot;
    const int ex = block_exclusive_scan(need, scan_lds, &tot);
    if (b < batch) off[b] = carry + ex;
    carry += tot;
  }
  const int top = *top_ptr;
  if (top < 0 || top > n_pages) bad |= SKV_STATUS_BADARG;
  else if (carry > top) bad |= SKV_STATUS_NOSPC;
  // combine flags over the block
  __shared__ int bad_all;
  if (tid == 0) bad_all = 0;
  __syncthreads();
  if (bad) atomicOr(&bad_all, bad);
  __syncthreads();
  if (bad_all) {
    if (tid == 0 && status) *status = bad_all;
    return;
  }
  if (tid == 0) off[batch] = carry;
  __syncthreads();
  for (int t = tid; t < carry; t += kReserveThreads) {
    // largest b with off[b] <= t (sequences with zero demand share offsets)
    int lo = 0, hi = batch;  // invariant: off[lo] <= t < off[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (off[mid] <= t) lo = mid; else hi = mid;
    }
    const int j = t - off[lo];
    bt[static_cast<int64_t>(lo) * bt_stride + first[lo] + j] = stack[top - 1 - t];
  }
  for (int b = tid; b < batch; b += kReserveThreads) {
    lens[b] += n_new ? n_new[b] : n_uni;
  }
  if (tid == 0) {
    *top_ptr = top - carry;
    if (status) *status = 0;
  }
}

// ---------------------------------------------------------------------------
// Work decomposition shared by the copy kernels: every workgroup builds the
// exclusive prefix of per-sequence unit counts in LDS, then walks units with
// a grid stride and finds the owning sequence by binary search.
// ---------------------------------------------------------------------------
struct CopyArgs {
  uint8_t* dst;
  const int64_t* dst_off;
  int64_t dst_stride_rows;
  int64_t dst_cap;  // rows in the dst allocation
  uint8_t* pool;
  int64_t row_bytes;
  int bs;
  int64_t n_pages;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* lens;
  const int32_t* n_new;
  int n_uni;
  const uint8_t* src;
  int64_t src_seq_stride;
  int64_t src_row_stride;
  int64_t src_len;  // rows per sequence available in src
  int batch;
};

// Copy `nchunks` 16-byte chunks; kCopyUnroll loads in flight per lane.
__device__ __forceinline__ void copy_chunks(u32x4* __restrict__ d, const u32x4* __restrict__ s,
                                            int nchunks) {
  for (int base = 0; base < nchunks; base += kCopyThreads * kCopyUnroll) {
    u32x4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int c = base + u * kCopyThreads + threadIdx.x;
      if (c < nchunks) v[u] = ld_stream(s + c);
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int c = base + u * kCopyThreads + threadIdx.x;
      if (c < nchunks) st_stream(d + c, v[u]);
    }
  }
}

// Copy rows [r0, r1) of a sequence's new-token source to the pool page (and
// optionally to dst); rows are not contiguous in the source.
__device__ __forceinline__ void copy_new_rows(const CopyArgs& a, int b, int L, int n, int r0, int r1,
                                              uint8_t* page_base, int page_r0, uint8_t* dst_rows) {
  const int row_chunks = static_cast<int>(a.row_bytes >> 4);
  const int nrows = r1 - r0;
  const int total = nrows * row_chunks;
  for (int c = threadIdx.x; c < total; c += kCopyThreads) {
    const int rr = c / row_chunks;
    const int cc = c - rr * row_chunks;
    const int row = r0 + rr;
    const int i = row - (L - n);  // index among this call's new rows
    if (i >= a.src_len) continue;  // caller passed fewer source rows than n_new: never read past src
    const u32x4* s = reinterpret_cast<const u32x4*>(a.src + b * a.src_seq_stride + i * a.src_row_stride) + cc;
    const u32x4 v = *s;
    u32x4* pd = reinterpret_cast<u32x4*>(page_base + static_cast<int64_t>(row - page_r0) * a.row_bytes) + cc;
    *pd = v;
    if (dst_rows) {
      u32x4* dd = reinterpret_cast<u32x4*>(dst_rows + static_cast<int64_t>(row) * a.row_bytes) + cc;
      st_stream(dd, v);
    }
  }
}

__device__ __forceinline__ int find_owner(const int* cum, int batch, int u) {
  int lo = 0, hi = batch;  // cum[lo] <= u < cum[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cum[mid] <= u) lo = mid; else hi = mid;
  }
  return lo;
}

// kMode 0: gather only; 1: append only; 2: fused append + gather.
template <int kMode>
__global__ __launch_bounds__(kCopyThreads) void k_paged_copy(CopyArgs a) {
  extern __shared__ int cum[];  // [batch + 1] then 17 scan words
  int* scan_lds = cum + a.batch + 1;
  int carry = 0;
  for (int base = 0; base < a.batch; base += kCopyThreads) {
    const int b = base + threadIdx.x;
    int units = 0;
    if (b < a.batch) {
      const int L = a.lens[b];
      if (kMode == 1) {
        const int n = a.n_new ? a.n_new[b] : a.n_uni;
        units = (n + kAppendRowsPerUnit - 1) / kAppendRowsPerUnit;
      } else {
        units = (L + a.bs - 1) / a.bs;
      }
    }
    int tot;
    const int ex = block_exclusive_scan(units, scan_lds, &tot);
    if (b < a.batch) cum[b] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) cum[a.batch] = carry;
  __syncthreads();
  const int total_units = carry;
  const int64_t page_bytes = static_cast<int64_t>(a.bs) * a.row_bytes;
  for (int u = blockIdx.x; u < total_units; u += gridDim.x) {
    const int b = find_owner(cum, a.batch, u);
    const int k = u - cum[b];
    const int L = a.lens[b];
    const int n = (kMode != 0) ? (a.n_new ? a.n_new[b] : a.n_uni) : 0;
    if (kMode == 1) {
      // rows [L-n + k*R, min(L, L-n + (k+1)*R)), possibly spanning pages
      int r = L - n + k * kAppendRowsPerUnit;
      const int r_end = min(L, r + kAppendRowsPerUnit);
      while (r < r_end) {
        const int p = r / a.bs;
        const int pr0 = p * a.bs;
        const int seg_end = min(r_end, pr0 + a.bs);
        const int32_t page = (p < a.bt_stride) ? a.bt[static_cast<int64_t>(b) * a.bt_stride + p] : -1;
        if (page >= 0 && page < a.n_pages) {  // an unmapped page is skipped, never dereferenced
          uint8_t* page_base = a.pool + static_cast<int64_t>(page) * page_bytes;
          copy_new_rows(a, b, L, n, r, seg_end, page_base, pr0, nullptr);
        }
        r = seg_end;
      }
      continue;
    }
    const int r0 = k * a.bs;
    const int r1 = min(L, r0 + a.bs);
    const int32_t page = (k < a.bt_stride) ? a.bt[static_cast<int64_t>(b) * a.bt_stride + k] : -1;
    if (page < 0 || page >= a.n_pages) continue;  // unmapped: skipped, never dereferenced
    uint8_t* page_base = a.pool + static_cast<int64_t>(page) * page_bytes;
    const int64_t drow0 = a.dst_off ? a.dst_off[b] : static_cast<int64_t>(b) * a.dst_stride_rows;
    if (drow0 < 0 || drow0 + r1 > a.dst_cap) continue;  // never write past the dst allocation
    uint8_t* dst_rows = a.dst + drow0 * a.row_bytes;  // row 0 of sequence b
    const int rc = (kMode == 2) ? max(r0, min(r1, L - n)) : r1;  // first new row in this page
    if (rc > r0) {
      copy_chunks(reinterpret_cast<u32x4*>(dst_rows + static_cast<int64_t>(r0) * a.row_bytes),
                  reinterpret_cast<const u32x4*>(page_base),
                  static_cast<int>((static_cast<int64_t>(rc - r0) * a.row_bytes) >> 4));
    }
    if (kMode == 2 && rc < r1) {
      copy_new_rows(a, b, L, n, rc, r1, page_base, r0, dst_rows);
    }
  }
}

static int validate_copy(const char* what, int64_t row_bytes, int64_t block_size, int64_t batch,
                         int64_t bt_stride, const void* p0, const void* p1) {
  if (row_bytes <= 0 || (row_bytes & 15)) {
    return set_error(SKV_EINVAL, "%s: row_bytes must be a positive multiple of 16; got %lld",
                     what, (long long)row_bytes);
  }
  if (block_size <= 0 || block_size > (1 << 20)) {
    return set_error(SKV_EINVAL, "%s: block_size must be in [1, 2^20]; got %lld", what,
                     (long long)block_size);
  }
  if (batch < 0 || batch > kMaxBatch) {
    return set_error(SKV_EINVAL, "%s: batch must be in [0, %d]; got %lld", what, kMaxBatch,
                     (long long)batch);
  }
  if (bt_stride <= 0) {
    return set_error(SKV_EINVAL, "%s: bt_stride must be positive; got %lld", what,
                     (long long)bt_stride);
  }
  if ((reinterpret_cast<uintptr_t>(p0) & 15) || (reinterpret_cast<uintptr_t>(p1) & 15)) {
    return set_error(SKV_EINVAL, "%s: data pointers must be 16-byte aligned", what);
  }
  if (block_size * row_bytes > (int64_t(1) << 31)) {
    return set_error(SKV_EINVAL, "%s: page of %lld bytes exceeds 2 GiB", what,
                     (long long)(block_size * row_bytes));
  }
  return SKV_OK;
}

static int validate_src(const char* what, const void* src, int64_t seq_stride, int64_t row_stride) {
  if (!src) return set_error(SKV_EINVAL, "%s: src is NULL", what);
  if ((reinterpret_cast<uintptr_t>(src) & 15) || (seq_stride & 15) || (row_stride & 15)) {
    return set_error(SKV_EINVAL, "%s: src pointer and strides must be 16-byte aligned", what);
  }
  return SKV_OK;
}

template <int kMode>
static int launch_copy(const CopyArgs& a, hipStream_t stream, const char* what) {
  if (a.batch == 0) return SKV_OK;
  const size_t shmem = (a.batch + 1 + 17) * sizeof(int);
  hipLaunchKernelGGL(k_paged_copy<kMode>, dim3(kPersistentBlocks), dim3(kCopyThreads), shmem,
                     stream, a);
  return check_launch(what);
}

// ---------------------------------------------------------------------------
// Decode step of a paged raw-token cache in two launches: a one-workgroup
// planner (reserve + page-unit table) and a copy over 4 KB slices of the page
// units, one 256-thread workgroup per slice (one 16-byte load per lane).
// Unit table: word 0 = unit count; unit u at words 8 + 8u:
//   page, sequence, rows, first new row (relative to the unit), dst row (int64)
// ---------------------------------------------------------------------------
constexpr int kUnitWords = 8;
constexpr int kUnitHeader = 8;
constexpr int kSliceThreads = 256;

__global__ __launch_bounds__(kReserveThreads) void k_plan_units(
    int32_t* __restrict__ stack, int32_t* __restrict__ top_ptr, int64_t n_pages,
    int32_t* __restrict__ bt, int64_t bt_stride, int32_t* __restrict__ lens,
    const int32_t* __restrict__ n_new, int32_t n_uni, int batch, int bs,
    const int64_t* __restrict__ dst_off, int64_t dst_seq_stride_rows, int32_t* __restrict__ units,
    int64_t max_units, int32_t* __restrict__ status) {
  __shared__ int off[kMaxBatch + 1];
  __shared__ int first[kMaxBatch];
  __shared__ int uoff[kMaxBatch + 1];
  __shared__ int scan_lds[17];
  __shared__ int bad_all;
  const int tid = threadIdx.x;
  if (tid == 0) bad_all = 0;
  int bad = 0;
  int carry = 0, ucarry = 0;
  for (int base = 0; base < batch; base += kReserveThreads) {
    const int b = base + tid;
    int need = 0, nu = 0;
    if (b < batch) {
      const int L = lens[b];
      const int n = n_new ? n_new[b] : n_uni;
      if (n < 0 || L < 0) {
        bad |= SKV_STATUS_BADARG;
      } else {
        const int64_t p0 = ceil_div(L, bs);
        const int64_t p1 = ceil_div(static_cast<int64_t>(L) + n, bs);
        if (p1 > bt_stride) bad |= SKV_STATUS_MAX_PAGES;
        need = static_cast<int>(p1 - p0);
        nu = static_cast<int>(p1);
        first[b] = static_cast<int>(p0);
      }
    }
    int tot, utot;
    const int ex = block_exclusive_scan(need, scan_lds, &tot);
    const int uex = block_exclusive_scan(nu, scan_lds, &utot);
    if (b < batch) {
      off[b] = carry + ex;
      uoff[b] = ucarry + uex;
    }
    carry += tot;
    ucarry += utot;
  }
  const int top = *top_ptr;
  if (top < 0 || top > n_pages) bad |= SKV_STATUS_BADARG;
  else if (carry > top) bad |= SKV_STATUS_NOSPC;
  if (ucarry > max_units) bad |= SKV_STATUS_UNITS;
  if (bad) atomicOr(&bad_all, bad);
  __syncthreads();
  if (bad_all) {
    if (tid == 0) {
      units[0] = 0;  // the copy launch finds no work
      if (status) *status = bad_all;
    }
    return;
  }
  if (tid == 0) {
    off[batch] = carry;
    uoff[batch] = ucarry;
  }
  __syncthreads();
  for (int t = tid; t < carry; t += kReserveThreads) {
    int lo = 0, hi = batch;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (off[mid] <= t) lo = mid; else hi = mid;
    }
    bt[static_cast<int64_t>(lo) * bt_stride + first[lo] + (t - off[lo])] = stack[top - 1 - t];
  }
  // unit table (pages popped above are taken from the stack, not re-read from bt)
  for (int t = tid; t < ucarry; t += kReserveThreads) {
    int lo = 0, hi = batch;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (uoff[mid] <= t) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int k = t - uoff[b];
    const int L0 = lens[b];
    const int n = n_new ? n_new[b] : n_uni;
    const int L = L0 + n;
    const int32_t page = (k >= first[b]) ? stack[top - 1 - (off[b] + k - first[b])]
                                         : bt[static_cast<int64_t>(b) * bt_stride + k];
    const int64_t drow = (dst_off ? dst_off[b] : static_cast<int64_t>(b) * dst_seq_stride_rows) +
                         static_cast<int64_t>(k) * bs;
    int32_t* e = units + kUnitHeader + static_cast<int64_t>(t) * kUnitWords;
    e[0] = page;
    e[1] = b;
    e[2] = min(bs, L - k * bs);
    e[3] = L0 - k * bs;  // rows at or after this index of the unit are new
    e[4] = static_cast<int32_t>(drow & 0xffffffffll);
    e[5] = static_cast<int32_t>(drow >> 32);
  }
  __syncthreads();  // every thread read lens[] before it advances
  for (int b = tid; b < batch; b += kReserveThreads) lens[b] += n_new ? n_new[b] : n_uni;
  if (tid == 0) {
    *top_ptr = top - carry;
    units[0] = ucarry;
    if (status) *status = 0;
  }
}

struct SliceArgs {
  uint8_t* dst;
  int64_t dst_cap;
  uint8_t* pool;
  int64_t row_bytes;
  int bs;
  int64_t n_pages;
  const uint8_t* src;
  int64_t src_seq_stride;
  int64_t src_row_stride;
  int64_t src_len;
  const int32_t* units;
  int slices;  // 4 KB slices per page
};

__global__ __launch_bounds__(kSliceThreads) void k_copy_slices(SliceArgs a) {
  const int u = blockIdx.x / a.slices;
  const int s = blockIdx.x - u * a.slices;
  if (u >= a.units[0]) return;
  const int32_t* e = a.units + kUnitHeader + static_cast<int64_t>(u) * kUnitWords;
  const int32_t page = e[0];
  const int b = e[1];
  const int rows = e[2];
  const int new_row0 = e[3];
  const int64_t drow = (static_cast<int64_t>(static_cast<uint32_t>(e[4]))) | (static_cast<int64_t>(e[5]) << 32);
  const int row_chunks = static_cast<int>(a.row_bytes >> 4);
  const int c = s * kSliceThreads + threadIdx.x;
  if (c >= rows * row_chunks || page < 0 || page >= a.n_pages || drow < 0 || drow + rows > a.dst_cap) return;
  u32x4* pslot = reinterpret_cast<u32x4*>(a.pool + static_cast<int64_t>(page) * a.bs * a.row_bytes) + c;
  u32x4* dslot = reinterpret_cast<u32x4*>(a.dst + drow * a.row_bytes) + c;
  if (c >= max(new_row0, 0) * row_chunks) {
    const int r = c / row_chunks;
    const int i = r - new_row0;  // index among this call's new rows
    if (i >= a.src_len) return;
    const u32x4 v = *(reinterpret_cast<const u32x4*>(a.src + b * a.src_seq_stride + i * a.src_row_stride) +
                      (c - r * row_chunks));
    *pslot = v;
    st_stream(dslot, v);
  } else {
    st_stream(dslot, ld_stream(pslot));
  }
}

// ---------------------------------------------------------------------------
// Allocation-free decode step: the page-unit table of k_plan_units /
// k_copy_slices lives in a file-scope device array (one copy per GPU, held
// until the process ends) instead of a caller workspace.  Its host-side name
// is not a device address: host code uses only the per-device pointer that
// hipGetSymbolAddress returns.
// ---------------------------------------------------------------------------
static __device__ __align__(256) int32_t scratch[kUnitHeader + kUnitWords * SKV_NOALLOC_MAX_UNITS];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static int32_t* g_scratch[kMaxDevices];

// The unit table of the calling thread's current device (the stream's
// device), resolved once per device.
static int scratch_units(hipStream_t stream, int32_t** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(SKV_EHIP, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(SKV_EINVAL, "%s: device %d out of range", what, dev);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) {
      return set_error(SKV_EHIP, "%s: hipStreamGetDevice failed: %s", what, hipGetErrorString(e));
    }
    if (sdev != dev) {
      return set_error(SKV_EINVAL, "%s: the stream belongs to device %d, the current device is %d", what,
                       static_cast<int>(sdev), dev);
    }
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      return set_error(SKV_EHIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                       hipGetErrorString(e));
    }
    g_scratch[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch[dev];
  return SKV_OK;
}

}  // namespace skv

using namespace skv;

extern "C" int skv_free_stack_init(int32_t* free_stack, int32_t* free_top, const int32_t* order,
                                   int64_t n_pages, void* stream) {
  if (n_pages <= 0 || n_pages > INT32_MAX) {
    return set_error(SKV_EINVAL, "skv_free_stack_init: n_pages must be in [1, 2^31); got %lld",
                     (long long)n_pages);
  }
  if (!free_stack || !free_top) return set_error(SKV_EINVAL, "skv_free_stack_init: NULL buffer");
  const int threads = 256;
  const int64_t blocks = ceil_div(n_pages, threads);
  hipLaunchKernelGGL(k_free_stack_init, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), free_stack, free_top, order, n_pages);
  return check_launch("skv_free_stack_init");
}

extern "C" int skv_reserve(int32_t* free_stack, int32_t* free_top, int64_t n_pages, int32_t* block_table,
                           int64_t bt_stride, int64_t max_pages, int32_t* seq_lens,
                           const int32_t* n_new, int32_t n_new_uniform, int64_t batch,
                           int64_t block_size, int32_t* status, void* stream) {
  if (batch < 0 || batch > kMaxBatch) {
    return set_error(SKV_EINVAL, "skv_reserve: batch must be in [0, %d]; got %lld", kMaxBatch,
                     (long long)batch);
  }
  if (block_size <= 0 || bt_stride <= 0 || max_pages < 0 || max_pages > bt_stride) {
    return set_error(SKV_EINVAL,
                     "skv_reserve: need block_size > 0 and 0 <= max_pages <= bt_stride; got "
                     "block_size=%lld max_pages=%lld bt_stride=%lld",
                     (long long)block_size, (long long)max_pages, (long long)bt_stride);
  }
  if (!n_new && n_new_uniform < 0) {
    return set_error(SKV_EINVAL, "skv_reserve: n_new_uniform must be >= 0; got %d", n_new_uniform);
  }
  if (batch == 0) return SKV_OK;
  hipLaunchKernelGGL(k_reserve, dim3(1), dim3(kReserveThreads), 0, static_cast<hipStream_t>(stream),
                     free_stack, free_top, n_pages, block_table, bt_stride, max_pages, seq_lens, n_new,
                     n_new_uniform, static_cast<int>(batch), static_cast<int>(block_size), status);
  return check_launch("skv_reserve");
}

extern "C" int skv_paged_append(void* pool, int64_t row_bytes, int64_t block_size, int64_t n_pages,
                                const int32_t* block_table, int64_t bt_stride,
                                const int32_t* seq_lens, const int32_t* n_new, int32_t n_new_uniform,
                                const void* src, int64_t src_seq_stride, int64_t src_row_stride,
                                int64_t src_len, int64_t batch, void* stream) {
  int rc = validate_copy("skv_paged_append", row_bytes, block_size, batch, bt_stride, pool, pool);
  if (rc) return rc;
  if ((rc = validate_src("skv_paged_append", src, src_seq_stride, src_row_stride))) return rc;
  CopyArgs a{};
  a.pool = static_cast<uint8_t*>(pool);
  a.row_bytes = row_bytes;
  a.bs = static_cast<int>(block_size);
  a.n_pages = n_pages;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.lens = seq_lens;
  a.n_new = n_new;
  a.n_uni = n_new_uniform;
  a.src = static_cast<const uint8_t*>(src);
  a.src_seq_stride = src_seq_stride;
  a.src_row_stride = src_row_stride;
  a.src_len = src_len;
  a.batch = static_cast<int>(batch);
  return launch_copy<1>(a, static_cast<hipStream_t>(stream), "skv_paged_append");
}

extern "C" int skv_paged_gather(void* dst, const int64_t* dst_row_offsets,
                                int64_t dst_seq_stride_rows, int64_t dst_capacity_rows,
                                const void* pool, int64_t row_bytes, int64_t block_size,
                                int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                                const int32_t* seq_lens, int64_t batch, void* stream) {
  int rc = validate_copy("skv_paged_gather", row_bytes, block_size, batch, bt_stride, pool, dst);
  if (rc) return rc;
  CopyArgs a{};
  a.dst = static_cast<uint8_t*>(dst);
  a.dst_off = dst_row_offsets;
  a.dst_stride_rows = dst_seq_stride_rows;
  a.dst_cap = dst_capacity_rows;
  a.pool = static_cast<uint8_t*>(const_cast<void*>(pool));
  a.row_bytes = row_bytes;
  a.bs = static_cast<int>(block_size);
  a.n_pages = n_pages;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.lens = seq_lens;
  a.batch = static_cast<int>(batch);
  return launch_copy<0>(a, static_cast<hipStream_t>(stream), "skv_paged_gather");
}

extern "C" int skv_append_gather(void* dst, const int64_t* dst_row_offsets,
                                 int64_t dst_seq_stride_rows, int64_t dst_capacity_rows, void* pool,
                                 int64_t row_bytes, int64_t block_size, int64_t n_pages,
                                 const int32_t* block_table, int64_t bt_stride,
                                 const int32_t* seq_lens, const int32_t* n_new,
                                 int32_t n_new_uniform, const void* src, int64_t src_seq_stride,
                                 int64_t src_row_stride, int64_t src_len, int64_t batch,
                                 void* stream) {
  int rc = validate_copy("skv_append_gather", row_bytes, block_size, batch, bt_stride, pool, dst);
  if (rc) return rc;
  if ((rc = validate_src("skv_append_gather", src, src_seq_stride, src_row_stride))) return rc;
  CopyArgs a{};
  a.dst = static_cast<uint8_t*>(dst);
  a.dst_off = dst_row_offsets;
  a.dst_stride_rows = dst_seq_stride_rows;
  a.dst_cap = dst_capacity_rows;
  a.pool = static_cast<uint8_t*>(pool);
  a.row_bytes = row_bytes;
  a.bs = static_cast<int>(block_size);
  a.n_pages = n_pages;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.lens = seq_lens;
  a.n_new = n_new;
  a.n_uni = n_new_uniform;
  a.src = static_cast<const uint8_t*>(src);
  a.src_seq_stride = src_seq_stride;
  a.src_row_stride = src_row_stride;
  a.src_len = src_len;
  a.batch = static_cast<int>(batch);
  return launch_copy<2>(a, static_cast<hipStream_t>(stream), "skv_append_gather");
}

extern "C" int skv_plan_units(int32_t* free_stack, int32_t* free_top, int64_t n_pages,
                              int32_t* block_table, int64_t bt_stride, int32_t* seq_lens,
                              const int32_t* n_new, int32_t n_new_uniform, int32_t* status,
                              const int64_t* dst_row_offsets, int64_t dst_seq_stride_rows,
                              int64_t block_size, int32_t* units, int64_t max_units, int64_t batch,
                              void* stream) {
  const char* what = "skv_plan_units";
  if (batch < 0 || batch > kMaxBatch) {
    return set_error(SKV_EINVAL, "%s: batch must be in [0, %d]; got %lld", what, kMaxBatch, (long long)batch);
  }
  if (block_size <= 0 || bt_stride <= 0 || n_pages <= 0 || n_pages > INT32_MAX) {
    return set_error(SKV_EINVAL, "%s: bad block_size/bt_stride/n_pages", what);
  }
  if (!n_new && n_new_uniform < 0) return set_error(SKV_EINVAL, "%s: n_new_uniform must be >= 0", what);
  if (!units || max_units < 0 || max_units > INT32_MAX / kUnitWords) {
    return set_error(SKV_EINVAL, "%s: need a unit table and 0 <= max_units < 2^28", what);
  }
  if (batch == 0) return SKV_OK;
  hipLaunchKernelGGL(k_plan_units, dim3(1), dim3(kReserveThreads), 0, static_cast<hipStream_t>(stream),
                     free_stack, free_top, n_pages, block_table, bt_stride, seq_lens, n_new, n_new_uniform,
                     static_cast<int>(batch), static_cast<int>(block_size), dst_row_offsets,
                     dst_seq_stride_rows, units, max_units, status);
  return check_launch(what);
}

extern "C" int skv_copy_slices(void* dst, int64_t dst_capacity_rows, void* pool, int64_t row_bytes,
                               int64_t block_size, int64_t n_pages, const void* src,
                               int64_t src_seq_stride, int64_t src_row_stride, int64_t src_len,
                               const int32_t* units, int64_t max_units, void* stream) {
  const char* what = "skv_copy_slices";
  int rc = validate_copy(what, row_bytes, block_size, 0, 1, pool, dst);
  if (rc) return rc;
  if ((rc = validate_src(what, src, src_seq_stride, src_row_stride))) return rc;
  if (!units || max_units < 0 || max_units > INT32_MAX / kUnitWords) {
    return set_error(SKV_EINVAL, "%s: need a unit table and 0 <= max_units < 2^28", what);
  }
  SliceArgs a{};
  a.dst = static_cast<uint8_t*>(dst);
  a.dst_cap = dst_capacity_rows;
  a.pool = static_cast<uint8_t*>(pool);
  a.row_bytes = row_bytes;
  a.bs = static_cast<int>(block_size);
  a.n_pages = n_pages;
  a.src = static_cast<const uint8_t*>(src);
  a.src_seq_stride = src_seq_stride;
  a.src_row_stride = src_row_stride;
  a.src_len = src_len;
  a.units = units;
  a.slices = static_cast<int>(ceil_div(block_size * (row_bytes >> 4), kSliceThreads));
  const int64_t grid = max_units * a.slices;
  if (grid == 0) return SKV_OK;
  if (grid > INT32_MAX) return set_error(SKV_EINVAL, "%s: too many slices", what);
  hipLaunchKernelGGL(k_copy_slices, dim3(static_cast<unsigned>(grid)), dim3(kSliceThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch(what);
}

extern "C" int skv_decode_append_gather(int32_t* free_stack, int32_t* free_top, int64_t n_pages,
                                        int32_t* block_table, int64_t bt_stride, int32_t* seq_lens,
                                        const int32_t* n_new, int32_t n_new_uniform, int32_t* status,
                                        void* dst, const int64_t* dst_row_offsets,
                                        int64_t dst_seq_stride_rows, int64_t dst_capacity_rows,
                                        void* pool, int64_t row_bytes, int64_t block_size,
                                        const void* src, int64_t src_seq_stride,
                                        int64_t src_row_stride, int64_t src_len, int32_t* units,
                                        int64_t max_units, int64_t batch, void* stream) {
  const char* what = "skv_decode_append_gather";
  int rc = validate_copy(what, row_bytes, block_size, batch, bt_stride, pool, dst);
  if (rc) return rc;
  if ((rc = validate_src(what, src, src_seq_stride, src_row_stride))) return rc;
  if (batch == 0) return SKV_OK;
  rc = skv_plan_units(free_stack, free_top, n_pages, block_table, bt_stride, seq_lens, n_new,
                      n_new_uniform, status, dst_row_offsets, dst_seq_stride_rows, block_size, units,
                      max_units, batch, stream);
  if (rc) return rc;
  return skv_copy_slices(dst, dst_capacity_rows, pool, row_bytes, block_size, n_pages, src,
                         src_seq_stride, src_row_stride, src_len, units, max_units, stream);
}

extern "C" int skv_decode_append_gather_noalloc(
    int32_t* free_stack, int32_t* free_top, int64_t n_pages, int32_t* block_table, int64_t bt_stride,
    int32_t* seq_lens, const int32_t* n_new, int32_t n_new_uniform, int32_t* status, void* dst,
    const int64_t* dst_row_offsets, int64_t dst_seq_stride_rows, int64_t dst_capacity_rows, void* pool,
    int64_t row_bytes, int64_t block_size, const void* src, int64_t src_seq_stride,
    int64_t src_row_stride, int64_t src_len, int64_t max_units, int64_t batch, void* stream) {
  const char* what = "skv_decode_append_gather_noalloc";
  if (max_units < 0 || max_units > SKV_NOALLOC_MAX_UNITS) {
    return set_error(SKV_EINVAL, "%s: max_units must be in [0, %d] (the static unit table); got %lld", what,
                     SKV_NOALLOC_MAX_UNITS, (long long)max_units);
  }
  int rc = validate_copy(what, row_bytes, block_size, batch, bt_stride, pool, dst);
  if (rc) return rc;
  if ((rc = validate_src(what, src, src_seq_stride, src_row_stride))) return rc;
  if (batch == 0) return SKV_OK;
  int32_t* units = nullptr;
  if ((rc = scratch_units(static_cast<hipStream_t>(stream), &units, what))) return rc;
  // k_plan_units writes the table's count word on every path (0 on a
  // refusal), so nothing of the previous call's table is read.
  rc = skv_plan_units(free_stack, free_top, n_pages, block_table, bt_stride, seq_lens, n_new,
                      n_new_uniform, status, dst_row_offsets, dst_seq_stride_rows, block_size, units,
                      max_units, batch, stream);
  if (rc) return rc;
  return skv_copy_slices(dst, dst_capacity_rows, pool, row_bytes, block_size, n_pages, src,
                         src_seq_stride, src_row_stride, src_len, units, max_units, stream);
}
