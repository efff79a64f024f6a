// Sliding-window (SWA) ring buffer: W rows per sequence, slot = position % W.
//
// Reference semantics: the visible keys of a decode query at position L-1 are
// positions k with k <= L-1 and (L-1) - k < W (swa.py:119-125, csa.py:352-360,
// hca.py:143-153), i.e. the last min(W, L) tokens.  The reference keeps the
// full history and masks it; the ring keeps only those rows.
#include "skv_common.h"

namespace skv {

constexpr int kRingThreads = 256;
constexpr int kRingRowsPerBlock = 16;

struct RingArgs {
  uint8_t* ring;
  int64_t window;
  int64_t row_bytes;
  const int32_t* lens;  // token counts after the append
  const int32_t* n_new;
  int n_uni;
  const uint8_t* src;
  int64_t src_seq_stride;
  int64_t src_row_stride;
  int64_t src_len;
  uint8_t* dst;
  int64_t dst_seq_stride_rows;
  int64_t dst_cap;
  int batch;
};

// grid: (ceil(W / rows), batch).  Row slot r of the ring of sequence b.
__global__ __launch_bounds__(kRingThreads) void k_ring_append(RingArgs a) {
  const int b = blockIdx.y;
  const int L = a.lens[b];
  const int n = a.n_new ? a.n_new[b] : a.n_uni;
  // only the last min(n, W) new rows survive; write each surviving row once
  const int keep = static_cast<int>(min<int64_t>(n, a.window));
  const int row_chunks = static_cast<int>(a.row_bytes >> 4);
  const int r0 = blockIdx.x * kRingRowsPerBlock;
  const int r1 = min(keep, r0 + kRingRowsPerBlock);
  if (r0 >= r1 || L < n) return;
  const int total = (r1 - r0) * row_chunks;
  for (int c = threadIdx.x; c < total; c += kRingThreads) {
    const int rr = r0 + c / row_chunks;
    const int cc = c % row_chunks;
    const int i = n - keep + rr;              // new-row index
    if (i >= a.src_len) continue;
    const int64_t pos = static_cast<int64_t>(L) - n + i;
    const int64_t slot = pos % a.window;
    const u32x4 v = *(reinterpret_cast<const u32x4*>(a.src + b * a.src_seq_stride +
                                                     i * a.src_row_stride) + cc);
    *(reinterpret_cast<u32x4*>(a.ring + (b * a.window + slot) * a.row_bytes) + cc) = v;
  }
}

// grid: (ceil(W / rows), batch).  Output row r = position L - cnt + r.
__global__ __launch_bounds__(kRingThreads) void k_ring_read(RingArgs a) {
  const int b = blockIdx.y;
  const int L = a.lens[b];
  const int cnt = static_cast<int>(min<int64_t>(max(L, 0), a.window));
  const int row_chunks = static_cast<int>(a.row_bytes >> 4);
  const int r0 = blockIdx.x * kRingRowsPerBlock;
  const int r1 = min(cnt, r0 + kRingRowsPerBlock);
  if (r0 >= r1) return;
  const int64_t drow0 = static_cast<int64_t>(b) * a.dst_seq_stride_rows;
  if (drow0 + r1 > a.dst_cap) return;
  const int total = (r1 - r0) * row_chunks;
  for (int c = threadIdx.x; c < total; c += kRingThreads) {
    const int r = r0 + c / row_chunks;
    const int cc = c % row_chunks;
    const int64_t slot = (static_cast<int64_t>(L) - cnt + r) % a.window;
    const u32x4 v = *(reinterpret_cast<const u32x4*>(a.ring + (b * a.window + slot) * a.row_bytes) + cc);
    *(reinterpret_cast<u32x4*>(a.dst + (drow0 + r) * a.row_bytes) + cc) = v;
  }
}

static int validate_ring(const char* what, int64_t window, int64_t row_bytes, int64_t batch,
                         const void* ring) {
  if (window <= 0 || window > (1 << 20)) {
    return set_error(SKV_EINVAL, "%s: window must be in [1, 2^20]; got %lld", what,
                     (long long)window);
  }
  if (row_bytes <= 0 || (row_bytes & 15)) {
    return set_error(SKV_EINVAL, "%s: row_bytes must be a positive multiple of 16; got %lld",
                     what, (long long)row_bytes);
  }
  if (batch < 0 || batch > 65535) {
    return set_error(SKV_EINVAL, "%s: batch must be in [0, 65535]; got %lld", what,
                     (long long)batch);
  }
  if (reinterpret_cast<uintptr_t>(ring) & 15) {
    return set_error(SKV_EINVAL, "%s: ring must be 16-byte aligned", what);
  }
  return SKV_OK;
}

}  // namespace skv

using namespace skv;

extern "C" int skv_ring_append(void* ring, int64_t window, int64_t row_bytes,
                               const int32_t* seq_lens, const int32_t* n_new, int32_t n_new_uniform,
                               const void* src, int64_t src_seq_stride, int64_t src_row_stride,
                               int64_t src_len, int64_t batch, void* stream) {
  int rc = validate_ring("skv_ring_append", window, row_bytes, batch, ring);
  if (rc) return rc;
  if (!src || (reinterpret_cast<uintptr_t>(src) & 15) || (src_seq_stride & 15) ||
      (src_row_stride & 15)) {
    return set_error(SKV_EINVAL, "skv_ring_append: src pointer and strides must be 16-byte aligned");
  }
  if (!n_new && n_new_uniform < 0) {
    return set_error(SKV_EINVAL, "skv_ring_append: n_new_uniform must be >= 0");
  }
  if (batch == 0) return SKV_OK;
  RingArgs a{};
  a.ring = static_cast<uint8_t*>(ring);
  a.window = window;
  a.row_bytes = row_bytes;
  a.lens = seq_lens;
  a.n_new = n_new;
  a.n_uni = n_new_uniform;
  a.src = static_cast<const uint8_t*>(src);
  a.src_seq_stride = src_seq_stride;
  a.src_row_stride = src_row_stride;
  a.src_len = src_len;
  a.batch = static_cast<int>(batch);
  const dim3 grid(static_cast<unsigned>(ceil_div(window, kRingRowsPerBlock)),
                  static_cast<unsigned>(batch));
  hipLaunchKernelGGL(k_ring_append, grid, dim3(kRingThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("skv_ring_append");
}

extern "C" int skv_ring_read(void* dst, int64_t dst_seq_stride_rows, int64_t dst_capacity_rows,
                             const void* ring, int64_t window, int64_t row_bytes,
                             const int32_t* seq_lens, int64_t batch, void* stream) {
  int rc = validate_ring("skv_ring_read", window, row_bytes, batch, ring);
  if (rc) return rc;
  if (!dst || (reinterpret_cast<uintptr_t>(dst) & 15)) {
    return set_error(SKV_EINVAL, "skv_ring_read: dst must be 16-byte aligned");
  }
  if (batch == 0) return SKV_OK;
  RingArgs a{};
  a.ring = static_cast<uint8_t*>(const_cast<void*>(ring));
  a.window = window;
  a.row_bytes = row_bytes;
  a.lens = seq_lens;
  a.dst = static_cast<uint8_t*>(dst);
  a.dst_seq_stride_rows = dst_seq_stride_rows;
  a.dst_cap = dst_capacity_rows;
  a.batch = static_cast<int>(batch);
  const dim3 grid(static_cast<unsigned>(ceil_div(window, kRingRowsPerBlock)),
                  static_cast<unsigned>(batch));
  hipLaunchKernelGGL(k_ring_read, grid, dim3(kRingThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("skv_ring_read");
}
