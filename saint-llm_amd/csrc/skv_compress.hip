// Token compression: softmax-weighted pooling of every m tokens into one
// compressed entry, written straight into the paged compressed cache (bf16, or
// FP8 e4m3fn with a 1x128 fp32 scale), plus staging of the incomplete block.
//
// Reference semantics:
//   TokenLevelCompressor.forward (csa.py:66-88):
//     z = z_b + bias_b ; w = softmax(z, dim=tokens) ; out = sum_tokens(w * c_b)
//   HCA/CSA append state machine (kv_cache.py:171-195, 291-315):
//     combined = cat(h_buffer[:, :cnt], h_new); n_complete = total // m;
//     blocks -> compressed[:, nb:nb+n_complete]; leftover -> h_buffer
//   FP8 quantize-on-write (quant/reference.py:75-110) on each 128-dim block.
// Here the buffered state of the incomplete block is the running online-softmax
// state of each channel (max, sum, weighted sum; fp32 [batch, 3, channels]),
// so a decode step costs O(channels) whatever m is, and a block emits from
// that state the same value a one-shot pooling of its m tokens gives.
#include "skv_pool_state.h"

namespace skv {

struct CompressArgs {
  uint8_t* pool;
  int64_t entry_bytes;
  int bs;
  int64_t n_pages;
  const int32_t* bt;
  int64_t bt_stride;
  float* state;  // [batch, 3, channels]: running max, sum of weights, weighted sum
  const uint8_t* c_new;
  const uint8_t* z_new;
  int64_t in_seq_stride;
  int64_t in_row_stride;
  int64_t in_len;
  const float* bias;
  const int32_t* lens;
  const int32_t* n_new;
  int n_uni;
  int m;
  int channels;
  int format;
  int fp8_main;  // main (quantized) channels in FP8 format
  int in_f32;    // c/z rows are fp32
};

__device__ __forceinline__ void state_emit(const PoolState& st, const CompressArgs& a, int b, int64_t e,
                                           int lane, int groups) {
  const int64_t page_idx = e / a.bs;
  const int32_t page = (page_idx < a.bt_stride) ? a.bt[b * a.bt_stride + page_idx] : -1;
  if (page < 0 || page >= a.n_pages) return;  // wave-uniform
  uint8_t* entry = a.pool + (static_cast<int64_t>(page) * a.bs + e % a.bs) * a.entry_bytes;
  state_emit_entry(st, entry, lane, groups, a.format, a.fp8_main);
}

// Token rows [p0, p1) of sequence b (all new in this call) folded into st.
__device__ __forceinline__ void fold_tokens(PoolState& st, const CompressArgs& a, int b, int64_t first_new,
                                            int64_t p0, int64_t p1, int lane, int groups) {
  for (int64_t p = p0; p < p1; ++p) {
    const int64_t i = p - first_new;
    const uint8_t* crow = a.c_new + b * a.in_seq_stride + i * a.in_row_stride;
    const uint8_t* zrow = a.z_new + b * a.in_seq_stride + i * a.in_row_stride;
    const float* brow = a.bias + (p % a.m) * a.channels;
    if (a.in_f32) {  // uniform: fp32 rows
      state_update(st, reinterpret_cast<const float*>(crow), reinterpret_cast<const float*>(zrow), brow, lane,
                   groups);
    } else {
      state_update(st, reinterpret_cast<const uint16_t*>(crow), reinterpret_cast<const uint16_t*>(zrow), brow,
                   lane, groups);
    }
  }
}

// grid: (units, batch); block: one wave.
//   unit 0      : block e0 (continuing from the stored state when the previous
//                 call left it incomplete); then, if further blocks complete and
//                 the last one stays incomplete, the state of that last block.
//   unit k >= 1 : complete block e0 + k (only new tokens).
// Only unit 0 touches the state buffer of its sequence.
__global__ __launch_bounds__(kPoolWave) void k_compress_append(CompressArgs a) {
  const int b = blockIdx.y;
  const int k = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t L = a.lens[b];
  const int64_t n = a.n_new ? a.n_new[b] : a.n_uni;
  if (n <= 0 || n > L || n > a.in_len) return;
  const int64_t first_new = L - n;
  const int64_t e0 = first_new / a.m;
  const int64_t e1 = L / a.m;  // entries [e0, e1) complete in this call
  const int64_t nb = e1 - e0;
  if (k >= max<int64_t>(nb, 1)) return;
  const int groups = a.channels >> 3;
  float* sbase = a.state + static_cast<int64_t>(b) * 3 * a.channels;
  PoolState st;
  if (k == 0) {
    if (first_new % a.m != 0) {
      state_load(st, sbase, a.channels, lane, groups);
    } else {
      state_reset(st);
    }
    const int64_t p1 = min(L, (e0 + 1) * a.m);
    fold_tokens(st, a, b, first_new, first_new, p1, lane, groups);
    if (p1 == (e0 + 1) * a.m) {
      state_emit(st, a, b, e0, lane, groups);
      if (nb >= 1 && L % a.m != 0) {
        // the incomplete last block e1 starts fresh; its state replaces the
        // one loaded above (same lanes, after the loads retired)
        __syncthreads();
        state_reset(st);
        fold_tokens(st, a, b, first_new, e1 * a.m, L, lane, groups);
        state_store(st, sbase, a.channels, lane, groups);
      }
    } else {
      state_store(st, sbase, a.channels, lane, groups);
    }
    return;
  }
  const int64_t e = e0 + k;
  state_reset(st);
  fold_tokens(st, a, b, first_new, e * a.m, (e + 1) * a.m, lane, groups);
  state_emit(st, a, b, e, lane, groups);
}

}  // namespace skv

using namespace skv;

extern "C" int skv_compress_append(void* pool, int64_t entry_bytes, int64_t block_size,
                                   int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                                   float* tail_state, const void* c_new, const void* z_new,
                                   int64_t in_seq_stride, int64_t in_row_stride, int64_t in_len,
                                   const float* bias, const int32_t* seq_lens, const int32_t* n_new,
                                   int32_t n_new_uniform, int64_t m, int64_t channels,
                                   int32_t format, int64_t batch, void* stream) {
  const char* what = "skv_compress_append";
  const bool in_f32 = (format & SKV_FMT_IN_F32) || (format & ~SKV_FMT_IN_F32) == SKV_FMT_F32;
  format &= ~SKV_FMT_IN_F32;
  if (m <= 0 || m > 4096) return set_error(SKV_EINVAL, "%s: compression_rate must be in [1, 4096]; got %lld", what, (long long)m);
  if (channels <= 0 || (channels & 7) || channels > kPoolWave * 8 * kMaxGroups) {
    return set_error(SKV_EINVAL, "%s: channels must be a multiple of 8 in [8, %d]; got %lld", what,
                     kPoolWave * 8 * kMaxGroups, (long long)channels);
  }
  if (block_size <= 0 || bt_stride <= 0 || batch < 0 || batch > 65535) {
    return set_error(SKV_EINVAL, "%s: bad block_size/bt_stride/batch", what);
  }
  const int fp8_main = (format == SKV_FMT_F32) ? ((entry_bytes == channels * 4) ? 0 : -1)
                                               : entry_layout(format, channels, entry_bytes);
  if (fp8_main < 0) {
    return set_error(SKV_EINVAL,
                     "%s: entry_bytes %lld does not match format %d with %lld channels (bf16: 2*channels; "
                     "fp32: 4*channels; fp8: channels = 128*q + %d, entry_bytes = %lld)",
                     what, (long long)entry_bytes, format, (long long)channels, SKV_FP8_ROPE_DIMS,
                     (long long)SKV_FP8_ENTRY_BYTES(channels));
  }
  const uintptr_t align = reinterpret_cast<uintptr_t>(pool) | reinterpret_cast<uintptr_t>(tail_state) |
                          reinterpret_cast<uintptr_t>(c_new) |
                          reinterpret_cast<uintptr_t>(z_new) | static_cast<uintptr_t>(in_seq_stride) |
                          static_cast<uintptr_t>(in_row_stride);
  if (align & 15) return set_error(SKV_EINVAL, "%s: pointers and strides must be 16-byte aligned", what);
  if (!bias || (reinterpret_cast<uintptr_t>(bias) & 3)) return set_error(SKV_EINVAL, "%s: bias must be fp32", what);
  if (!n_new && n_new_uniform < 0) return set_error(SKV_EINVAL, "%s: n_new_uniform must be >= 0", what);
  if (batch == 0 || in_len <= 0) return SKV_OK;
  CompressArgs a{};
  a.pool = static_cast<uint8_t*>(pool);
  a.entry_bytes = entry_bytes;
  a.bs = static_cast<int>(block_size);
  a.n_pages = n_pages;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.state = tail_state;
  a.c_new = static_cast<const uint8_t*>(c_new);
  a.z_new = static_cast<const uint8_t*>(z_new);
  a.in_seq_stride = in_seq_stride;
  a.in_row_stride = in_row_stride;
  a.in_len = in_len;
  a.bias = bias;
  a.lens = seq_lens;
  a.n_new = n_new;
  a.n_uni = n_new_uniform;
  a.m = static_cast<int>(m);
  a.channels = static_cast<int>(channels);
  a.format = format;
  a.fp8_main = fp8_main;
  a.in_f32 = in_f32 ? 1 : 0;
  // at most floor((in_len + m - 1) / m) + 1 blocks complete in one call
  const int64_t units = (in_len + m - 1) / m + 1;
  if (units > INT32_MAX) return set_error(SKV_EINVAL, "%s: in_len too large", what);
  hipLaunchKernelGGL(k_compress_append, dim3(static_cast<unsigned>(units), static_cast<unsigned>(batch)),
                     dim3(kPoolWave), 0, static_cast<hipStream_t>(stream), a);
  return check_launch(what);
}
