// FP8 e4m3fn quantize-on-write for paged entries (1x128 blocks, fp32 scale).
//
// Reference semantics: cast_to_fp8(x.reshape(-1, 128), axis=0) from
// packages/kernels/src/saint_llm_kernels/quant/reference.py:75-111:
//   scale = max(amax(|x|) / 448, FLT_MIN);  q = clamp(x / scale, -448, 448)
//   code  = q.to(float8_e4m3fn)  (round to nearest even)
// The 64 rope dims of each entry are kept in bf16 (mixed-precision storage
// planned in saint_llm_inference/__init__.py:9).
#include "skv_entry.h"

namespace skv {

constexpr int kQuantWave = 64;

struct QuantAppendArgs {
  uint8_t* pool;
  int64_t entry_bytes;
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
  int64_t src_len;
  int channels;
  int fp8_main;
};

// grid: (src rows, batch); block: one wave per row.
__global__ __launch_bounds__(kQuantWave) void k_fp8_quant_append(QuantAppendArgs a) {
  const int b = blockIdx.y;
  const int i = blockIdx.x;
  const int64_t L = a.lens[b];
  const int64_t n = a.n_new ? a.n_new[b] : a.n_uni;
  if (i >= n || n > L || i >= a.src_len) return;
  const int64_t pos = L - n + i;
  const int64_t p = pos / a.bs;
  const int32_t page = (p < a.bt_stride) ? a.bt[b * a.bt_stride + p] : -1;
  if (page < 0 || page >= a.n_pages) return;
  uint8_t* entry = a.pool + (static_cast<int64_t>(page) * a.bs + pos % a.bs) * a.entry_bytes;
  const uint16_t* row = reinterpret_cast<const uint16_t*>(a.src + b * a.src_seq_stride + i * a.src_row_stride);
  const int groups = a.channels >> 3;
  for (int g0 = 0; g0 < groups; g0 += kQuantWave) {
    const int grp = g0 + threadIdx.x;
    float v[8];
    if (grp < groups) {
      unpack8_bf16(*reinterpret_cast<const u32x4*>(row + grp * 8), v);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.f;
    }
    store_entry_group(entry, v, grp, groups, SKV_FMT_FP8, a.fp8_main);
  }
}

}  // namespace skv

using namespace skv;

extern "C" int skv_fp8_quant_append(void* pool, int64_t entry_bytes, int64_t block_size,
                                    int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                                    const int32_t* seq_lens, const int32_t* n_new,
                                    int32_t n_new_uniform, const void* src, int64_t src_seq_stride,
                                    int64_t src_row_stride, int64_t src_len, int64_t channels,
                                    int64_t batch, void* stream) {
  const char* what = "skv_fp8_quant_append";
  const int fp8_main = entry_layout(SKV_FMT_FP8, channels, entry_bytes);
  if (fp8_main <= 0) {
    return set_error(SKV_EINVAL, "%s: fp8 entries need channels = 128*q + %d and entry_bytes = %lld; got channels=%lld entry_bytes=%lld",
                     what, SKV_FP8_ROPE_DIMS, (long long)SKV_FP8_ENTRY_BYTES(channels),
                     (long long)channels, (long long)entry_bytes);
  }
  if (block_size <= 0 || bt_stride <= 0 || batch < 0 || batch > 65535 || src_len < 0 ||
      src_len > INT32_MAX) {
    return set_error(SKV_EINVAL, "%s: bad block_size/bt_stride/batch/src_len", what);
  }
  if ((reinterpret_cast<uintptr_t>(pool) | reinterpret_cast<uintptr_t>(src) |
       static_cast<uintptr_t>(src_seq_stride) | static_cast<uintptr_t>(src_row_stride)) & 15) {
    return set_error(SKV_EINVAL, "%s: pool, src and strides must be 16-byte aligned", what);
  }
  if (!n_new && n_new_uniform < 0) return set_error(SKV_EINVAL, "%s: n_new_uniform must be >= 0", what);
  if (batch == 0 || src_len == 0) return SKV_OK;
  QuantAppendArgs a{};
  a.pool = static_cast<uint8_t*>(pool);
  a.entry_bytes = entry_bytes;
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
  a.channels = static_cast<int>(channels);
  a.fp8_main = fp8_main;
  hipLaunchKernelGGL(k_fp8_quant_append, dim3(static_cast<unsigned>(src_len), static_cast<unsigned>(batch)),
                     dim3(kQuantWave), 0, static_cast<hipStream_t>(stream), a);
  return check_launch(what);
}

// Host-side entry to the same e4m3fn encoder the kernels use, so that the
// codec can be checked exhaustively on a CPU-only host.  Not a compute path.
extern "C" int skv_fp8_encode_host(const float* x, uint8_t* codes, int64_t n) {
  if (n < 0 || (n > 0 && (!x || !codes))) return set_error(SKV_EINVAL, "skv_fp8_encode_host: bad buffers");
  for (int64_t i = 0; i < n; ++i) codes[i] = f32_to_e4m3fn(x[i]);
  return SKV_OK;
}

extern "C" int skv_fp8_decode_host(const uint8_t* codes, float* x, int64_t n) {
  if (n < 0 || (n > 0 && (!x || !codes))) return set_error(SKV_EINVAL, "skv_fp8_decode_host: bad buffers");
  for (int64_t i = 0; i < n; ++i) x[i] = e4m3fn_to_f32(codes[i]);
  return SKV_OK;
}
