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
// Here the buffered state is the per-token (c, z) pair of the incomplete block
// (the projections are per-token, so buffering them is equivalent to
// buffering h and projecting at emission).
#include "skv_entry.h"

namespace skv {

constexpr int kPoolWave = 64;
constexpr int kMaxGroups = 4;  // 8-channel groups per lane: channels <= 64*8*4 = 2048

struct CompressArgs {
  uint8_t* pool;
  int64_t entry_bytes;
  int bs;
  int64_t n_pages;
  const int32_t* bt;
  int64_t bt_stride;
  uint16_t* tail_c;
  uint16_t* tail_z;
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
};

// Row pointer of token position p of sequence b (tail slot or new input row).
__device__ __forceinline__ const uint16_t* token_row(const CompressArgs& a, const uint16_t* tail,
                                                     const uint8_t* in, int b, int64_t p,
                                                     int64_t first_new) {
  if (p < first_new) {
    return tail + (static_cast<int64_t>(b) * a.m + (p % a.m)) * a.channels;
  }
  const int64_t i = p - first_new;
  return reinterpret_cast<const uint16_t*>(in + b * a.in_seq_stride + i * a.in_row_stride);
}

// grid: (units, batch); block: one wave.  Unit k of sequence b pools completed
// block e0 + k; unit 0 then stages the incomplete block's new tokens.
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

  if (k < nb) {
    const int64_t e = e0 + k;
    float acc[kMaxGroups][8], mx[kMaxGroups][8], sum[kMaxGroups][8];
#pragma unroll
    for (int g = 0; g < kMaxGroups; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[g][j] = 0.f;
        mx[g][j] = -INFINITY;
        sum[g][j] = 0.f;
      }
    for (int i = 0; i < a.m; ++i) {
      const int64_t p = e * a.m + i;
      const uint16_t* crow = token_row(a, a.tail_c, a.c_new, b, p, first_new);
      const uint16_t* zrow = token_row(a, a.tail_z, a.z_new, b, p, first_new);
      const float* brow = a.bias + static_cast<int64_t>(i) * a.channels;
#pragma unroll
      for (int g = 0; g < kMaxGroups; ++g) {
        const int grp = lane + g * kPoolWave;
        if (grp >= groups) break;
        float c[8], z[8];
        unpack8_bf16(*reinterpret_cast<const u32x4*>(crow + grp * 8), c);
        unpack8_bf16(*reinterpret_cast<const u32x4*>(zrow + grp * 8), z);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = z[j] + brow[grp * 8 + j];
          // online softmax over the m tokens of this channel
          if (v > mx[g][j]) {
            const float s = expf(mx[g][j] - v);
            sum[g][j] = sum[g][j] * s + 1.f;
            acc[g][j] = acc[g][j] * s + c[j];
            mx[g][j] = v;
          } else {
            const float w = expf(v - mx[g][j]);
            sum[g][j] += w;
            acc[g][j] += w * c[j];
          }
        }
      }
    }
    const int64_t page_idx = e / a.bs;
    const int32_t page = (page_idx < a.bt_stride) ? a.bt[b * a.bt_stride + page_idx] : -1;
    if (page >= 0 && page < a.n_pages) {
      uint8_t* entry = a.pool + (static_cast<int64_t>(page) * a.bs + e % a.bs) * a.entry_bytes;
#pragma unroll
      for (int g = 0; g < kMaxGroups; ++g) {
        const int grp = lane + g * kPoolWave;
        // every lane takes part in the shuffles; only lanes with a group store
        float out[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float r = (grp < groups) ? acc[g][j] / sum[g][j] : 0.f;
          out[j] = bf16_to_f32(f32_to_bf16(r));  // the compressor emits bf16 entries
        }
        store_entry_group(entry, out, grp, groups, a.format, a.fp8_main);
      }
    }
  }

  if (k == 0) {
    // Stage the new tokens of the still-incomplete block e1 (positions >= e1*m).
    // Each lane rewrites only the channels it read above, after its own loads.
    __syncthreads();
    const int64_t p0 = max(first_new, e1 * a.m);
    for (int64_t p = p0; p < L; ++p) {
      const int64_t i = p - first_new;
      const int64_t slot = (static_cast<int64_t>(b) * a.m + (p % a.m)) * a.channels;
      const uint16_t* crow = reinterpret_cast<const uint16_t*>(a.c_new + b * a.in_seq_stride + i * a.in_row_stride);
      const uint16_t* zrow = reinterpret_cast<const uint16_t*>(a.z_new + b * a.in_seq_stride + i * a.in_row_stride);
      for (int grp = lane; grp < groups; grp += kPoolWave) {
        *reinterpret_cast<u32x4*>(a.tail_c + slot + grp * 8) = *reinterpret_cast<const u32x4*>(crow + grp * 8);
        *reinterpret_cast<u32x4*>(a.tail_z + slot + grp * 8) = *reinterpret_cast<const u32x4*>(zrow + grp * 8);
      }
    }
  }
}

}  // namespace skv

using namespace skv;

extern "C" int skv_compress_append(void* pool, int64_t entry_bytes, int64_t block_size,
                                   int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                                   void* tail_c, void* tail_z, const void* c_new, const void* z_new,
                                   int64_t in_seq_stride, int64_t in_row_stride, int64_t in_len,
                                   const float* bias, const int32_t* seq_lens, const int32_t* n_new,
                                   int32_t n_new_uniform, int64_t m, int64_t channels,
                                   int32_t format, int64_t batch, void* stream) {
  const char* what = "skv_compress_append";
  if (m <= 0 || m > 4096) return set_error(SKV_EINVAL, "%s: compression_rate must be in [1, 4096]; got %lld", what, (long long)m);
  if (channels <= 0 || (channels & 7) || channels > kPoolWave * 8 * kMaxGroups) {
    return set_error(SKV_EINVAL, "%s: channels must be a multiple of 8 in [8, %d]; got %lld", what,
                     kPoolWave * 8 * kMaxGroups, (long long)channels);
  }
  if (block_size <= 0 || bt_stride <= 0 || batch < 0 || batch > 65535) {
    return set_error(SKV_EINVAL, "%s: bad block_size/bt_stride/batch", what);
  }
  const int fp8_main = entry_layout(format, channels, entry_bytes);
  if (fp8_main < 0) {
    return set_error(SKV_EINVAL,
                     "%s: entry_bytes %lld does not match format %d with %lld channels (bf16: 2*channels; "
                     "fp8: channels = 128*q + %d, entry_bytes = %lld)",
                     what, (long long)entry_bytes, format, (long long)channels, SKV_FP8_ROPE_DIMS,
                     (long long)SKV_FP8_ENTRY_BYTES(channels));
  }
  const uintptr_t align = reinterpret_cast<uintptr_t>(pool) | reinterpret_cast<uintptr_t>(tail_c) |
                          reinterpret_cast<uintptr_t>(tail_z) | reinterpret_cast<uintptr_t>(c_new) |
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
  a.tail_c = static_cast<uint16_t*>(tail_c);
  a.tail_z = static_cast<uint16_t*>(tail_z);
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
  // at most floor((in_len + m - 1) / m) + 1 blocks complete in one call
  const int64_t units = (in_len + m - 1) / m + 1;
  if (units > INT32_MAX) return set_error(SKV_EINVAL, "%s: in_len too large", what);
  hipLaunchKernelGGL(k_compress_append, dim3(static_cast<unsigned>(units), static_cast<unsigned>(batch)),
                     dim3(kPoolWave), 0, static_cast<hipStream_t>(stream), a);
  return check_launch(what);
}
