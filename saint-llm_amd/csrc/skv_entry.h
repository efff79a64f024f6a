// Writing one compressed entry from a wave: every lane holds 8 consecutive
// channels (groups lane, lane+64, ...) as fp32 already rounded to bf16.
//
// bf16 format : the 2*channels bytes of the entry are the bf16 values.
// fp32 format : the 4*channels bytes of the entry are the fp32 values (the
//               values are not rounded).
// fp8 format  : [main e4m3fn codes][main/128 fp32 scales][rope bf16], with
//               main = channels - SKV_FP8_ROPE_DIMS; each 128-channel block is
//               16 lanes of the wave.  scale = max(amax / 448, FLT_MIN),
//               code = RNE_e4m3fn(clamp(x / scale, -448, 448))
//               (quant/reference.py:75-79, 109-110).
#pragma once

#include "skv_common.h"

namespace skv {

__device__ __forceinline__ u32x4 pack8_bf16(const float* f) {
  u32x4 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = bf16_pack2(f[2 * q], f[2 * q + 1]);
  return v;
}

__device__ __forceinline__ void unpack8_bf16(u32x4 v, float* f) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = bf16_to_f32(static_cast<uint16_t>(v[q] & 0xffffu));
    f[2 * q + 1] = bf16_to_f32(static_cast<uint16_t>(v[q] >> 16));
  }
}

// Store channel group `grp` (8 values) of an entry.  Must be reached by all
// 64 lanes of the wave with the same `grp - lane` (the fp8 path shuffles
// across the 16 lanes of a 128-channel block).  Lanes with grp >= groups
// take part in no shuffle group that matters and store nothing.
__device__ __forceinline__ void store_entry_group(uint8_t* entry, const float* v, int grp,
                                                  int groups, int format, int fp8_main) {
  if (format == SKV_FMT_F32) {
    if (grp < groups) {
      u32x4 lo, hi;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[j] = __float_as_uint(v[j]);
        hi[j] = __float_as_uint(v[j + 4]);
      }
      *reinterpret_cast<u32x4*>(entry + grp * 32) = lo;
      *reinterpret_cast<u32x4*>(entry + grp * 32 + 16) = hi;
    }
    return;
  }
  if (format == SKV_FMT_BF16) {
    if (grp < groups) *reinterpret_cast<u32x4*>(entry + grp * 16) = pack8_bf16(v);
    return;
  }
  if (grp * 8 < fp8_main) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) amax = fmaxf(amax, __shfl_xor(amax, d, 16));
    const float scale = fmaxf(amax / kE4M3Max, kF32Tiny);
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = fminf(fmaxf(v[j] / scale, -kE4M3Max), kE4M3Max);
    u32x2 codes;
    codes[0] = e4m3fn_pack2<true>(q[2], q[3], e4m3fn_pack2<false>(q[0], q[1], 0u));
    codes[1] = e4m3fn_pack2<true>(q[6], q[7], e4m3fn_pack2<false>(q[4], q[5], 0u));
    *reinterpret_cast<u32x2*>(entry + grp * 8) = codes;
    if ((grp & 15) == 0) *reinterpret_cast<float*>(entry + fp8_main + (grp >> 4) * 4) = scale;
  } else if (grp < groups) {
    const int64_t off = fp8_main + (fp8_main >> 7) * 4 + (grp * 8 - fp8_main) * 2;
    *reinterpret_cast<u32x4*>(entry + off) = pack8_bf16(v);
  }
}

// Validate (format, channels, entry_bytes); returns fp8_main (0 for bf16) or -1.
inline int entry_layout(int format, int64_t channels, int64_t entry_bytes) {
  if (channels <= 0 || (channels & 7)) return -1;
  if (format == SKV_FMT_BF16) return entry_bytes == channels * 2 ? 0 : -1;
  if (format == SKV_FMT_FP8) {
    const int64_t main = channels - SKV_FP8_ROPE_DIMS;
    if (main <= 0 || (main % 128) || entry_bytes != SKV_FP8_ENTRY_BYTES(channels)) return -1;
    return static_cast<int>(main);
  }
  return -1;
}

}  // namespace skv
