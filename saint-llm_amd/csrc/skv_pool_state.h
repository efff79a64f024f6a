// Online-softmax pooling state of one compressed entry, held by one wave:
// lane l owns channel groups l, l+64, ... (8 channels each).  Pooling of a
// block of m tokens (TokenLevelCompressor, csa.py:81-87):
//   v_i = z_i + bias_i ; out = sum_i exp(v_i) c_i / sum_i exp(v_i)
// folded token by token with the running max for stability.
#pragma once

#include "skv_entry.h"

namespace skv {

constexpr int kPoolWave = 64;
constexpr int kMaxGroups = 4;  // 8-channel groups per lane: channels <= 64*8*4 = 2048

struct PoolState {
  float mx[kMaxGroups][8];
  float sum[kMaxGroups][8];
  float acc[kMaxGroups][8];
};

__device__ __forceinline__ void state_reset(PoolState& st) {
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      st.mx[g][j] = -INFINITY;
      st.sum[g][j] = 0.f;
      st.acc[g][j] = 0.f;
    }
}

__device__ __forceinline__ void state_load(PoolState& st, const float* base, int channels, int lane,
                                           int groups) {
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g) {
    const int grp = lane + g * kPoolWave;
    if (grp >= groups) break;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      st.mx[g][j] = base[grp * 8 + j];
      st.sum[g][j] = base[channels + grp * 8 + j];
      st.acc[g][j] = base[2 * channels + grp * 8 + j];
    }
  }
}

__device__ __forceinline__ void state_store(const PoolState& st, float* base, int channels, int lane,
                                            int groups) {
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g) {
    const int grp = lane + g * kPoolWave;
    if (grp >= groups) break;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      base[grp * 8 + j] = st.mx[g][j];
      base[channels + grp * 8 + j] = st.sum[g][j];
      base[2 * channels + grp * 8 + j] = st.acc[g][j];
    }
  }
}

// The 8 channels of group grp of a bf16 (uint16_t) or fp32 token row.
__device__ __forceinline__ void load8(const uint16_t* row, int grp, float* f) {
  unpack8_bf16(*reinterpret_cast<const u32x4*>(row + grp * 8), f);
}
__device__ __forceinline__ void load8(const float* row, int grp, float* f) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(row + grp * 8);
  const u32x4 hi = *reinterpret_cast<const u32x4*>(row + grp * 8 + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = __uint_as_float(lo[j]);
    f[j + 4] = __uint_as_float(hi[j]);
  }
}

// Fold token (c, z) rows (bf16 or fp32) with bias row `brow` into the running
// state: online softmax over the tokens of the block, per channel.
template <class Row>
__device__ __forceinline__ void state_update(PoolState& st, const Row* crow, const Row* zrow,
                                             const float* brow, int lane, int groups) {
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g) {
    const int grp = lane + g * kPoolWave;
    if (grp >= groups) break;
    float c[8], z[8];
    load8(crow, grp, c);
    load8(zrow, grp, z);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = z[j] + brow[grp * 8 + j];
      if (v > st.mx[g][j]) {
        const float s = expf(st.mx[g][j] - v);
        st.sum[g][j] = st.sum[g][j] * s + 1.f;
        st.acc[g][j] = st.acc[g][j] * s + c[j];
        st.mx[g][j] = v;
      } else {
        const float w = expf(v - st.mx[g][j]);
        st.sum[g][j] += w;
        st.acc[g][j] += w * c[j];
      }
    }
  }
}

// Write acc/sum (rounded to bf16, except for fp32 entries) as one entry; see
// store_entry_group.
__device__ __forceinline__ void state_emit_entry(const PoolState& st, uint8_t* entry, int lane, int groups,
                                                 int format, int fp8_main) {
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g) {
    const int grp = lane + g * kPoolWave;
    // every lane takes part in the fp8 shuffles; only lanes with a group store
    float out[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = (grp < groups) ? st.acc[g][j] / st.sum[g][j] : 0.f;
    if (format != SKV_FMT_F32) {
#pragma unroll
      for (int j = 0; j < 8; j += 2) bf16_round2(out[j], out[j + 1]);  // a bf16 compressor's entries
    }
    store_entry_group(entry, out, grp, groups, format, fp8_main);
  }
}

}  // namespace skv
