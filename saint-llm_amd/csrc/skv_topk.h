// Top-k selection of one score row by one 1024-thread workgroup.
//
// Radix select (8 bits per pass) on order-preserving uint32 keys finds the
// threshold key T of rank `sel`; keys > T and the lowest-index keys == T are
// collected, then ranked by (key descending, index ascending).  Rows with at
// most kLdsKeys valid scores are staged in LDS, longer rows re-read global
// memory (L2-resident) on each pass.
#pragma once

#include "skv_common.h"

namespace skv {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;
constexpr int kLdsKeys = 28672;  // rows with at most this many valid scores are staged in LDS
constexpr int kMaxTopK = 2048;

constexpr uint32_t kKeyNaN = 0xffffffffu;
constexpr uint32_t kKeyPosInf = 0xff800000u;
constexpr uint32_t kKeyNegInf = 0x007fffffu;

// Order-preserving map fp32 -> uint32 (larger float -> larger key); -0.0 is
// folded onto +0.0 and every NaN onto the largest key (torch.topk ranks NaN
// above +inf).
__device__ __forceinline__ uint32_t score_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return kKeyNaN;
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ bool key_finite(uint32_t k) {
  return k != kKeyNaN && k != kKeyPosInf && k != kKeyNegInf;
}

struct TopkSmem {
  uint32_t keys[kLdsKeys];
  int whist[kTopkWaves][256];
  int hist[256];
  uint32_t cand_key[kMaxTopK];
  int cand_idx[kMaxTopK];
  int scan_lds[17];
  int digit, above, cnt;
};

// out[0, k): the sel = min(k, n_cols, n_valid) best of row[0, n_valid) in
// (score desc, index asc) order, -1 for non-finite picks and ranks >= sel.
// Every thread of the workgroup must call it (it synchronises).
__device__ __forceinline__ void topk_row(TopkSmem& sm, const float* row, int n_cols, int n_valid, int k,
                                         int32_t* out) {
  const int tid = threadIdx.x;
  const int wid = tid / kWave;
  n_cols = max(n_cols, 0);
  n_valid = max(0, min(n_valid, n_cols));
  const int k_eff = min(k, n_cols);
  const int sel = min(k_eff, n_valid);
  for (int j = sel + tid; j < k; j += kTopkThreads) out[j] = -1;
  if (sel == 0) return;
  const bool in_lds = n_valid <= kLdsKeys;
  if (in_lds) {
    for (int i = tid; i < n_valid; i += kTopkThreads) sm.keys[i] = score_key(row[i]);
    __syncthreads();
  }
  auto key_at = [&](int i) -> uint32_t { return in_lds ? sm.keys[i] : score_key(row[i]); };

  // ---- radix select: the sel-th largest key, 8 bits per pass ---------------
  uint32_t prefix = 0, pmask = 0;
  int remaining = sel;  // rank (1-based) of the target among keys matching prefix
  int eq_total = 0;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < kTopkWaves * 256; i += kTopkThreads) (&sm.whist[0][0])[i] = 0;
    __syncthreads();
    for (int i = tid; i < n_valid; i += kTopkThreads) {
      const uint32_t key = key_at(i);
      if ((key & pmask) == prefix) atomicAdd(&sm.whist[wid][(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid < 256) {
      int s = 0;
#pragma unroll
      for (int w = 0; w < kTopkWaves; ++w) s += sm.whist[w][tid];
      sm.hist[tid] = s;
    }
    __syncthreads();
    // suffix counts: above(d) = sum of sm.hist[d+1..255]; thread t owns bin 255-t
    {
      const int bin = 255 - tid;
      const int v = (tid < 256) ? sm.hist[bin] : 0;
      int tot;
      const int ex = block_exclusive_scan(v, sm.scan_lds, &tot);  // count of bins > bin
      if (tid < 256 && ex < remaining && remaining <= ex + v) {
        sm.digit = bin;
        sm.above = ex;
      }
      __syncthreads();
    }
    const int d = sm.digit;
    remaining -= sm.above;
    prefix |= static_cast<uint32_t>(d) << shift;
    pmask |= 255u << shift;
    eq_total = sm.hist[d];
    __syncthreads();
  }
  const uint32_t T = prefix;
  const int need_eq = remaining;  // keys == T to take (smallest indices first)
  const int n_gt = sel - need_eq;

  // ---- collect the sel winners ------------------------------------------------
  if (tid == 0) sm.cnt = 0;
  __syncthreads();
  for (int i = tid; i < n_valid; i += kTopkThreads) {
    const uint32_t key = key_at(i);
    if (key > T || (key == T && eq_total == need_eq)) {
      const int slot = atomicAdd(&sm.cnt, 1);
      sm.cand_key[slot] = key;
      sm.cand_idx[slot] = i;
    }
  }
  __syncthreads();
  if (eq_total != need_eq) {
    // ties at the threshold: take the need_eq smallest indices, in index order
    int carry = 0;
    for (int base = 0; base < n_valid; base += kTopkThreads) {
      const int i = base + tid;
      const int is_eq = (i < n_valid && key_at(i) == T) ? 1 : 0;
      int tot;
      const int rank = carry + block_exclusive_scan(is_eq, sm.scan_lds, &tot);
      if (is_eq && rank < need_eq) {
        sm.cand_key[n_gt + rank] = T;
        sm.cand_idx[n_gt + rank] = i;
      }
      carry += tot;
      if (carry >= need_eq) break;  // uniform: carry is the same on every thread
    }
    __syncthreads();
  }

  // ---- order the winners: key descending, index ascending ------------------
  for (int c = tid; c < sel; c += kTopkThreads) {
    const uint32_t kc = sm.cand_key[c];
    const int ic = sm.cand_idx[c];
    int rank = 0;
    for (int j = 0; j < sel; ++j) {
      const uint32_t kj = sm.cand_key[j];
      rank += (kj > kc) || (kj == kc && sm.cand_idx[j] < ic);
    }
    out[rank] = key_finite(kc) ? ic : -1;
  }
}

}  // namespace skv
