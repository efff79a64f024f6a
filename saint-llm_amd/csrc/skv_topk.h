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

template <int kThreads>
struct TopkSmemT {
  int whist[kThreads / kWave][256];
  int hist[256];
  uint32_t cand_key[kMaxTopK];
  int cand_idx[kMaxTopK];
  int scan_lds[17];
  int digit, above, cnt;
};
using TopkSmem = TopkSmemT<kTopkThreads>;

// emit(j, v) for every output position j in [0, k), once each: the sel =
// min(k, n_cols, n_valid) best of row[0, n_valid) in (score desc, index asc)
// order, -1 for non-finite picks and ranks >= sel.  `keys` (kLdsKeys words
// of LDS) stages short rows; nullptr reads global memory on every pass.
// Every thread of the kThreads-thread workgroup (kThreads >= 256) must call
// it.
template <int kThreads, class Emit>
__device__ __forceinline__ void topk_row_emit(TopkSmemT<kThreads>& sm, uint32_t* keys, const float* row,
                                              int n_cols, int n_valid, int k, Emit emit) {
  static_assert(kThreads >= 256 && kThreads % kWave == 0, "topk_row needs >= 256 threads");
  constexpr int kWaves = kThreads / kWave;
  const int tid = threadIdx.x;
  const int wid = tid / kWave;
  n_cols = max(n_cols, 0);
  n_valid = max(0, min(n_valid, n_cols));
  const int k_eff = min(k, n_cols);
  const int sel = min(k_eff, n_valid);
  for (int j = sel + tid; j < k; j += kThreads) emit(j, -1);
  if (sel == 0) return;
  const bool in_lds = keys != nullptr && n_valid <= kLdsKeys;
  if (in_lds) {
    for (int i = tid; i < n_valid; i += kThreads) keys[i] = score_key(row[i]);
    __syncthreads();
  }
  auto key_at = [&](int i) -> uint32_t { return in_lds ? keys[i] : score_key(row[i]); };

  // ---- radix select: the sel-th largest key, 8 bits per pass ---------------
  uint32_t prefix = 0, pmask = 0;
  int remaining = sel;  // rank (1-based) of the target among keys matching prefix
  int eq_total = 0;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < kWaves * 256; i += kThreads) (&sm.whist[0][0])[i] = 0;
    __syncthreads();
    for (int i = tid; i < n_valid; i += kThreads) {
      const uint32_t key = key_at(i);
      if ((key & pmask) == prefix) atomicAdd(&sm.whist[wid][(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid < 256) {
      int s = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += sm.whist[w][tid];
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
  for (int i = tid; i < n_valid; i += kThreads) {
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
    for (int base = 0; base < n_valid; base += kThreads) {
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
  for (int c = tid; c < sel; c += kThreads) {
    const uint32_t kc = sm.cand_key[c];
    const int ic = sm.cand_idx[c];
    int rank = 0;
    for (int j = 0; j < sel; ++j) {
      const uint32_t kj = sm.cand_key[j];
      rank += (kj > kc) || (kj == kc && sm.cand_idx[j] < ic);
    }
    emit(rank, key_finite(kc) ? ic : -1);
  }
}

// out[0, k) as topk_row_emit gives it.
template <int kThreads = kTopkThreads>
__device__ __forceinline__ void topk_row(TopkSmemT<kThreads>& sm, uint32_t* keys, const float* row,
                                         int n_cols, int n_valid, int k, int32_t* out) {
  topk_row_emit<kThreads>(sm, keys, row, n_cols, n_valid, k, [&](int j, int v) { out[j] = v; });
}

// ===========================================================================
// Multi-workgroup selection in three launches (kernel boundaries order the
// phases; no workgroup waits for or fences against another):
//   hist   : every kTkChunk-score chunk of a row adds its 11-bit key histogram
//            (top bits of the order key) to the row's global histogram.
//   filter : every chunk finds the threshold bin t (the bin holding rank sel)
//            from the histogram and appends its keys in bins > t ("sure") and
//            == t ("ties") to the row's lists, one atomic per list per chunk.
//   final  : orders the winners by (key desc, index asc).  Every sure key
//            wins; in bin t only the first `need` = sel - n_sure survive.
//            Standalone select: one workgroup per row (topk_final_row), which
//            then zeroes the row's histogram and counters.  Decode step:
//            several workgroups per row each rank a share of the candidates
//            and gather their entries (the gather launch of skv_decode_step).
// A tie bin larger than kTkTieCap makes final fall back to the single-
// workgroup select over the row.
// ===========================================================================
constexpr int kTkChunk = 2048;
constexpr int kTkPartThreads = 256;  // hist / filter workgroups
constexpr int kTkBins = 2048;
constexpr int kTkShift = 21;
constexpr int kTkTieCap = 4096;
// per-row workspace layout, int32 words
constexpr int kTkWsHist = 0;
constexpr int kTkWsCnt = kTkBins;       // n_sure, n_tie, tie-overflow flag, (spare)
constexpr int kTkWsFlag = kTkWsCnt + 2;
constexpr int kTkWsSure = kTkWsCnt + 4; // (key, idx) pairs, kMaxTopK of them
constexpr int kTkWsTie = kTkWsSure + 2 * kMaxTopK;
// filter chunk c < kTkRunCap: (first slot, count) of its run in the sure
// list, then in the tie list, so that a reader can put the lists in entry
// order without sorting them
constexpr int kTkRunCap = 64;
constexpr int kTkWsRuns = kTkWsTie + 2 * kTkTieCap;
constexpr int kTkWsWords = kTkWsRuns + 4 * kTkRunCap;
static_assert(kTkWsRuns % 4 == 0 && kTkWsWords % 4 == 0, "16-byte run entries in 16-byte aligned rows");

__device__ __forceinline__ int topk_sel(int k, int n_cols, int n_valid) {
  n_cols = max(n_cols, 0);
  n_valid = max(0, min(n_valid, n_cols));
  return min(min(k, n_cols), n_valid);
}

struct TopkHistSmem {
  int hist[kTkBins];
};

// row holds at least `width` (>= 1) readable scores; cols(n_cols, n_valid)
// gives the row's extent.  The score loads (indices clamped into the row,
// all in flight together) are issued before cols is called, so that a
// caller's loads of the extent overlap them.
template <class Cols>
__device__ __forceinline__ void topk_hist_chunk_at(TopkHistSmem& sm, const float* row, int width, Cols cols,
                                                   int k, int chunk, int32_t* ws) {
  const int tid = threadIdx.x;
  const int i0 = chunk * kTkChunk;
  constexpr int kPer = kTkChunk / kTkPartThreads;
  float f[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) f[q] = row[min(i0 + q * kTkPartThreads + tid, width - 1)];
  int n_cols, n_valid;
  cols(n_cols, n_valid);
  if (topk_sel(k, n_cols, n_valid) == 0) return;  // uniform
  n_valid = max(0, min(n_valid, n_cols));
  const int i1 = min(n_valid, i0 + kTkChunk);
  if (i0 >= i1) return;
  for (int b = tid; b < kTkBins; b += kTkPartThreads) sm.hist[b] = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (i0 + q * kTkPartThreads + tid < i1) atomicAdd(&sm.hist[score_key(f[q]) >> kTkShift], 1);
  }
  __syncthreads();
  for (int b = tid; b < kTkBins; b += kTkPartThreads) {
    if (sm.hist[b]) atomicAdd(&ws[kTkWsHist + b], sm.hist[b]);
  }
}

__device__ __forceinline__ void topk_hist_chunk(TopkHistSmem& sm, const float* row, int n_cols,
                                                int n_valid, int k, int chunk, int32_t* ws) {
  if (topk_sel(k, n_cols, n_valid) == 0) return;  // uniform; otherwise at least one valid score
  topk_hist_chunk_at(
      sm, row, max(0, min(n_valid, n_cols)),
      [&](int& c, int& v) {
        c = n_cols;
        v = n_valid;
      },
      k, chunk, ws);
}

// Threshold bin of rank sel from the row histogram (every thread gets it).
// hist[] is the histogram staged in LDS; nthreads * per == kTkBins.
// total (optional): the histogram's sum; when it is below sel no bin holds
// rank sel and t / above / ties are undefined.
template <int kThreads>
__device__ __forceinline__ void topk_threshold(const int* hist, int sel, int* scan_lds, int* sh,
                                               int& t, int& above, int& ties, int* total = nullptr) {
  constexpr int per = kTkBins / kThreads;
  const int tid = threadIdx.x;
  const int hi = kTkBins - 1 - tid * per;  // this thread's bins: hi, hi-1, ..., hi-per+1
  int v[per];
  int sum = 0;
#pragma unroll
  for (int q = 0; q < per; ++q) {
    v[q] = hist[hi - q];
    sum += v[q];
  }
  int tot;
  int ex = block_exclusive_scan(sum, scan_lds, &tot);  // keys in bins > hi
  if (total) *total = tot;
#pragma unroll
  for (int q = 0; q < per; ++q) {
    if (ex < sel && sel <= ex + v[q]) {
      sh[0] = hi - q;
      sh[1] = ex;
      sh[2] = v[q];
    }
    ex += v[q];
  }
  __syncthreads();
  t = sh[0];
  above = sh[1];
  ties = sh[2];
  __syncthreads();
}

// Stages the kTkBins-word row histogram in LDS (16-byte aligned): each of
// kTkBins/8 threads (a 256-thread workgroup) fetches two 16-byte pieces and
// later puts them, so that other loads can be issued in between.
constexpr int kTkHistHalf = kTkBins / 8;
static_assert(kTkHistHalf == kTkPartThreads, "one thread per hist piece pair");
__device__ __forceinline__ void hist_fetch(int4& a, int4& b, const int32_t* g) {
  a = reinterpret_cast<const int4*>(g)[threadIdx.x];
  b = reinterpret_cast<const int4*>(g)[threadIdx.x + kTkHistHalf];
}
__device__ __forceinline__ void hist_put(int* lds, const int4& a, const int4& b) {
  reinterpret_cast<int4*>(lds)[threadIdx.x] = a;
  reinterpret_cast<int4*>(lds)[threadIdx.x + kTkHistHalf] = b;
}

struct TopkFilterSmem {
  alignas(16) int hist[kTkBins];
  int scan_lds[17];
  int sh[3];
  int wcnt[2][kTkPartThreads / kWave];  // per-wave candidate counts of this chunk
  int base[2];                          // this chunk's first slots in the row's lists
};

// The chunk's keys stay in registers: a first ballot pass counts each wave's
// sure and tie candidates, one global atomic per list reserves the chunk's
// slots (recorded in the row's run table), and a second ballot pass writes
// every candidate to its slot (waves in order, lanes in order, so each list
// is index-sorted within a chunk).  The
// scores are loaded before the histogram is read, so the two memory
// latencies overlap.  A tie bin above kTkTieCap is flagged in ws[kTkWsFlag]
// by chunk 0 and no list is written.
// row / width / cols as for topk_hist_chunk_at: the score and histogram
// loads are issued before the row's extent is known.
template <class Cols>
__device__ __forceinline__ void topk_filter_chunk_at(TopkFilterSmem& sm, const float* row, int width, Cols cols,
                                                     int k, int chunk, int32_t* ws) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  constexpr int kWaves = kTkPartThreads / kWave;
  constexpr int kRun = kTkChunk / kWaves;  // each wave owns a contiguous run of scores
  constexpr int kPer = kRun / kWave;
  const int i0 = chunk * kTkChunk;
  const int r0 = i0 + wid * kRun;
  // unconditional loads (index clamped into the row) so that all of them
  // are in flight together; lanes past the chunk drop the value
  float f[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) f[q] = row[min(r0 + q * kWave + lane, width - 1)];
  int4 ha, hb;
  hist_fetch(ha, hb, ws + kTkWsHist);
  int n_cols, n_valid;
  cols(n_cols, n_valid);
  hist_put(sm.hist, ha, hb);
  const int sel = topk_sel(k, n_cols, n_valid);
  if (sel == 0) return;  // uniform
  n_valid = max(0, min(n_valid, n_cols));
  const int i1 = min(n_valid, i0 + kTkChunk);
  if (i0 >= i1) return;
  uint32_t keys[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) keys[q] = (r0 + q * kWave + lane < i1) ? score_key(f[q]) : 0u;
  __syncthreads();
  int t, above, ties;
  topk_threshold<kTkPartThreads>(sm.hist, sel, sm.scan_lds, sm.sh, t, above, ties);
  if (ties > kTkTieCap) {  // the final step falls back to a full single-workgroup select
    if (chunk == 0 && tid == 0) ws[kTkWsFlag] = 1;
    return;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int ns = 0, nt = 0;  // wave-uniform counts
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const bool valid = r0 + q * kWave + lane < i1;
    const int b = static_cast<int>(keys[q] >> kTkShift);
    ns += __popcll(__ballot(valid && b > t));
    nt += __popcll(__ballot(valid && b == t));
  }
  if (lane == 0) {
    sm.wcnt[0][wid] = ns;
    sm.wcnt[1][wid] = nt;
  }
  __syncthreads();
  if (tid < 2) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += sm.wcnt[tid][w];
    const int base = tot ? atomicAdd(&ws[kTkWsCnt + tid], tot) : 0;
    sm.base[tid] = base;
    if (chunk < kTkRunCap) {
      ws[kTkWsRuns + 4 * chunk + 2 * tid] = base;
      ws[kTkWsRuns + 4 * chunk + 2 * tid + 1] = tot;
    }
  }
  __syncthreads();
  int ps = sm.base[0], pt = sm.base[1];
  for (int w = 0; w < wid; ++w) {
    ps += sm.wcnt[0][w];
    pt += sm.wcnt[1][w];
  }
  int2* sure_list = reinterpret_cast<int2*>(ws + kTkWsSure);
  int2* tie_list = reinterpret_cast<int2*>(ws + kTkWsTie);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int i = r0 + q * kWave + lane;
    const bool valid = i < i1;
    const int b = static_cast<int>(keys[q] >> kTkShift);
    const bool sure = valid && b > t;
    const bool tie = valid && b == t;
    const uint64_t ms = __ballot(sure);
    const uint64_t mt = __ballot(tie);
    if (sure) sure_list[ps + __popcll(ms & below)] = make_int2(static_cast<int32_t>(keys[q]), i);
    if (tie) tie_list[pt + __popcll(mt & below)] = make_int2(static_cast<int32_t>(keys[q]), i);
    ps += __popcll(ms);
    pt += __popcll(mt);
  }
}

__device__ __forceinline__ void topk_filter_chunk(TopkFilterSmem& sm, const float* row, int n_cols,
                                                  int n_valid, int k, int chunk, int32_t* ws) {
  if (topk_sel(k, n_cols, n_valid) == 0) return;  // uniform; otherwise at least one valid score
  topk_filter_chunk_at(
      sm, row, max(0, min(n_valid, n_cols)),
      [&](int& c, int& v) {
        c = n_cols;
        v = n_valid;
      },
      k, chunk, ws);
}

constexpr int kTkBuckets = 4096;  // final ordering: buckets of the top 15 key bits
constexpr int kTkCand = kMaxTopK + kTkTieCap;

struct TopkFinalSmem {
  int scan_lds[17];
  int sh[3];
  union {
    TopkSmem full;  // single-workgroup fallback (global-memory passes)
    struct {
      alignas(16) int hist[kTkBins];
      int cursor[kTkBuckets];  // counts, then running cursors (bucket ends after the scatter)
      int start[kTkBuckets];   // first slot of each bucket (descending key order)
      uint32_t key[kTkCand];   // candidates as read from the lists
      int idx[kTkCand];
      uint32_t skey[kTkCand];  // candidates in bucket order
      int sidx[kTkCand];
    } fin;
  } u;
};

__device__ __forceinline__ void topk_clear_ws(int32_t* ws) {
  for (int b = threadIdx.x; b < kTkBins; b += kTopkThreads) ws[kTkWsHist + b] = 0;
  if (threadIdx.x < 4) ws[kTkWsCnt + threadIdx.x] = 0;
}

// One 1024-thread workgroup per row.  The candidates (every key in bins > t
// and every tie in bin t) are counting-sorted by bucket = (key >> 17) - (t << 4)
// (clamped to the last bucket: a monotone map of the key), ranked by
// (key desc, index asc) inside their bucket, and the first sel are written.
__device__ __forceinline__ void topk_final_row(TopkFinalSmem& sm, const float* row, int n_cols,
                                               int n_valid, int k, int32_t* ws, int32_t* out) {
  const int tid = threadIdx.x;
  const int sel = topk_sel(k, n_cols, n_valid);
  n_valid = max(0, min(n_valid, max(n_cols, 0)));
  for (int j = sel + tid; j < k; j += kTopkThreads) out[j] = -1;
  if (sel == 0) {
    topk_clear_ws(ws);
    return;
  }
  auto& F = sm.u.fin;
  if (tid < kTkHistHalf) {
    int4 ha, hb;
    hist_fetch(ha, hb, ws + kTkWsHist);
    hist_put(F.hist, ha, hb);
  }
  for (int b = tid; b < kTkBuckets; b += kTopkThreads) F.cursor[b] = 0;
  __syncthreads();
  int t, above, ties;
  topk_threshold<kTopkThreads>(F.hist, sel, sm.scan_lds, sm.sh, t, above, ties);
  if (ties > kTkTieCap) {
    topk_row(sm.u.full, nullptr, row, n_cols, n_valid, k, out);
    __syncthreads();
    topk_clear_ws(ws);
    return;
  }
  const uint32_t base = static_cast<uint32_t>(t) << 4;
  auto bucket_of = [&](uint32_t key) -> int {
    return static_cast<int>(min((key >> 17) - base, static_cast<uint32_t>(kTkBuckets - 1)));
  };
  const int total = above + ties;
  constexpr int kLoad = (kTkCand + kTopkThreads - 1) / kTopkThreads;  // every list load in flight at once
  {
    int2 v[kLoad];
#pragma unroll
    for (int u = 0; u < kLoad; ++u) {
      const int c = min(tid + u * kTopkThreads, total - 1);  // total >= sel > 0
      v[u] = reinterpret_cast<const int2*>(ws + (c < above ? kTkWsSure : kTkWsTie))[c < above ? c : c - above];
    }
#pragma unroll
    for (int u = 0; u < kLoad; ++u) {
      const int c = tid + u * kTopkThreads;
      if (c < total) {
        const uint32_t key = static_cast<uint32_t>(v[u].x);
        F.key[c] = key;
        F.idx[c] = v[u].y;
        atomicAdd(&F.cursor[bucket_of(key)], 1);
      }
    }
  }
  __syncthreads();
  {
    constexpr int per = kTkBuckets / kTopkThreads;  // buckets per thread, descending
    const int hi = kTkBuckets - 1 - tid * per;
    int v[per];
    int sum = 0;
#pragma unroll
    for (int q = 0; q < per; ++q) {
      v[q] = F.cursor[hi - q];
      sum += v[q];
    }
    int tot;
    int ex = block_exclusive_scan(sum, sm.scan_lds, &tot);  // candidates in higher buckets
#pragma unroll
    for (int q = 0; q < per; ++q) {
      F.start[hi - q] = ex;
      F.cursor[hi - q] = ex;
      ex += v[q];
    }
  }
  __syncthreads();
  for (int c = tid; c < total; c += kTopkThreads) {
    const uint32_t key = F.key[c];
    const int slot = atomicAdd(&F.cursor[bucket_of(key)], 1);
    F.skey[slot] = key;
    F.sidx[slot] = F.idx[c];
  }
  __syncthreads();
  for (int c = tid; c < total; c += kTopkThreads) {
    const uint32_t kc = F.skey[c];
    const int ic = F.sidx[c];
    const int bkt = bucket_of(kc);
    const int s0 = F.start[bkt];
    if (s0 >= sel) continue;  // the whole bucket ranks past the winners
    const int s1 = F.cursor[bkt];
    int rank = 0;
    for (int j = s0; j < s1; ++j) {
      const uint32_t kj = F.skey[j];
      rank += (kj > kc) || (kj == kc && F.sidx[j] < ic);
    }
    if (s0 + rank < sel) out[s0 + rank] = key_finite(kc) ? ic : -1;
  }
  __syncthreads();
  topk_clear_ws(ws);
}

}  // namespace skv
