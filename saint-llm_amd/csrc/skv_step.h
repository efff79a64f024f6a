// Definitions shared by the decode step (skv_decode.hip) and the decode
// attention that runs as the step's last launch (skv_attention.hip): the
// step's kernel-argument map, the XCD placement of a launch's blocks and the
// ranking of a CSA row's top-k candidates.
#pragma once

#include "skv_topk.h"

namespace skv {

constexpr int kDecodeMaxBatch = 1024;
constexpr int kStepThreads = 256;  // every workgroup of the decode step
constexpr int kGatherRowsD = 32;   // output rows per dense gather tile
// Longest sequence the step accepts (longer ones are refused with
// SKV_STATUS_BADARG): lengths, entry counts, page indices and grid indices
// stay below 2^24, so the kernels divide with udiv24.
constexpr int kMaxTokLen = (1 << 24) - (1 << 16);
static_assert(kTkPartThreads == kStepThreads, "top-k chunk workgroups are step workgroups");

// Where each workgroup's layer is, passed by value with every launch: kernel
// arguments come with a workgroup's first scalar loads, so no workgroup
// walks the descriptor's layer list through dependent loads to find it.
struct StepMap {
  int32_t batch;
  int32_t lanes;  // xcd_lanes(batch), a power of two
  int32_t n_own;  // the append launch's (layer, sequence) blocks, before its filter chunks
  int32_t n_layers;
  int32_t n_csa;
  uint32_t hca_mask;                  // bit l: layer l is an HCA layer
  uint64_t csa;                       // layer of the i-th CSA layer in bits [4i, 4i + 4)
  int32_t tiles[SKV_MAX_LAYERS];      // dense gather tiles per sequence of each layer
  int32_t tile_end[SKV_MAX_LAYERS];   // dense workgroups of layers 0..l (tiles x batch, running sum)
  int8_t group[SKV_MAX_LAYERS];       // page group of an HCA/CSA layer, -1 for an SWA layer
  uint32_t group_first;               // bit l: layer l is the first layer of its page group
  int32_t n_groups;
  int32_t* tok_lens;                  // the descriptor's
  int32_t* status;
  int32_t* step_lens;
  int32_t* step_top;
  // the groups' (unused groups: null pointers, bt_stride, block_size, m and n_pages 1)
  int32_t* block_table[SKV_MAX_GROUPS];
  int32_t* n_entries[SKV_MAX_GROUPS];
  int32_t* free_stack[SKV_MAX_GROUPS];
  int32_t* free_top[SKV_MAX_GROUPS];
  int32_t bt_stride[SKV_MAX_GROUPS];
  int32_t block_size[SKV_MAX_GROUPS];
  int32_t m[SKV_MAX_GROUPS];
  int32_t n_pages[SKV_MAX_GROUPS];
  // of the i-th CSA layer
  int32_t* topk_ws[SKV_MAX_LAYERS];
  const float* scores[SKV_MAX_LAYERS];
  int32_t score_stride[SKV_MAX_LAYERS];
  int32_t top_k[SKV_MAX_LAYERS];
};
static_assert(SKV_MAX_LAYERS <= 16, "CSA layer indices are 4-bit fields");

// A page group's table and sizes, from the kernel arguments.
struct GroupRef {
  const int32_t* block_table;
  int bt_stride, block_size, n_pages, m;
};

__device__ __forceinline__ GroupRef group_ref(const StepMap& map, int g) {
  return GroupRef{map.block_table[g], map.bt_stride[g], map.block_size[g], map.n_pages[g], map.m[g]};
}

// Score columns of a CSA query at length L (entries L/m; the causal mask
// keeps (L-1)/m of them), clamped to the row's width so that no length can
// send a read past the row.
__device__ __forceinline__ void score_cols(int64_t score_stride, int m, int L, int& n_cols, int& n_valid) {
  const uint32_t Lc = static_cast<uint32_t>(min(max(L, 0), kMaxTokLen));
  n_cols = static_cast<int>(min<int64_t>(udiv24(Lc, m), score_stride));
  n_valid = Lc > 0 ? static_cast<int>(min<int64_t>(udiv24(Lc - 1, m), score_stride)) : 0;
}

// Blocks go to the XCDs in turn (block i to XCD i % X on a device of X
// XCDs, each with its own L2).  With `lanes` = X (a batch that is a multiple
// of X, so that every XCD gets the same work), a region of lanes *
// ceil(batch / lanes) * per_seq blocks that starts at a multiple of X gives
// the per_seq items of sequence b to blocks of XCD b % X, in every launch of
// the step: the scores, candidate lists and block-table row of b that one
// launch writes or reads, the next one finds in the same L2.  With lanes = 1
// (one XCD, or smaller or ragged batches) the items go sequence by sequence
// to consecutive blocks, spread over every XCD.  Item r of sequence b for
// block u of the region, or false for a block past the batch.
inline int xcd_lanes(int batch) {
  const int x = device_xcds();
  return (x > 1 && batch % x == 0) ? x : 1;
}

__host__ __device__ constexpr int64_t xcd_region(int batch, int64_t per_seq) {
  return static_cast<int64_t>(batch) * per_seq;  // lanes divide the batch
}

// lanes: xcd_lanes(batch) of the launch (a kernel argument, a power of two).
__device__ __forceinline__ bool xcd_item(uint32_t u, int per_seq, int batch, int lanes, int& b, int& r) {
  const int sh = __builtin_ctz(static_cast<uint32_t>(lanes));
  const uint32_t k = u >> sh;  // the block's turn on its XCD
  const uint32_t sb = udiv24(k, per_seq);
  b = static_cast<int>((u & (lanes - 1)) + (sb << sh));
  r = static_cast<int>(k - sb * per_seq);
  return b < batch;
}

// 64-bit order key of a candidate (key, index): larger means earlier in the
// top-k output (score descending, then index ascending).
__device__ __forceinline__ uint64_t order_key(int2 v) {
  return (static_cast<uint64_t>(static_cast<uint32_t>(v.x)) << 32) | static_cast<uint32_t>(~v.y);
}

constexpr int kRankR = 4;  // candidates a lane compares with each key it reads


// Lanes that share a group of kRankR candidates: the largest power of two
// in [1, 64] that still gives every group of the round its lanes.
template <int NT>
__device__ __forceinline__ int rank_lanes(int n_groups) {
  int sub_n = kWave;
  while (sub_n > 1 && sub_n * n_groups > NT) sub_n >>= 1;
  return sub_n;
}

// Sum of v over an aligned group of sub_n (a power of two <= 64) lanes, by
// DPP adds: quad exchanges, the half-row and row mirrors (every lane of a
// group of <= 16 then holds the sum), then row broadcasts of lanes 15 and 31
// (the group's last lane holds the sum of 32 or 64).  Every lane of the
// group must be active; no lane reads outside its group.
__device__ __forceinline__ int lane_group_sum(int v, int sub_n) {
  if (sub_n >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
  if (sub_n >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
  if (sub_n >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  if (sub_n >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false); // row_mirror
  if (sub_n >= 32) v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false); // row_bcast15 into rows 1, 3
  if (sub_n >= 64) v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false); // row_bcast31 into rows 2, 3
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave (lane i: the values of
// lanes 0..i): shifts by 1, 2, 4 and 8 within each row of 16 lanes, then each
// row's last lane added to the rows after it.  Every lane must be active.
__device__ __forceinline__ int wave_prefix_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast31 into rows 2, 3
  return v;
}

// Ranks a part's own candidates: cand(cls, j) is the list index (sure list
// [0, S), tie list [S, C)) of its j-th own candidate of class cls (0 sure,
// 1 tie), n_sure_mine and n_tie_mine of them.  The part's first n_pf
// candidates (its sure ones first, then its ties) get their output
// position, or -1 for a tie past the winners, in own_pos[j] instead of being
// collected; every other winner is handed to win(position, index) (index -1
// for a non-finite key), by one lane.  NT threads of the workgroup (threads
// 0..NT-1) take part.  KU: list keys a lane reads at once (1: a loop over its
// own keys, which needs the fewest registers).
// A candidate's position is its class's first position plus the keys of its
// class above it (every sure key is above every tie key).
template <int NT, int KU = 1, class KeyAt, class Win, class Cand>
__device__ __forceinline__ void rank_candidates_of(Win win, KeyAt ck, Cand cand, int n_sure_mine, int n_tie_mine,
                                                   int S, int C, int sel, int* own_pos = nullptr, int n_pf = 0) {
  const int tid = threadIdx.x;
  // the lane groups of both classes (sure candidates against the sure list,
  // ties against the tie list) run side by side
  const int ng_sure = (n_sure_mine + kRankR - 1) / kRankR;
  const int n_groups = ng_sure + (n_tie_mine + kRankR - 1) / kRankR;
  const int sub_n = rank_lanes<NT>(n_groups);  // uniform
  const int sub = tid & (sub_n - 1);
  for (int g0 = 0; g0 < n_groups; g0 += NT / sub_n) {
    const int g = g0 + tid / sub_n;  // this lane group's group
    if (g >= n_groups) break;        // uniform over the lane group
    const int cls = g >= ng_sure;
    const int lo = cls ? S : 0;
    const int hi = cls ? C : S;
    const int n_mine = cls ? n_tie_mine : n_sure_mine;
    const int j0 = (cls ? g - ng_sure : g) * kRankR;  // the group's first candidate
    // the group's candidates: their list indices first, clamped into the
    // group (n_mine >= 1 here), so that every read is issued before any is
    // waited for, then their keys; a candidate past the group never counts
    uint64_t mine[kRankR];
    int rank[kRankR];
    int ci[kRankR];
#pragma unroll
    for (int r = 0; r < kRankR; ++r) ci[r] = cand(cls, min(j0 + r, n_mine - 1));
#pragma unroll
    for (int r = 0; r < kRankR; ++r) {
      mine[r] = ck(ci[r]);
      rank[r] = 0;
    }
#pragma unroll
    for (int r = 0; r < kRankR; ++r) mine[r] = (j0 + r < n_mine) ? mine[r] : ~0ull;
    if constexpr (KU == 1) {
#pragma unroll 4
      for (int q = lo + sub; q < hi; q += sub_n) {
        const uint64_t key = ck(q);
#pragma unroll
        for (int r = 0; r < kRankR; ++r) rank[r] += key > mine[r];
      }
    } else {
      // KU key reads in flight per lane: the trip count is the lane group's
      // (a lane's own count makes the loop divergent, and each read is then
      // waited for before the next is issued).  Whole chunks of KU * sub_n
      // keys first, every read inside the list and every compare counted (a
      // per-key mask would put a scalar AND between each compare and its
      // add); then the chunk the list ends in, its reads clamped to the
      // list's last key and not counted past the end
      // the next chunk's keys are read before this chunk's are compared
      const auto count = [&](const uint64_t(&key)[KU]) {
#pragma unroll
        for (int u = 0; u < KU; ++u) {
#pragma unroll
          for (int r = 0; r < kRankR; ++r) rank[r] += key[u] > mine[r];
        }
      };
      int q0 = lo;
      if (q0 + KU * sub_n <= hi) {
        uint64_t key[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u) key[u] = ck(q0 + sub + u * sub_n);
        for (q0 += KU * sub_n; q0 + KU * sub_n <= hi; q0 += KU * sub_n) {
          uint64_t nxt[KU];
#pragma unroll
          for (int u = 0; u < KU; ++u) nxt[u] = ck(q0 + sub + u * sub_n);
          count(key);
#pragma unroll
          for (int u = 0; u < KU; ++u) key[u] = nxt[u];
        }
        count(key);
      }
      if (q0 < hi) {  // uniform over the lane group
        uint64_t key[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u) key[u] = ck(min(q0 + sub + u * sub_n, hi - 1));
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const bool in = q0 + sub + u * sub_n < hi;
#pragma unroll
          for (int r = 0; r < kRankR; ++r) rank[r] += in && key[u] > mine[r];
        }
      }
    }
    // sum over the lane group, two counts (< 2^16: a list holds at most
    // kTkTieCap keys) per word
    static_assert(kRankR == 4 && kTkTieCap < (1 << 16), "packed counts");
    const int p01 = lane_group_sum(rank[0] | (rank[1] << 16), sub_n);
    const int p23 = lane_group_sum(rank[2] | (rank[3] << 16), sub_n);
    rank[0] = p01 & 0xffff;
    rank[1] = p01 >> 16;
    rank[2] = p23 & 0xffff;
    rank[3] = p23 >> 16;
    if (sub == sub_n - 1) {  // the lane that holds the group's sums
#pragma unroll
      for (int r = 0; r < kRankR; ++r) {
        const int j = j0 + r;
        if (j >= n_mine) break;
        const int pos = lo + rank[r];
        const int own = (cls ? n_sure_mine : 0) + j;
        if (own < n_pf) {
          own_pos[own] = (pos < sel) ? pos : -1;
        } else if (pos < sel) {
          const uint32_t key = static_cast<uint32_t>(mine[r] >> 32);
          const int idx = static_cast<int>(~static_cast<uint32_t>(mine[r]));
          win(pos, key_finite(key) ? idx : -1);
        }
      }
    }
  }
}

// rank_candidates_of with the part's own candidates at list positions part,
// part + parts, ... of each class.
template <int NT, int KU = 1, class KeyAt, class Win>
__device__ __forceinline__ void rank_candidates(Win win, KeyAt ck, int S, int C, int sel, int part, int parts,
                                                int* own_pos = nullptr, int n_pf = 0) {
  const int n_sure_mine = (part < S) ? static_cast<int>(ceil_div24(S - part, parts)) : 0;
  const int n_tie_mine = (part < C - S) ? static_cast<int>(ceil_div24(C - S - part, parts)) : 0;
  rank_candidates_of<NT, KU>(
      win, ck, [&](int cls, int j) { return (cls ? S : 0) + part + j * parts; }, n_sure_mine, n_tie_mine, S, C, sel,
      own_pos, n_pf);
}

// The attention launches that end skv_decode_step_attend, after the step's
// hist and append launches (skv_attention.hip).  With map == nullptr nothing
// is launched: it checks the descriptors (and, with `call`, the caller's
// pointers and workspace) and reports the workspace bytes in *ws_need.
int decode_attend(const skv_attention_desc* d, const skv_decode_desc* h, const StepMap* map, void* workspace,
                  int64_t ws_bytes, hipStream_t s, int64_t* ws_need, bool call);

}  // namespace skv
