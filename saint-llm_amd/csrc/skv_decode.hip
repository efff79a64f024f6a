// Fused decode step over a stack of heterogeneous layers in three launches,
//   hist   : top-k histogram chunks of the CSA layers' score rows
//   append : step page plan (computed by every workgroup) + SWA ring rows +
//            pooling fold / entry emission, beside the top-k filter chunks
//            (candidate lists); the top-k of a step reads no output of its
//            append, so it runs ahead of it
//   gather : per (CSA layer, sequence, part) ordering of the candidates and
//            the sparse gather of the winners' entries, interleaved with the
//            dense HCA / window copies and the commit of the step's lengths
// Every kernel boundary orders a producer before its consumers; no workgroup
// waits for or fences against another.
//
// Reference: one cached decode call of SaintLLM.forward walks the blocks and
// hands each attention its cache layer (model.py:294-315); the per-layer cache
// work is SWAKVCacheLayer/HCAKVCacheLayer/CSAKVCacheLayer.append
// (kv_cache.py:63-83, 138-202, 266-322), the CSA indexer top-k
// (csa.py:377-422), the sparse gather (csa.py:326-331), the HCA dense read
// (hca.py:126-141) and the SWA window (swa.py:115-125).
#include "skv_pool_state.h"
#include "skv_step.h"
#include "skv_indexer_tile.h"

namespace skv {

__device__ __forceinline__ const skv_decode_layer* csa_layer(const skv_decode_desc* d, const StepMap& map,
                                                             int want) {
  if (want < 0 || want >= map.n_csa) return nullptr;
  return &d->layers[(map.csa >> (4 * want)) & 15];
}

__device__ __forceinline__ void score_cols(const skv_decode_layer& Ly, int m, int L, int& n_cols, int& n_valid) {
  score_cols(Ly.score_stride, m, L, n_cols, n_valid);
}

// Top-k chunk u of a launch's region: (chunk, sequence, CSA layer); ok is
// false for a block past the batch.
struct TopkChunk {
  int chunk, b, z;
  bool ok;
};

__device__ __forceinline__ TopkChunk topk_chunk(uint32_t u, int n_chunks, const StepMap& map) {
  TopkChunk c;
  int r;
  c.ok = xcd_item(u, n_chunks * map.n_csa, map.batch, map.lanes, c.b, r);
  c.z = static_cast<int>(udiv24(r, n_chunks));
  c.chunk = r - c.z * n_chunks;
  return c;
}

// ---------------------------------------------------------------------------
// 1. step plan.  skv_reserve policy over the page groups: a sequence whose
//    entry count (L+1)/m needs more pages takes them from the group's free
//    stack, pops in ascending sequence order; all-or-nothing over every
//    group and sequence.  Every workgroup of the append launch computes it
//    from the same inputs with the same arithmetic, so each knows the
//    outcome and its own sequence's pops without waiting for another.
// ---------------------------------------------------------------------------
struct PlanSmem {
  int bad;
  int tot[SKV_MAX_GROUPS];  // pages the step pops from each group
  int pre[SKV_MAX_GROUPS];  // of which for the sequences before this workgroup's
};

struct OwnPlan {
  int bad;   // SKV_STATUS_* bits, 0 when the step goes ahead
  int len;   // tokens of sequence b before the step
  int top;   // free-stack top of group g_own before the step
  int off;   // pops of the sequences before b in group g_own
  int p0;    // pages sequence b held before the step
  int need;  // pages sequence b takes
};

// g_own < 0: no group (SWA layer).  write_tops: this workgroup also writes
// the groups' tops after the step to step_top.  early(len) is called with
// sequence b's token count once the plan's loads are in flight, so that the
// caller's loads that depend on it overlap the plan's reductions.
template <class Early>
__device__ __forceinline__ OwnPlan step_plan(PlanSmem& sm, const StepMap& map, int b, int g_own,
                                             bool write_tops, Early early) {
  constexpr int kPerT = kDecodeMaxBatch / kStepThreads;
  const int tid = threadIdx.x;
  const int batch = map.batch;
  const int ng = map.n_groups;
  OwnPlan P{0, map.tok_lens[b], 0, 0, 0, 0};
  if (ng == 0) return P;  // uniform: no page group, nothing to plan
  // every load first (clamped indices), so they are all in flight together;
  // the bounds (batch slices, groups) are uniform, so a small batch or a
  // single group issues one load of each kind, not kPerT * SKV_MAX_GROUPS
  int len1[kPerT] = {};
  int cur[kPerT][SKV_MAX_GROUPS] = {};
#pragma unroll
  for (int j = 0; j < kPerT; ++j) {
    if (j * kStepThreads >= batch) break;
    const int s = min(tid + j * kStepThreads, batch - 1);
    len1[j] = map.tok_lens[s] + 1;
#pragma unroll
    for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
      if (g >= ng) break;
      cur[j][g] = map.n_entries[g][s];
    }
  }
  int top[SKV_MAX_GROUPS] = {};
#pragma unroll
  for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
    if (g >= ng) break;
    top[g] = *map.free_top[g];
  }
  const int own_cur = map.n_entries[min(max(g_own, 0), ng - 1)][b];
  early(P.len);
  if (tid == 0) {
    sm.bad = 0;
#pragma unroll
    for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
      sm.tot[g] = 0;
      sm.pre[g] = 0;
    }
  }
  __syncthreads();
  // only sequences that take pages (or are refused) touch the LDS counters
  int bad = 0;
#pragma unroll
  for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
    if (g >= ng) continue;
    const uint32_t m = static_cast<uint32_t>(map.m[g]);
    const uint32_t bs = static_cast<uint32_t>(map.block_size[g]);
#pragma unroll
    for (int j = 0; j < kPerT; ++j) {
      const int s = tid + j * kStepThreads;
      if (s >= batch) continue;
      if (len1[j] <= 0 || len1[j] > kMaxTokLen || cur[j][g] < 0 || cur[j][g] > kMaxTokLen) {
        bad |= SKV_STATUS_BADARG;
        continue;
      }
      const uint32_t target = udiv24(static_cast<uint32_t>(len1[j]), m);
      const uint32_t c = static_cast<uint32_t>(cur[j][g]);
      if (target < c) {
        bad |= SKV_STATUS_BADARG;
        continue;
      }
      const uint32_t p0 = ceil_div24(c, bs);
      const uint32_t p1 = ceil_div24(target, bs);
      if (p1 > static_cast<uint32_t>(map.bt_stride[g])) bad |= SKV_STATUS_MAX_PAGES;
      const int need = static_cast<int>(p1 - p0);
      if (need) {
        atomicAdd(&sm.tot[g], need);
        if (s < b) atomicAdd(&sm.pre[g], need);
      }
    }
  }
  if (bad) atomicOr(&sm.bad, bad);
  __syncthreads();
  bad = sm.bad;
  int tot[SKV_MAX_GROUPS], pre[SKV_MAX_GROUPS];
#pragma unroll
  for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
    tot[g] = sm.tot[g];
    pre[g] = sm.pre[g];
  }
  __syncthreads();  // the counters share the caller's LDS union
#pragma unroll
  for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
    if (g >= ng) continue;
    if (top[g] < 0 || top[g] > map.n_pages[g]) bad |= SKV_STATUS_BADARG;
    else if (tot[g] > top[g]) bad |= SKV_STATUS_NOSPC;
  }
  P.bad = bad;
  if (bad) return P;
  if (write_tops && tid == 0) {
#pragma unroll
    for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
      if (g < ng) map.step_top[g] = top[g] - tot[g];
    }
  }
#pragma unroll
  for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
    if (g == g_own) {
      const uint32_t c0 = static_cast<uint32_t>(own_cur);
      const uint32_t target = udiv24(static_cast<uint32_t>(P.len + 1), map.m[g]);
      P.top = top[g];
      P.off = pre[g];
      P.p0 = static_cast<int>(ceil_div24(c0, map.block_size[g]));
      P.need = static_cast<int>(ceil_div24(target, map.block_size[g])) - P.p0;
    }
  }
  return P;
}

// ---------------------------------------------------------------------------
// 2. append launch, 256-thread workgroups:
//    blocks [0, batch*layers)        : (sequence, layer) appends — waves 0-1
//                                      fold the main stream, wave 2 the
//                                      indexer stream, wave 3 copies the ring
//                                      row;
//    then                            : top-k filter chunks (after the hist
//                                      launch).
// ---------------------------------------------------------------------------

// Raw inputs of one 8-channel group of a stream: running state (max, sum,
// acc) and the token's c and z.  They depend on the sequence only, so the
// append launch issues them before the step plan.
struct FoldIn {
  u32x4 m0, m1, s0, s1, a0, a1, cv, zv;
  u32x4 b0, b1;  // the bias row's 8 channels (token position p % m)
};

__device__ __forceinline__ void fold_bias(FoldIn& in, const float* bias, uint32_t pm, int channels, int grp) {
  const u32x4* bp = reinterpret_cast<const u32x4*>(bias + pm * channels + grp * 8);
  in.b0 = bp[0];
  in.b1 = bp[1];
}

__device__ __forceinline__ void fold_load(FoldIn& in, const float* state, const void* c_all, const void* z_all,
                                          int b, int channels, int grp) {
  const float* sbase = state + static_cast<int64_t>(b) * 3 * channels;
  const u32x4* sp = reinterpret_cast<const u32x4*>(sbase + grp * 8);
  const u32x4* ss = reinterpret_cast<const u32x4*>(sbase + channels + grp * 8);
  const u32x4* sa = reinterpret_cast<const u32x4*>(sbase + 2 * channels + grp * 8);
  in.m0 = sp[0];
  in.m1 = sp[1];
  in.s0 = ss[0];
  in.s1 = ss[1];
  in.a0 = sa[0];
  in.a1 = sa[1];
  in.cv = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(c_all) + static_cast<int64_t>(b) * channels + grp * 8);
  in.zv = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(z_all) + static_cast<int64_t>(b) * channels + grp * 8);
}

// Where an emitted entry goes: slot `in_page` of page `page` (checked against
// n_pages only when the entry is stored, so that the page's load overlaps
// the fold).
struct EmitSlot {
  uint8_t* pool;
  int64_t row_bytes;
  int32_t page;
  int32_t n_pages;
  int32_t block_size;
  int32_t in_page;
};

// Fold the token into the running state of channel groups t, t + nt (8
// channels each) of one stream and store the entry at `slot` if the token
// completes the block.  All threads t in [0, nt) of a stream must call it
// (fp8 amax shuffles span the 16 lanes of a 128-channel block, which
// nt = 128 keeps inside a wave).  `first` holds the inputs of group t.
__device__ __forceinline__ void decode_fold_part(int m, int b, int64_t p, const EmitSlot& slot, float* state,
                                                 const float* bias, const void* c_all, const void* z_all,
                                                 int channels, int format, int fp8_main, int t, int nt,
                                                 const FoldIn& first) {
  const int groups = channels >> 3;
  float* sbase = state + static_cast<int64_t>(b) * 3 * channels;
  const uint32_t pm = umod24(static_cast<uint32_t>(p), m);  // p < 2^24
  const bool fresh = pm == 0;
  const bool emit = pm + 1 == static_cast<uint32_t>(m);
  for (int grp0 = t; grp0 < ((groups + nt - 1) / nt) * nt; grp0 += nt) {
    const bool mine = grp0 < groups;
    const int grp = mine ? grp0 : groups - 1;  // in-range address for every lane
    FoldIn in = first;  // group t's inputs and bias row were loaded early
    if (grp0 != t) {
      fold_load(in, state, c_all, z_all, b, channels, grp);
      fold_bias(in, bias, pm, channels, grp);
    }
    const u32x4 b0 = in.b0, b1 = in.b1;
    float mx[8], sum[8], acc[8], c[8], z[8], bb[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mx[j] = fresh ? -INFINITY : __uint_as_float(in.m0[j]);
      mx[j + 4] = fresh ? -INFINITY : __uint_as_float(in.m1[j]);
      sum[j] = fresh ? 0.f : __uint_as_float(in.s0[j]);
      sum[j + 4] = fresh ? 0.f : __uint_as_float(in.s1[j]);
      acc[j] = fresh ? 0.f : __uint_as_float(in.a0[j]);
      acc[j + 4] = fresh ? 0.f : __uint_as_float(in.a1[j]);
      bb[j] = __uint_as_float(b0[j]);
      bb[j + 4] = __uint_as_float(b1[j]);
    }
    unpack8_bf16(in.cv, c);
    unpack8_bf16(in.zv, z);
    float out[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = z[j] + bb[j];
      if (v > mx[j]) {
        const float sc = expf(mx[j] - v);
        sum[j] = sum[j] * sc + 1.f;
        acc[j] = acc[j] * sc + c[j];
        mx[j] = v;
      } else {
        const float w = expf(v - mx[j]);
        sum[j] += w;
        acc[j] += w * c[j];
      }
      out[j] = mine ? acc[j] / sum[j] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; j += 2) bf16_round2(out[j], out[j + 1]);  // the compressor emits bf16 entries
    if (emit) {
      if (slot.page >= 0 && slot.page < slot.n_pages) {
        uint8_t* entry = slot.pool + (static_cast<int64_t>(slot.page) * slot.block_size + slot.in_page) * slot.row_bytes;
        store_entry_group(entry, out, grp0, groups, format, fp8_main);
      }
    } else if (mine) {
      u32x4* wp = reinterpret_cast<u32x4*>(sbase + grp * 8);
      wp[0] = u32x4{__float_as_uint(mx[0]), __float_as_uint(mx[1]), __float_as_uint(mx[2]), __float_as_uint(mx[3])};
      wp[1] = u32x4{__float_as_uint(mx[4]), __float_as_uint(mx[5]), __float_as_uint(mx[6]), __float_as_uint(mx[7])};
      u32x4* ws = reinterpret_cast<u32x4*>(sbase + channels + grp * 8);
      ws[0] = u32x4{__float_as_uint(sum[0]), __float_as_uint(sum[1]), __float_as_uint(sum[2]), __float_as_uint(sum[3])};
      ws[1] = u32x4{__float_as_uint(sum[4]), __float_as_uint(sum[5]), __float_as_uint(sum[6]), __float_as_uint(sum[7])};
      u32x4* wa = reinterpret_cast<u32x4*>(sbase + 2 * channels + grp * 8);
      wa[0] = u32x4{__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]), __float_as_uint(acc[3])};
      wa[1] = u32x4{__float_as_uint(acc[4]), __float_as_uint(acc[5]), __float_as_uint(acc[6]), __float_as_uint(acc[7])};
    }
  }
}

// Score row extent of chunk c's sequence after the step (tokens + 1): the
// top-k of the step runs beside the append, which a refusal discards.
__device__ __forceinline__ void chunk_cols(const StepMap& map, const TopkChunk& c, int& n_cols, int& n_valid) {
  score_cols(map.score_stride[c.z], map.m[map.group[(map.csa >> (4 * c.z)) & 15]], map.tok_lens[c.b] + 1, n_cols,
             n_valid);
}

// Hist launch: top-k histogram chunks (the grid holds n_chunks x batch x CSA
// layers blocks).  Chunk 0 zeroes the row's list counters, which the previous
// step's gather launch read; the gather launch zeroes the histogram again,
// also after a refusal.
__global__ __launch_bounds__(kTkPartThreads) void k_decode_hist(int n_chunks, StepMap map) {
  __shared__ TopkHistSmem sm;
  const TopkChunk c = topk_chunk(blockIdx.x, n_chunks, map);
  if (!c.ok) return;
  int32_t* ws = map.topk_ws[c.z] + static_cast<int64_t>(c.b) * kTkWsWords;
  if (c.chunk == 0 && threadIdx.x < 3) ws[kTkWsCnt + threadIdx.x] = 0;
  const int width = map.score_stride[c.z];
  topk_hist_chunk_at(
      sm, map.scores[c.z] + static_cast<int64_t>(c.b) * width, width,
      [&](int& n_cols, int& n_valid) { chunk_cols(map, c, n_cols, n_valid); }, map.top_k[c.z], c.chunk, ws);
}

// Score launch (in place of the hist launch when the step computes its own
// scores): workgroup (tile, sequence, CSA layer) scores kIdxTile of the
// layer's indexer entries before the step (the n_valid visible to the new
// token: floor(L / m) of L tokens before it), writes them to the layer's
// score row and adds their 11-bit key histogram to the row's, exactly as
// the hist launch would from the written row.  Tile 0 zeroes the row's list
// counters.
struct ScoreMap {
  const uint8_t* q[SKV_MAX_LAYERS];     // of the i-th CSA layer: [batch, heads, c] bf16
  const float* w[SKV_MAX_LAYERS];       // [batch, heads]
  const uint8_t* pool[SKV_MAX_LAYERS];  // indexer stream pages
  int32_t heads[SKV_MAX_LAYERS];
  int32_t c;                            // indexer channels
};

__global__ __launch_bounds__(kIdxThreads, 2) void k_decode_score_hist(int n_tiles, StepMap map, ScoreMap sc) {
  __shared__ IndexerSmem sm;
  __shared__ TopkHistSmem hs;
  const TopkChunk c = topk_chunk(blockIdx.x, n_tiles, map);
  if (!c.ok) return;
  const int tid = threadIdx.x;
  int32_t* ws = map.topk_ws[c.z] + static_cast<int64_t>(c.b) * kTkWsWords;
  if (c.chunk == 0 && tid < 3) ws[kTkWsCnt + tid] = 0;
  const int li = static_cast<int>((map.csa >> (4 * c.z)) & 15);
  const GroupRef G = group_ref(map, map.group[li]);
  const int heads = sc.heads[c.z];
  const IndexerRow r{sc.q[c.z] + static_cast<int64_t>(c.b) * heads * sc.c * 2,
                     sc.w[c.z] + static_cast<int64_t>(c.b) * heads,
                     sc.pool[c.z],
                     G.block_table + static_cast<int64_t>(c.b) * G.bt_stride,
                     G.bt_stride,
                     G.block_size,
                     G.n_pages,
                     heads,
                     sc.c};
  for (int i = tid; i < kTkBins; i += kIdxThreads) hs.hist[i] = 0;  // ordered by the tile's barrier
  const int width = map.score_stride[c.z];
  float* row = const_cast<float*>(map.scores[c.z]) + static_cast<int64_t>(c.b) * width;
  bool hist = false;
  const bool live = indexer_tile(
      sm, r, c.chunk,
      [&] {
        int n_cols, n_valid;
        score_cols(width, G.m, map.tok_lens[c.b] + 1, n_cols, n_valid);
        hist = topk_sel(map.top_k[c.z], n_cols, n_valid) > 0;
        return max(0, min(n_valid, n_cols));
      },
      [&](int e, float v) {
        row[e] = v;
        if (hist) atomicAdd(&hs.hist[score_key(v) >> kTkShift], 1);
      });
  if (!live || !hist) return;  // uniform
  lds_barrier();  // the histogram is complete; the score stores stay in flight
  for (int i = tid; i < kTkBins; i += kIdxThreads) {
    if (hs.hist[i]) atomicAdd(&ws[kTkWsHist + i], hs.hist[i]);
  }
}

union AppendSmem {
  PlanSmem plan;
  TopkFilterSmem filter;
};

__global__ __launch_bounds__(kStepThreads) void k_decode_append(const skv_decode_desc* __restrict__ d,
                                                                int n_chunks, StepMap map) {
  __shared__ AppendSmem sm;
  const int n_append = map.n_own;
  const int tid = threadIdx.x;
  if (static_cast<int>(blockIdx.x) >= n_append) {
    // top-k filter chunk: candidate lists from the complete histogram
    const TopkChunk c = topk_chunk(blockIdx.x - n_append, n_chunks, map);
    if (!c.ok) return;
    const int width = map.score_stride[c.z];
    topk_filter_chunk_at(
        sm.filter, map.scores[c.z] + static_cast<int64_t>(c.b) * width, width,
        [&](int& n_cols, int& n_valid) { chunk_cols(map, c, n_cols, n_valid); }, map.top_k[c.z], c.chunk,
        map.topk_ws[c.z] + static_cast<int64_t>(c.b) * kTkWsWords);
    return;
  }
  int b, l;
  if (!xcd_item(blockIdx.x, map.n_layers, map.batch, map.lanes, b, l)) return;  // block 0 is (layer 0, sequence 0)
  const skv_decode_layer& Ly = d->layers[l];
  const bool paged = Ly.kind != SKV_LAYER_SWA;
  const int wave = tid / kWave;
  // the fold's state and token inputs go out before the plan's loads
  const bool main_stream = wave < 2;
  const bool idx_stream = wave == 2 && Ly.kind == SKV_LAYER_CSA && Ly.idx_pool;
  FoldIn first{};
  if (paged && (main_stream || idx_stream)) {
    const int channels = main_stream ? d->latent : d->c_indexer;
    const int t = main_stream ? tid : tid - 2 * kWave;
    fold_load(first, global_field(main_stream ? Ly.state : Ly.idx_state),
              global_field(main_stream ? Ly.c_new : Ly.ci_new), global_field(main_stream ? Ly.z_new : Ly.zi_new), b,
              channels, min(t, (channels >> 3) - 1));
  }
  const int g = map.group[l];  // < 0 for an SWA layer
  // with the token count: the bias rows of the fold and the block-table slot
  // of the entry this token completes (a page held before the step)
  int32_t held_page = -1;
  const auto early = [&](int len) {
    if (!paged) return;  // uniform
    const uint32_t p1 = static_cast<uint32_t>(min(max(len, 0), kMaxTokLen - 1)) + 1;
    const int mm = map.m[g];
    if (main_stream || idx_stream) {
      const int channels = main_stream ? d->latent : d->c_indexer;
      const int t = main_stream ? tid : tid - 2 * kWave;
      fold_bias(first, global_field(main_stream ? Ly.bias : Ly.idx_bias), umod24(p1 - 1, mm), channels,
                min(t, (channels >> 3) - 1));
    }
    const uint32_t e1 = udiv24(p1, mm);
    const int pi = static_cast<int>(udiv24(e1 > 0 ? e1 - 1 : 0, map.block_size[g]));
    held_page = map.block_table[g][static_cast<int64_t>(b) * map.bt_stride[g] + min(pi, map.bt_stride[g] - 1)];
  };
  const OwnPlan P = step_plan(sm.plan, map, b, g, blockIdx.x == 0, early);
  if (P.bad) {
    if (blockIdx.x == 0 && tid == 0) *map.status = P.bad;
    return;  // refused: nothing changes
  }
  if (blockIdx.x == 0 && tid == 0) *map.status = 0;
  const int L0 = P.len;
  const int64_t p = L0;  // position of the new token
  if (l == 0 && tid == 0) map.step_lens[b] = L0 + 1;
  if (wave == 3) {
    const int row_chunks = d->latent >> 3;  // 16-byte chunks of a bf16 row
    const u32x4* src = static_cast<const u32x4*>(global_field(Ly.kv_new)) + static_cast<int64_t>(b) * row_chunks;
    u32x4* dst = static_cast<u32x4*>(global_field(Ly.ring)) + (static_cast<int64_t>(b) * d->window + umod24(static_cast<uint32_t>(p), d->window)) * row_chunks;
    for (int c = tid - 3 * kWave; c < row_chunks; c += kWave) dst[c] = src[c];
    return;
  }
  if (!paged) return;
  const int m = map.m[g], bs = map.block_size[g];
  int32_t* const bt_row = map.block_table[g] + static_cast<int64_t>(b) * map.bt_stride[g];
  const int32_t* const stack = map.free_stack[g];
  // the group's first layer records the sequence's new pages in the table
  if (((map.group_first >> l) & 1) && tid < P.need) bt_row[P.p0 + tid] = stack[P.top - 1 - P.off - tid];
  // the page of the entry this token completes, if any (its load overlaps the fold)
  const uint32_t e1 = udiv24(static_cast<uint32_t>(p + 1), m);  // entries after the token
  const uint32_t e = e1 > 0 ? e1 - 1 : 0;
  const int pi = static_cast<int>(udiv24(e, bs));
  int32_t page = -1;
  if (e1 * m == static_cast<uint32_t>(p + 1)) {  // uniform
    if (pi < P.p0) page = held_page;
    else if (pi - P.p0 < P.need) page = stack[P.top - 1 - P.off - (pi - P.p0)];
  }
  const int in_page = static_cast<int>(e) - pi * bs;
  if (main_stream) {
    const int fp8_main = (Ly.format == SKV_FMT_FP8) ? d->latent - SKV_FP8_ROPE_DIMS : 0;
    const EmitSlot slot{static_cast<uint8_t*>(global_field(Ly.pool)), Ly.entry_bytes, page, map.n_pages[g], bs,
                        in_page};
    decode_fold_part(m, b, p, slot, global_field(Ly.state), global_field(Ly.bias), global_field(Ly.c_new),
                     global_field(Ly.z_new), d->latent, Ly.format, fp8_main,
                     tid, 2 * kWave, first);
  } else if (idx_stream) {
    const EmitSlot slot{static_cast<uint8_t*>(global_field(Ly.idx_pool)), static_cast<int64_t>(d->c_indexer) * 2,
                        page, map.n_pages[g], bs, in_page};
    decode_fold_part(m, b, p, slot, global_field(Ly.idx_state), global_field(Ly.idx_bias), global_field(Ly.ci_new),
                     global_field(Ly.zi_new), d->c_indexer,
                     SKV_FMT_BF16, 0, tid - 2 * kWave, kWave, first);
  }
}

// ---------------------------------------------------------------------------
// Row copies shared by the gather tiles and the sparse gather.  Row kinds:
// 0 skip, 1 copy a bf16 row, 2 dequantize an fp8 entry to bf16, 3 zero row.
// ---------------------------------------------------------------------------

// 16 fp8 e4m3fn codes times their block scale -> 16 bf16 (two 16-byte chunks).
__device__ __forceinline__ void dequant_codes(const u32x4 codes, float scale, u32x4& o0, u32x4& o1) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float f[4];
    e4m3fn_x4_to_f32(codes[q], f);
#pragma unroll
    for (int h = 0; h < 4; ++h) f[h] *= scale;
    const uint32_t lo = bf16_pack2(f[0], f[1]);
    const uint32_t hi = bf16_pack2(f[2], f[3]);
    if (q < 2) {
      o0[2 * q] = lo;
      o0[2 * q + 1] = hi;
    } else {
      o1[2 * (q - 2)] = lo;
      o1[2 * (q - 2) + 1] = hi;
    }
  }
}

struct RowRef {
  const uint8_t* src;
  uint8_t* dst;
  int kind;
};

// Stores of the gathered rows: nontemporal, or (kWB) plain stores that
// allocate in the caches and are written back later.  The host picks per
// launch from the bytes the step gathers.
template <bool kWB>
__device__ __forceinline__ void st_out(u32x4* p, u32x4 v) {
  if constexpr (kWB) {
    *p = v;
  } else {
    st_stream(p, v);
  }
}

// Copies rows [0, n) with all kStepThreads threads, kTPR threads per row
// (kStepThreads / kTPR rows at a time); row(r) gives row r's RowRef.  A
// thread copies chunks sub, sub + kTPR, ... of its row, issuing kU 16-byte
// loads before their stores.  The loads are unconditional (a lane with
// nothing to load reads 16 bytes at `safe`, any readable device address,
// and drops them): a load under a divergent branch is waited for before the
// branch joins, which would serialize the memory round trips.  `fp8` says
// whether any row may be of kind 2 (uniform over the workgroup); kWB picks
// the stores (st_out).
template <int kTPR, int kU, bool kWB, class RowFn>
__device__ __forceinline__ void copy_rows(int n, RowFn row, int latent, bool fp8, const void* safe) {
  constexpr int kRowsAtOnce = kStepThreads / kTPR;
  const u32x4* safe4 = static_cast<const u32x4*>(safe);
  const int sub = threadIdx.x % kTPR;
  const int bf_chunks = latent >> 3;  // 16-byte chunks of an output row
  const int fp8_main = latent - SKV_FP8_ROPE_DIMS;
  const int code_chunks = fp8_main >> 4;  // 16 codes -> 2 output chunks
  const int fp8_tasks = code_chunks + (SKV_FP8_ROPE_DIMS >> 3);
  for (int r0 = 0; r0 < n; r0 += kRowsAtOnce) {
    const int r = r0 + static_cast<int>(threadIdx.x) / kTPR;
    RowRef rf = row(min(r, n - 1));
    if (r >= n) rf.kind = 0;
    for (int c0 = sub; c0 < bf_chunks; c0 += kTPR * kU) {
      u32x4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int c = min(c0 + u * kTPR, bf_chunks - 1);
        v[u] = ld_stream(rf.kind == 1 ? reinterpret_cast<const u32x4*>(rf.src) + c : safe4);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int c = c0 + u * kTPR;
        if (c < bf_chunks && (rf.kind == 1 || rf.kind == 3)) {
          st_out<kWB>(reinterpret_cast<u32x4*>(rf.dst) + c, rf.kind == 1 ? v[u] : u32x4{0u, 0u, 0u, 0u});
        }
      }
    }
    if (!fp8) continue;
    // an fp8 row of 576 channels is 40 tasks: fewer chunks in flight than a
    // bf16 row needs (and fewer registers)
    constexpr int kUF = (40 + kTPR - 1) / kTPR < kU ? (40 + kTPR - 1) / kTPR : kU;
    for (int c0 = sub; c0 < fp8_tasks; c0 += kTPR * kUF) {
      u32x4 v[kUF];
      float scale[kUF];
#pragma unroll
      for (int u = 0; u < kUF; ++u) {
        const int c = min(c0 + u * kTPR, fp8_tasks - 1);
        const bool live = rf.kind == 2;
        const bool is_code = c < code_chunks;
        const uint8_t* src = is_code ? rf.src + c * 16
                                     : rf.src + fp8_main + (fp8_main >> 7) * 4 + (c - code_chunks) * 16;
        v[u] = *(live ? reinterpret_cast<const u32x4*>(src) : safe4);
        scale[u] = *(live && is_code ? reinterpret_cast<const float*>(rf.src + fp8_main + (c >> 3) * 4)
                                     : reinterpret_cast<const float*>(safe4));
      }
#pragma unroll
      for (int u = 0; u < kUF; ++u) {
        const int c = c0 + u * kTPR;
        if (c >= fp8_tasks || rf.kind != 2) continue;
        u32x4* o = reinterpret_cast<u32x4*>(rf.dst);
        if (c < code_chunks) {
          u32x4 o0, o1;
          dequant_codes(v[u], scale[u], o0, o1);
          st_out<kWB>(o + 2 * c, o0);
          st_out<kWB>(o + 2 * c + 1, o1);
        } else {
          st_out<kWB>(o + (fp8_main >> 3) + (c - code_chunks), v[u]);
        }
      }
    }
  }
}

// Source of compressed entry e of sequence b: the row kind (1 bf16, 2 fp8)
// and its address, or 0 when e is past n_ent or its page is not mapped.
// The first n_lds entries of the sequence's block-table row may be staged
// in LDS (bt_lds).
// The descriptor fields of a layer that the gather launch reads.  A
// workgroup loads them at its start and holds them (hold_fields) once its
// first round trip is in flight: scalar loads left at their first use would
// be issued after the status check, one more dependent round trip.
struct GatherLayer {
  const uint8_t* pool;
  int64_t entry_bytes;
  void* out_entries;
  int32_t* topk_idx;      // CSA
  const uint8_t* ring;    // dense tiles
  void* out_window;       // dense tiles
  int64_t out_rows;       // dense tiles (HCA)
  int32_t format;
  int32_t latent;
  int32_t window;
};

__device__ __forceinline__ GatherLayer gather_layer(const skv_decode_desc* d, const skv_decode_layer& Ly) {
  return GatherLayer{static_cast<const uint8_t*>(global_field(Ly.pool)), Ly.entry_bytes,
                     global_field(Ly.out_entries), global_field(Ly.topk_idx),
                     static_cast<const uint8_t*>(global_field(Ly.ring)), global_field(Ly.out_window), Ly.out_rows,
                     Ly.format, d->latent, d->window};
}

// The values must be loaded here (scalar registers): the compiler keeps the
// loads ahead of this point instead of sinking them to their uses.
__device__ __forceinline__ void hold_fields(const GatherLayer& g, bool dense) {
  if (dense) {
    asm volatile("" ::"s"(g.pool), "s"(g.entry_bytes), "s"(g.out_entries), "s"(g.ring), "s"(g.out_window),
                 "s"(g.out_rows), "s"(g.format), "s"(g.latent), "s"(g.window));
  } else {
    asm volatile("" ::"s"(g.pool), "s"(g.entry_bytes), "s"(g.out_entries), "s"(g.topk_idx), "s"(g.format),
                 "s"(g.latent));
  }
}

__device__ __forceinline__ int entry_source(const GroupRef& G, const GatherLayer& Ly, int b, int e,
                                            int n_ent, const uint8_t** src, const int32_t* bt_lds = nullptr,
                                            int n_lds = 0) {
  if (e < 0 || e >= n_ent) return 0;
  const int pi = static_cast<int>(udiv24(e, G.block_size));  // e < 2^24
  const int32_t page = (pi < n_lds) ? bt_lds[pi]
                       : (pi < G.bt_stride) ? G.block_table[static_cast<int64_t>(b) * G.bt_stride + pi] : -1;
  if (page < 0 || page >= G.n_pages) return 0;
  *src = Ly.pool + (static_cast<int64_t>(page) * G.block_size + (e - pi * G.block_size)) * Ly.entry_bytes;
  return (Ly.format == SKV_FMT_FP8) ? 2 : 1;
}

// One compressed-entry output row split over kTPR threads: thread `sub`
// takes tasks sub, sub + kTPR, ... (a bf16 layer: the row's 16-byte chunks;
// an fp8 layer: 16-code chunks, each giving two output chunks, then the
// rope chunks).  Kind 3 rows are written as zeros.  The loads of a share can
// be issued long before its stores (see the rank parts).
template <int kU>
struct EntryShare {
  u32x4 v[kU];
  float sc[kU];
};

template <int kTPR, int kU>
__device__ __forceinline__ int entry_tasks(int latent, bool fp8) {
  return fp8 ? ((latent - SKV_FP8_ROPE_DIMS) >> 4) + (SKV_FP8_ROPE_DIMS >> 3) : (latent >> 3);
}

template <int kTPR, int kU>
__device__ __forceinline__ void entry_share_load(EntryShare<kU>& sh, const uint8_t* src, int kind, int latent,
                                                 bool fp8, const u32x4* safe4) {
  const int sub = threadIdx.x % kTPR;
  const int n = entry_tasks<kTPR, kU>(latent, fp8);
  const int fp8_main = latent - SKV_FP8_ROPE_DIMS;
  const int code_chunks = fp8_main >> 4;
  const bool live = fp8 ? kind == 2 : kind == 1;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    // uniform: tasks past the row's (an fp8 row has 40 of 72) and the scales
    // of bf16 rows and rope chunks are not loaded; the store reads neither
    sh.v[u] = u32x4{0u, 0u, 0u, 0u};
    sh.sc[u] = 0.f;
    if (u * kTPR >= n) continue;
    const int c = min(sub + u * kTPR, n - 1);
    const bool is_code = fp8 && c < code_chunks;
    const uint8_t* p = !fp8 ? src + c * 16
                            : is_code ? src + c * 16 : src + fp8_main + (fp8_main >> 7) * 4 + (c - code_chunks) * 16;
    sh.v[u] = ld_stream(live ? reinterpret_cast<const u32x4*>(p) : safe4);
    if (fp8 && u * kTPR < code_chunks) {
      sh.sc[u] = *(live && is_code ? reinterpret_cast<const float*>(src + fp8_main + (c >> 3) * 4)
                                   : reinterpret_cast<const float*>(safe4));
    }
  }
}

template <int kTPR, int kU, bool kWB>
__device__ __forceinline__ void entry_share_store(const EntryShare<kU>& sh, uint8_t* dst, int kind, int latent,
                                                  bool fp8) {
  const int sub = threadIdx.x % kTPR;
  const int n = entry_tasks<kTPR, kU>(latent, fp8);
  const int fp8_main = latent - SKV_FP8_ROPE_DIMS;
  const int code_chunks = fp8_main >> 4;
  u32x4* o = reinterpret_cast<u32x4*>(dst);
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int c = sub + u * kTPR;
    if (c >= n || kind == 0) continue;
    if (!fp8) {
      st_out<kWB>(o + c, kind == 1 ? sh.v[u] : zero);
    } else if (c < code_chunks) {
      u32x4 o0 = zero, o1 = zero;
      if (kind == 2) dequant_codes(sh.v[u], sh.sc[u], o0, o1);
      st_out<kWB>(o + 2 * c, o0);
      st_out<kWB>(o + 2 * c + 1, o1);
    } else {
      st_out<kWB>(o + (fp8_main >> 3) + (c - code_chunks), kind == 2 ? sh.v[u] : zero);
    }
  }
}

// ---------------------------------------------------------------------------
// 3. dense gather tiles (HCA entries and SWA windows) and the commit of the
//    step: blocks of the gather launch.
//    Tile t of (layer, sequence) copies rows [32t, 32t+32) of the layer's
//    dense row space [HCA entries (out_rows) | window], kDenseTPR threads
//    per row.  Each thread loads its row's block-table entry together with
//    the length and the status (one round trip), then the row.  Tile 0 of
//    (layer 0, b) commits the step's length of b (tokens and entry counts),
//    tile 0 of (layer 0, 0) the free-stack tops; nothing in these launches
//    reads them.
// ---------------------------------------------------------------------------
constexpr int kDenseTPR = kStepThreads / kGatherRowsD;  // threads per dense row
constexpr int kDenseU = 9;  // 16-byte chunks per thread and pass: 8 x 9 x 16 B = a 576-channel bf16 row

// Dense tile u of the gather launch.
template <bool kWB>
__device__ __forceinline__ void dense_block(const skv_decode_desc* d, const StepMap& map, int u) {
  // the block's layer: the first l with u < tile_end[l] (kernel arguments only)
  int l = 0, base = 0, tiles = map.tiles[0];
#pragma unroll
  for (int i = 0; i + 1 < SKV_MAX_LAYERS; ++i) {
    if (u >= map.tile_end[i]) {
      l = i + 1;
      base = map.tile_end[i];
      tiles = map.tiles[i + 1];
    }
  }
  const int rem = u - base;
  const int b = static_cast<int>(udiv24(rem, tiles));
  const int tile = rem - b * tiles;
  const int g = ((map.hca_mask >> l) & 1) ? map.group[l] : -1;  // uniform; < 0: no HCA entries
  const int r = tile * kGatherRowsD + static_cast<int>(threadIdx.x) / kDenseTPR;  // this thread's row
  // one round trip: length, status and the row's block-table entry (clamped
  // into the sequence's row, so that the load needs no branch)
  const int gi = max(g, 0);
  const int bs = map.block_size[gi];
  const int pi = static_cast<int>(udiv24(r, bs));
  const int32_t* bt = (g >= 0) ? map.block_table[gi] + static_cast<int64_t>(b) * map.bt_stride[gi] +
                                     min(pi, map.bt_stride[gi] - 1)
                               : map.step_lens + b;
  const GatherLayer Ly = gather_layer(d, d->layers[l]);
  const int32_t page = *bt;
  const int L = map.step_lens[b];
  const int status = *map.status;
  hold_fields(Ly, true);
  if (status) return;  // refused step
  if (l == 0 && tile == 0 && threadIdx.x == 0) {
    map.tok_lens[b] = L;
    for (int gg = 0; gg < map.n_groups; ++gg) map.n_entries[gg][b] = udiv24(L, map.m[gg]);
    if (b == 0) {
      for (int gg = 0; gg < map.n_groups; ++gg) *map.free_top[gg] = map.step_top[gg];
    }
  }
  const int latent = Ly.latent;
  const int64_t out_row = static_cast<int64_t>(latent) * 2;
  // row space of the layer's tile: HCA entries if they are copied, then the
  // window if it is copied
  const int n_dense = (g >= 0 && Ly.out_entries) ? static_cast<int>(Ly.out_rows) : 0;
  RowRef rf{nullptr, nullptr, 0};
  if (r < n_dense) {
    // dense HCA rows past the entries stay untouched
    if (r < static_cast<int>(udiv24(L, map.m[gi])) && pi < map.bt_stride[gi] && page >= 0 &&
        page < map.n_pages[gi]) {
      rf.src = Ly.pool + (static_cast<int64_t>(page) * bs + (r - pi * bs)) * Ly.entry_bytes;
      rf.dst = static_cast<uint8_t*>(Ly.out_entries) + (static_cast<int64_t>(b) * Ly.out_rows + r) * out_row;
      rf.kind = (Ly.format == SKV_FMT_FP8) ? 2 : 1;
    }
  } else if (Ly.out_window && r < n_dense + Ly.window) {
    const int w = r - n_dense;
    const int cnt = min(max(L, 0), Ly.window);
    if (w < cnt) {
      const int64_t slot = umod24(static_cast<uint32_t>(L - cnt + w), Ly.window);
      rf.src = Ly.ring + (static_cast<int64_t>(b) * Ly.window + slot) * out_row;
      rf.dst = static_cast<uint8_t*>(Ly.out_window) + (static_cast<int64_t>(b) * Ly.window + w) * out_row;
      rf.kind = 1;
    }
  }
  // one pass of copy_rows covers the tile (kGatherRowsD rows at once), so
  // row(r) is always this thread's own row
  copy_rows<kDenseTPR, kDenseU, kWB>(
      kGatherRowsD, [&](int) { return rf; }, latent, g >= 0 && Ly.format == SKV_FMT_FP8, d);
}

// ---------------------------------------------------------------------------
// 4. top-k ordering + sparse gather of one part of a row.  Part p of a row
//    owns output positions [p*rank_out, (p+1)*rank_out), rank_out 8, 16 or 32.
//    The row's candidates sit in LDS as 64-bit order keys (key << 32 | ~idx:
//    larger means earlier in the output), the sure list [0, S) then the tie
//    list [S, C), each in the same order in every part.  A part ranks its
//    candidates p, p + parts, ... of each list within that list (a lane
//    group per kRankR candidates, each lane comparing a strided share of the
//    list with all of them; the groups of both lists run side by side),
//    writes every winner's index and entry at its output position, and gives the
//    positions in [sel, top_k) it owns index -1 and entry 0 (the reference's
//    clamp(min=0) before its gather).
// ---------------------------------------------------------------------------
constexpr int kRankOutMin = 8;
constexpr int kRankOut = 32;
constexpr int kRankMaxRows = 512;                    // rows one part can collect (checked below)

// Rows a part collects, worst case over top_k and the part size: its sure
// winners (at most ceil(top_k/parts) <= part size), its tie winners (at most
// ceil(kTkTieCap/parts) and at most top_k in all) and its fills (< part size).
constexpr int rank_rows_max() {
  int worst = 0;
  for (int out = kRankOutMin; out <= kRankOut; out *= 2) {
    for (int k = 1; k <= kMaxTopK; ++k) {
      const int parts = (k + out - 1) / out;
      int win = out + (kTkTieCap + parts - 1) / parts;
      if (win > k) win = k;
      if (win + out > worst) worst = win + out;
    }
  }
  return worst;
}
static_assert(rank_rows_max() <= kRankMaxRows, "rank row lists too small");

struct RankRows {
  int n_rows;
  int2 win[kRankMaxRows];            // (output position, pick)
  uintptr_t src_kind[kRankMaxRows];  // entry address | row kind (entries are 4-byte aligned)
};

// Adds the fills [f0, o1), writes the indices and copies every collected row.
// n_rows: rows collected so far (read after a barrier by the caller).
template <bool kWB>
__device__ __forceinline__ void finish_rows(RankRows& rr, int n_rows, int f0, int o1,
                                            const skv_decode_desc* d, const GatherLayer& Ly, int k,
                                            const GroupRef& G, int b, int L, const int32_t* bt_lds, int n_lds) {
  const int tid = threadIdx.x;
  if (tid < o1 - f0) rr.win[n_rows + tid] = make_int2(f0 + tid, -1);
  n_rows += max(0, o1 - f0);
  __syncthreads();
  const int n_ent = static_cast<int>(udiv24(L, G.m));
  const int64_t out_row = static_cast<int64_t>(Ly.latent) * 2;
  int32_t* out_idx = Ly.topk_idx + static_cast<int64_t>(b) * k;
  if (!Ly.out_entries) {  // uniform: the step writes the indices only
    for (int w = tid; w < n_rows; w += kStepThreads) out_idx[rr.win[w].x] = rr.win[w].y;
    return;
  }
  uint8_t* out_base = static_cast<uint8_t*>(Ly.out_entries) + static_cast<int64_t>(b) * k * out_row;
  for (int w = tid; w < n_rows; w += kStepThreads) {
    const int2 pw = rr.win[w];
    out_idx[pw.x] = pw.y;
    const uint8_t* s = nullptr;
    const int kind = entry_source(G, Ly, b, pw.y < 0 ? 0 : pw.y, n_ent, &s, bt_lds, n_lds);
    rr.src_kind[w] = reinterpret_cast<uintptr_t>(s) | static_cast<uintptr_t>(kind ? kind : 3);
  }
  __syncthreads();
  copy_rows<8, 9, kWB>(
      n_rows,
      [&](int r) {
        const uintptr_t sk = rr.src_kind[r];
        return RowRef{global_from_bits<const uint8_t>(sk & ~static_cast<uintptr_t>(3)),
                      out_base + rr.win[r].x * out_row, static_cast<int>(sk & 3)};
      },
      Ly.latent, Ly.format == SKV_FMT_FP8, d);
}

// ---------------------------------------------------------------------------
// 5. gather launch: rank parts, each loading its row's candidate lists,
//    ranking and gathering, interleaved with the dense tiles, whose copies
//    keep HBM busy while the rank parts wait on their round trips.  Part 0
//    of a row zeroes the row's histogram for the next step, also after a
//    refusal.
// ---------------------------------------------------------------------------
constexpr int kRankHead = 2 * kStepThreads;  // entries of each candidate list fetched with the counters
constexpr int kRankBt = 16 * kStepThreads;   // most block-table entries of a sequence staged in LDS
constexpr int kRankPf = kStepThreads / 8;    // own candidates whose entries are loaded before ranking

// Dynamic LDS of the gather launch, sized by the host for the launch's rows:
//   RankHead | block-table row (bt_lds entries) | candidates (ck_cap order keys)
//                                                  or the full-select fallback
struct RankHead {
  RankRows rr;
  int own_pos[kRankPf];
};
struct RankFallback {
  TopkSmemT<kStepThreads> full;
};

__host__ __device__ constexpr int64_t align16(int64_t x) { return (x + 15) & ~static_cast<int64_t>(15); }

__host__ __device__ constexpr int64_t rank_lds_bytes(int bt_lds, int ck_cap) {
  const int64_t region = static_cast<int64_t>(ck_cap) * 8 > static_cast<int64_t>(sizeof(RankFallback))
                             ? static_cast<int64_t>(ck_cap) * 8 : static_cast<int64_t>(sizeof(RankFallback));
  return align16(sizeof(RankHead)) + align16(static_cast<int64_t>(bt_lds) * 4) + region;
}

// One memory round trip brings the status, the length, the list counters,
// the heads of both candidate lists and the sequence's block-table row;
// longer lists take a second one.  Ranking then runs on LDS (or, for lists
// longer than the launch's LDS holds, on the lists in global memory), page
// lookups read the LDS table, and the entry copy is the last round trip.
template <bool kWB>
__device__ __forceinline__ void rank_part_body(const skv_decode_desc* __restrict__ d, const StepMap& map,
                                               uint8_t* rank_lds, int part, int b, int z, int rank_out, int bt_lds,
                                               int ck_cap) {
  RankHead& sm = *reinterpret_cast<RankHead*>(rank_lds);
  int32_t* sm_bt = reinterpret_cast<int32_t*>(rank_lds + align16(sizeof(RankHead)));
  uint8_t* region = rank_lds + align16(sizeof(RankHead)) + align16(static_cast<int64_t>(bt_lds) * 4);
  uint64_t* sm_ck = reinterpret_cast<uint64_t*>(region);
  RankFallback& fb = *reinterpret_cast<RankFallback*>(region);
  const int li = static_cast<int>((map.csa >> (4 * z)) & 15);
  const GatherLayer Ly = gather_layer(d, d->layers[li]);
  const int gi = map.group[li];
  const int tid = threadIdx.x;
  int32_t* ws = map.topk_ws[z] + static_cast<int64_t>(b) * kTkWsWords;
  const int2* sure_list = reinterpret_cast<const int2*>(ws + kTkWsSure);
  const int2* tie_list = reinterpret_cast<const int2*>(ws + kTkWsTie);
  const int32_t* bt_row = map.block_table[gi] + static_cast<int64_t>(b) * map.bt_stride[gi];
  const int n_bt = min(map.bt_stride[gi], bt_lds);
  // every load of the first round trip, unconditional (clamped indices)
  const int status = *map.status;
  const int L = map.step_lens[b];
  const int cnt0 = ws[kTkWsCnt], cnt1 = ws[kTkWsCnt + 1], flag = ws[kTkWsCnt + 2];
  int2 sh[kRankHead / kStepThreads], th[kRankHead / kStepThreads];
#pragma unroll
  for (int u = 0; u < kRankHead / kStepThreads; ++u) {
    sh[u] = sure_list[tid + u * kStepThreads];
    th[u] = tie_list[tid + u * kStepThreads];
  }
  // the row's slices only (uniform bound): short rows issue one load, not 16
  int32_t btv[kRankBt / kStepThreads];
#pragma unroll
  for (int u = 0; u < kRankBt / kStepThreads; ++u) {
    if (u * kStepThreads >= n_bt) break;
    btv[u] = bt_row[min(tid + u * kStepThreads, n_bt - 1)];
  }
  hold_fields(Ly, false);
  const int k = map.top_k[z];
  const int parts = static_cast<int>(ceil_div24(k, rank_out));
  if (part >= parts) return;  // the grid is sized for the largest top_k
  const GroupRef G = group_ref(map, gi);
  if (status) return;  // refused step
  int n_cols, n_valid;
  score_cols(map.score_stride[z], G.m, L, n_cols, n_valid);
  const int sel = topk_sel(k, n_cols, n_valid);
#pragma unroll
  for (int u = 0; u < kRankBt / kStepThreads; ++u) {
    if (u * kStepThreads >= n_bt) break;
    if (tid + u * kStepThreads < n_bt) sm_bt[tid + u * kStepThreads] = btv[u];
  }
  if (tid == 0) sm.rr.n_rows = 0;
  const int o0 = part * rank_out;
  const int o1 = min(k, o0 + rank_out);
  if (sel > 0 && flag) {
    // tie bin over the list capacity: full select of the row, keeping this
    // part's positions (each is emitted once)
    topk_row_emit<kStepThreads>(fb.full, nullptr, map.scores[z] + static_cast<int64_t>(b) * map.score_stride[z],
                                n_cols, n_valid, k, [&](int j, int v) {
                                  if (j >= o0 && j < o1) sm.rr.win[j - o0] = make_int2(j, v);
                                });
    __syncthreads();
    finish_rows<kWB>(sm.rr, o1 - o0, o1, o1, d, Ly, k, G, b, L, sm_bt, n_bt);
    return;
  }
  if (sel > 0) {
    const int S = min(cnt0, kMaxTopK);
    const int T = min(cnt1, kTkTieCap);
    const int C = S + T;
    const bool in_lds = C <= ck_cap;  // uniform
    if (in_lds) {
#pragma unroll
      for (int u = 0; u < kRankHead / kStepThreads; ++u) {
        const int c = tid + u * kStepThreads;
        if (c < S) sm_ck[c] = order_key(sh[u]);
        if (c < T) sm_ck[S + c] = order_key(th[u]);
      }
      if (S > kRankHead || T > kRankHead) {  // uniform: the rest of the lists
        constexpr int kLoad = 8;  // list loads in flight per thread
        for (int c0 = tid; c0 < C; c0 += kStepThreads * kLoad) {
          int2 v[kLoad];
#pragma unroll
          for (int u = 0; u < kLoad; ++u) {
            const int c = min(c0 + u * kStepThreads, C - 1);  // unconditional: C >= sel > 0
            v[u] = (c < S ? sure_list : tie_list - S)[c];
          }
#pragma unroll
          for (int u = 0; u < kLoad; ++u) {
            const int c = c0 + u * kStepThreads;
            const bool in_head = c < S ? c < kRankHead : c - S < kRankHead;
            // keyed unconditionally: a load used only under a branch that a
            // wave may skip stays pending in the compiler's count, and later
            // register reuse would then wait for every load in flight
            const uint64_t key = order_key(v[u]);
            asm volatile("" ::"v"(key));
            if (c < C && !in_head) sm_ck[c] = key;
          }
        }
      }
    }
    __syncthreads();
    const auto lds_key = [&](int q) { return sm_ck[q]; };
    const auto collect = [&](int pos, int idx) { sm.rr.win[atomicAdd(&sm.rr.n_rows, 1)] = make_int2(pos, idx); };
    const auto global_key = [&](int q) { return order_key(q < S ? sure_list[q] : tie_list[q - S]); };
    // the entries of up to kRankPf of the part's candidates (all of them, or
    // else its sure ones, which always win) are loaded first, so that the
    // loads overlap the ranking; they are stored after it, and the other
    // winners are collected and copied after it
    const int n_sure_mine = (part < S) ? static_cast<int>(ceil_div24(S - part, parts)) : 0;
    const int n_own = n_sure_mine + ((part < T) ? static_cast<int>(ceil_div24(T - part, parts)) : 0);
    constexpr int kPfU = 9;  // 8 threads x 9 tasks cover a 576-channel row (bf16 72 chunks, fp8 40 tasks)
    const bool fp8 = Ly.format == SKV_FMT_FP8;
    const int n_pf = (n_own <= kRankPf) ? n_own : min(n_sure_mine, kRankPf);
    if (in_lds && n_pf > 0 && Ly.out_entries && entry_tasks<8, kPfU>(Ly.latent, fp8) <= 8 * kPfU) {  // uniform
      const int r = tid / 8;
      int pick = -1, kind = 0;
      const uint8_t* src = nullptr;
      if (r < n_pf) {
        const int c = (r < n_sure_mine) ? part + r * parts : S + part + (r - n_sure_mine) * parts;
        const uint64_t v = sm_ck[c];
        pick = key_finite(static_cast<uint32_t>(v >> 32)) ? static_cast<int>(~static_cast<uint32_t>(v)) : -1;
        kind = entry_source(G, Ly, b, pick < 0 ? 0 : pick, static_cast<int>(udiv24(L, G.m)), &src, sm_bt, n_bt);
        if (kind == 0) kind = 3;
      }
      EntryShare<kPfU> share;
      entry_share_load<8, kPfU>(share, src, kind, Ly.latent, fp8, reinterpret_cast<const u32x4*>(d));
      rank_candidates<kStepThreads>(collect, lds_key, S, C, sel, part, parts, sm.own_pos, n_pf);
      __syncthreads();
      const int pos = (r < n_pf) ? sm.own_pos[r] : -1;
      if (pos >= 0) {
        const int64_t out_row = static_cast<int64_t>(Ly.latent) * 2;
        if ((tid & 7) == 0) Ly.topk_idx[static_cast<int64_t>(b) * k + pos] = pick;
        entry_share_store<8, kPfU, kWB>(share, static_cast<uint8_t*>(Ly.out_entries) +
                                              (static_cast<int64_t>(b) * k + pos) * out_row,
                                   kind, Ly.latent, fp8);
      }
      // the other winners and the fills
      finish_rows<kWB>(sm.rr, sm.rr.n_rows, max(o0, sel), o1, d, Ly, k, G, b, L, sm_bt, n_bt);
      return;
    }
    if (in_lds) rank_candidates<kStepThreads>(collect, lds_key, S, C, sel, part, parts);
    else rank_candidates<kStepThreads>(collect, global_key, S, C, sel, part, parts);
  }
  __syncthreads();
  finish_rows<kWB>(sm.rr, sm.rr.n_rows, max(o0, sel), o1, d, Ly, k, G, b, L, sm_bt, n_bt);
}

// A rank part; part 0 then clears the row's histogram for the next step
// (also after a refusal).  The clear comes last: stores issued while the
// part's loads are in flight would make every later wait for a load wait for
// all of them (the compiler cannot count on a mix of loads and stores
// completing in order).
template <bool kWB>
__device__ __forceinline__ void rank_part(const skv_decode_desc* __restrict__ d, const StepMap& map,
                                          uint8_t* rank_lds, int part, int b, int z, int rank_out, int bt_lds,
                                          int ck_cap) {
  rank_part_body<kWB>(d, map, rank_lds, part, b, z, rank_out, bt_lds, ck_cap);
  if (part == 0) {
    int32_t* ws = map.topk_ws[z] + static_cast<int64_t>(b) * kTkWsWords;
    for (int i = static_cast<int>(threadIdx.x); i < kTkBins; i += kStepThreads) ws[kTkWsHist + i] = 0;
  }
}

// Blocks of the gather launch, in groups of map.lanes blocks (one block per
// XCD when the lanes are the XCDs): group i * period is the i-th group
// of rank parts (batch * parts_max * CSA layers of them, placed as xcd_item
// places them), every other group holds the next dense tiles.  period *
// n_rank_groups <= the groups of the grid, so every rank group is in it;
// blocks past the dense tiles exit.
struct GatherGrid {
  int32_t n_rank_groups;
  int32_t parts_max;
  int32_t period;
  int32_t n_dense;
};

template <bool kWB>
__global__ __launch_bounds__(kStepThreads) void k_decode_gather(const skv_decode_desc* __restrict__ d,
                                                                GatherGrid gg, int rank_out, int bt_lds,
                                                                int ck_cap, StepMap map) {
  extern __shared__ __align__(16) uint8_t rank_lds[];
  const uint32_t u = blockIdx.x;  // grids stay below 2^24 workgroups
  const int lanes = map.lanes;  // a power of two
  const uint32_t g = u >> __builtin_ctz(static_cast<uint32_t>(lanes));  // the block's group
  const uint32_t i = udiv24(g, gg.period);
  if (g == i * gg.period && static_cast<int>(i) < gg.n_rank_groups) {
    int b, r;
    if (!xcd_item(i * lanes + (u & (lanes - 1)), gg.parts_max * map.n_csa, map.batch, lanes, b, r)) return;
    const int z = static_cast<int>(udiv24(r, gg.parts_max));
    rank_part<kWB>(d, map, rank_lds, r - z * gg.parts_max, b, z, rank_out, bt_lds, ck_cap);
    return;
  }
  const int dense = static_cast<int>(u) - lanes * min(static_cast<int>(ceil_div24(g, gg.period)), gg.n_rank_groups);
  if (dense < gg.n_dense) dense_block<kWB>(d, map, dense);
}

}  // namespace skv

using namespace skv;

namespace {

constexpr int64_t kLdsPerCu = 160 * 1024;
// LDS is allocated to a workgroup in 1280-byte granules on MI355X (measured:
// four workgroups of 40,960 bytes share a CU, three of 53,744 do, three of
// 54,272 do not); the runtime's occupancy calculator assumes a finer granule.
constexpr int64_t kLdsGranule = 1280;

// Most LDS bytes a rank workgroup may take while a CU still holds as many of
// them as it does with `lds` bytes each (the register-limited count caps
// it), a whole number of granules.
template <bool kWB>
int gather_blocks_by_regs() {
  static const int by_regs = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_decode_gather<kWB>, kStepThreads, 0) != hipSuccess ||
        n <= 0) {
      (void)hipGetLastError();
      n = 1 << 20;
    }
    return n;
  }();
  return by_regs;
}

int64_t rank_lds_budget(int64_t lds, bool wb) {
  const int by_regs = wb ? gather_blocks_by_regs<true>() : gather_blocks_by_regs<false>();
  int64_t wgs = kLdsPerCu / ((lds + kLdsGranule - 1) / kLdsGranule * kLdsGranule);
  if (wgs > by_regs) wgs = by_regs;
  if (wgs < 1) wgs = 1;
  return kLdsPerCu / wgs / kLdsGranule * kLdsGranule;
}

}  // namespace

extern "C" int skv_decode_desc_sizes(int64_t* out) {
  if (!out) return set_error(SKV_EINVAL, "skv_decode_desc_sizes: out is NULL");
  out[0] = sizeof(skv_decode_desc);
  out[1] = sizeof(skv_decode_layer);
  out[2] = sizeof(skv_page_group);
  return SKV_OK;
}

extern "C" int skv_decode_step_launches(const skv_decode_desc* h) {
  if (!h) return set_error(SKV_EINVAL, "skv_decode_step_launches: NULL descriptor");
  if (h->batch <= 0 || h->n_layers <= 0) return 0;
  for (int l = 0; l < h->n_layers && l < SKV_MAX_LAYERS; ++l) {
    if (h->layers[l].kind == SKV_LAYER_CSA) return 3;
  }
  return 2;
}

namespace {

// The step's launches; with `att`, the gather launch is replaced by the
// attention launches of decode_attend (checked before anything launches).
int decode_step(const skv_decode_desc* h, const skv_decode_desc* dd, void* stream, const skv_attention_desc* att,
                void* att_ws, int64_t att_ws_bytes, const char* what) {
  if (!h || !dd) return set_error(SKV_EINVAL, "%s: NULL descriptor", what);
  if (h->batch < 0 || h->batch > kDecodeMaxBatch) {
    return set_error(SKV_EINVAL, "%s: batch must be in [0, %d]; got %d", what, kDecodeMaxBatch, h->batch);
  }
  if (h->n_layers < 0 || h->n_layers > SKV_MAX_LAYERS || h->n_groups < 0 || h->n_groups > SKV_MAX_GROUPS) {
    return set_error(SKV_EINVAL, "%s: n_layers <= %d and n_groups <= %d", what, SKV_MAX_LAYERS, SKV_MAX_GROUPS);
  }
  if (h->latent <= 0 || (h->latent & 7) || h->latent > kPoolWave * 8 * kMaxGroups ||
      h->c_indexer < 0 || (h->c_indexer & 7) || h->c_indexer > kPoolWave * 8 * kMaxGroups ||
      h->window <= 0) {
    return set_error(SKV_EINVAL, "%s: latent/c_indexer must be multiples of 8 in range and window > 0", what);
  }
  if (!h->tok_lens || !h->status || !h->step_lens || !h->step_top) {
    return set_error(SKV_EINVAL, "%s: NULL tok_lens/status/step_lens/step_top", what);
  }
  for (int g = 0; g < h->n_groups; ++g) {
    const skv_page_group& G = h->groups[g];
    if (!G.free_stack || !G.free_top || !G.block_table || !G.n_entries || G.m <= 0 ||
        G.block_size <= 0 || G.bt_stride <= 0 || G.n_pages <= 0) {
      return set_error(SKV_EINVAL, "%s: page group %d is incomplete", what, g);
    }
    if (G.bt_stride >= (1 << 24) || G.n_pages > 0x7fffffff) {
      return set_error(SKV_EINVAL, "%s: page group %d needs bt_stride < 2^24 and n_pages < 2^31", what, g);
    }
  }
  StepMap map{};
  map.batch = h->batch;
  map.lanes = xcd_lanes(h->batch);
  // the append launch's filter chunk i runs on the XCD (block index mod XCDs)
  // that ran histogram chunk i, and re-reads its scores from that XCD's L2:
  // the (layer, sequence) blocks before the chunks fill whole rounds of XCDs
  // (with lanes = XCDs they already do; the extra blocks exit at once)
  {
    const int64_t own = xcd_region(h->batch, h->n_layers), x = device_xcds();
    map.n_own = static_cast<int32_t>(map.lanes == 1 && x > 1 ? ceil_div(own, x) * x : own);
  }
  map.n_layers = h->n_layers;
  map.n_groups = h->n_groups;
  map.tok_lens = h->tok_lens;
  map.status = h->status;
  map.step_lens = h->step_lens;
  map.step_top = h->step_top;
  for (int g = 0; g < SKV_MAX_GROUPS; ++g) {
    const bool used = g < h->n_groups;
    map.block_table[g] = used ? h->groups[g].block_table : nullptr;
    map.n_entries[g] = used ? h->groups[g].n_entries : nullptr;
    map.free_stack[g] = used ? h->groups[g].free_stack : nullptr;
    map.free_top[g] = used ? h->groups[g].free_top : nullptr;
    map.bt_stride[g] = used ? static_cast<int32_t>(h->groups[g].bt_stride) : 1;
    map.block_size[g] = used ? h->groups[g].block_size : 1;
    map.m[g] = used ? h->groups[g].m : 1;
    map.n_pages[g] = used ? static_cast<int32_t>(h->groups[g].n_pages) : 1;
  }
  uint32_t groups_seen = 0;
  int n_csa = 0, max_top_k = 0, n_scored = 0;
  ScoreMap sc{};
  sc.c = h->c_indexer;
  int64_t max_score_cols = 1, n_tiles = 0;
  int64_t out_rows = 0;  // rows the gather launch may write (capacity)
  for (int l = 0; l < h->n_layers; ++l) {
    const skv_decode_layer& Ly = h->layers[l];
    map.group[l] = (Ly.kind == SKV_LAYER_SWA) ? -1 : static_cast<int8_t>(Ly.group);
    if (Ly.kind != SKV_LAYER_SWA && Ly.group >= 0 && Ly.group < SKV_MAX_GROUPS && !((groups_seen >> Ly.group) & 1)) {
      groups_seen |= 1u << Ly.group;
      map.group_first |= 1u << l;
    }
    if (!Ly.ring || !Ly.kv_new) return set_error(SKV_EINVAL, "%s: layer %d lacks ring/kv_new", what, l);
    int64_t dense = Ly.out_window ? h->window : 0;
    if (Ly.kind == SKV_LAYER_HCA || Ly.kind == SKV_LAYER_CSA) {
      if (Ly.group < 0 || Ly.group >= h->n_groups) return set_error(SKV_EINVAL, "%s: layer %d group out of range", what, l);
      if (!Ly.pool || !Ly.state || !Ly.bias || !Ly.c_new || !Ly.z_new) {
        return set_error(SKV_EINVAL, "%s: layer %d lacks pool/state/bias/c/z", what, l);
      }
      if (entry_layout(Ly.format, h->latent, Ly.entry_bytes) < 0) {
        return set_error(SKV_EINVAL, "%s: layer %d entry_bytes %lld does not match format %d", what, l,
                         (long long)Ly.entry_bytes, Ly.format);
      }
      if (Ly.kind == SKV_LAYER_CSA) {
        if (Ly.top_k <= 0 || Ly.top_k > kMaxTopK || !Ly.scores || !Ly.topk_idx || !Ly.topk_ws ||
            Ly.score_stride <= 0) {
          return set_error(SKV_EINVAL, "%s: CSA layer %d needs 0 < top_k <= %d, scores, topk_idx and topk_ws",
                           what, l, kMaxTopK);
        }
        max_score_cols = max(max_score_cols, Ly.score_stride);
        if (Ly.idx_pool && (!Ly.idx_state || !Ly.idx_bias || !Ly.ci_new || !Ly.zi_new || h->c_indexer <= 0)) {
          return set_error(SKV_EINVAL, "%s: CSA layer %d indexer stream incomplete", what, l);
        }
        if (Ly.idx_q) {
          if (!Ly.idx_pool || !Ly.idx_w || Ly.idx_heads < 1 || Ly.idx_heads > 16 * kIdxMaxHB ||
              h->c_indexer > 32 * kIdxMaxKS) {
            return set_error(SKV_EINVAL,
                             "%s: CSA layer %d: step scores need the indexer stream, idx_w, 1 <= idx_heads <= %d "
                             "and c_indexer <= %d",
                             what, l, 16 * kIdxMaxHB, 32 * kIdxMaxKS);
          }
          sc.q[n_csa] = static_cast<const uint8_t*>(Ly.idx_q);
          sc.w[n_csa] = Ly.idx_w;
          sc.pool[n_csa] = static_cast<const uint8_t*>(Ly.idx_pool);
          sc.heads[n_csa] = Ly.idx_heads;
          ++n_scored;
        }
        if (Ly.score_stride >= (1 << 24)) {
          return set_error(SKV_EINVAL, "%s: CSA layer %d score_stride >= 2^24", what, l);
        }
        map.csa |= static_cast<uint64_t>(l) << (4 * n_csa);
        map.topk_ws[n_csa] = Ly.topk_ws;
        map.scores[n_csa] = Ly.scores;
        map.score_stride[n_csa] = static_cast<int32_t>(Ly.score_stride);
        map.top_k[n_csa] = Ly.top_k;
        ++n_csa;
        max_top_k = max(max_top_k, Ly.top_k);
      } else {
        map.hca_mask |= 1u << l;
        if (Ly.out_entries) {
          if (Ly.out_rows <= 0 || Ly.out_rows > (1 << 24)) {
            return set_error(SKV_EINVAL, "%s: HCA layer %d needs 0 < out_rows <= 2^24", what, l);
          }
          dense += Ly.out_rows;
        }
      }
    } else if (Ly.kind != SKV_LAYER_SWA) {
      return set_error(SKV_EINVAL, "%s: layer %d has unknown kind %d", what, l, Ly.kind);
    }
    if (dense >= (1 << 24)) return set_error(SKV_EINVAL, "%s: layer %d has 2^24 dense rows or more", what, l);
    out_rows += (dense + ((Ly.kind == SKV_LAYER_CSA && Ly.out_entries) ? Ly.top_k : 0)) * h->batch;
    // layer 0 keeps a tile per sequence even with nothing to copy: its tile 0
    // commits the step
    const int64_t tiles = (l == 0 && dense == 0) ? 1 : ceil_div(dense, kGatherRowsD);
    map.tiles[l] = static_cast<int32_t>(tiles);
    n_tiles += tiles * h->batch;
    map.tile_end[l] = static_cast<int32_t>(n_tiles < (1 << 24) ? n_tiles : (1 << 24));
  }
  for (int l = h->n_layers; l < SKV_MAX_LAYERS; ++l) {
    map.tiles[l] = 1;
    map.tile_end[l] = static_cast<int32_t>(n_tiles < (1 << 24) ? n_tiles : (1 << 24));
  }
  map.n_csa = n_csa;
  if (n_scored != 0 && n_scored != n_csa) {
    return set_error(SKV_EINVAL, "%s: either every CSA layer sets idx_q or none does", what);
  }
  if (att) {  // every argument of the attention launches, before anything launches
    const int rc = decode_attend(att, h, nullptr, att_ws, att_ws_bytes, nullptr, nullptr, true);
    if (rc != SKV_OK) return rc;
  }
  if (h->batch == 0 || h->n_layers == 0) return SKV_OK;
  const int n_chunks = static_cast<int>(ceil_div(max_score_cols, kTkChunk));
  const int64_t n_append = map.n_own + xcd_region(h->batch, static_cast<int64_t>(n_chunks) * n_csa);
  const int64_t n_hist = xcd_region(h->batch, static_cast<int64_t>(n_chunks) * n_csa);
  // smaller parts when the rows alone would leave most CUs idle
  int rank_out = kRankOut;
  while (rank_out > kRankOutMin && static_cast<int64_t>(h->batch) * n_csa * ceil_div(max_top_k, rank_out) < 512) {
    rank_out >>= 1;
  }
  const int64_t parts_max = ceil_div(max_top_k, rank_out);
  const int lanes = map.lanes;
  const int64_t n_rank_groups = xcd_region(h->batch, parts_max * n_csa) / lanes;
  const int64_t n_gather = lanes * ceil_div(lanes * n_rank_groups + n_tiles, lanes);
  if (n_append >= (1 << 24) || n_gather >= (1 << 24)) {
    return set_error(SKV_EINVAL, "%s: score_stride/out_rows give a grid of 2^24 workgroups or more", what);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
  if (n_hist > 0 && n_scored > 0) {
    const int n_score_tiles = static_cast<int>(ceil_div(max_score_cols, kIdxTile));
    const int64_t n_score = xcd_region(h->batch, static_cast<int64_t>(n_score_tiles) * n_csa);
    if (n_score >= (1 << 24)) return set_error(SKV_EINVAL, "%s: score grid of 2^24 workgroups or more", what);
    hipLaunchKernelGGL(k_decode_score_hist, dim3(static_cast<unsigned>(n_score)), dim3(kIdxThreads), 0, s,
                       n_score_tiles, map, sc);
    if ((rc = check_launch(what))) return rc;
  } else if (n_hist > 0) {
    hipLaunchKernelGGL(k_decode_hist, dim3(static_cast<unsigned>(n_hist)), dim3(kTkPartThreads), 0, s, n_chunks,
                       map);
    if ((rc = check_launch(what))) return rc;
  }
  hipLaunchKernelGGL(k_decode_append, dim3(static_cast<unsigned>(n_append)), dim3(kStepThreads), 0, s, dd,
                     n_chunks, map);
  if ((rc = check_launch(what))) return rc;
  if (att) return decode_attend(att, h, &map, att_ws, att_ws_bytes, s, nullptr, true);
  GatherGrid gg;
  gg.n_rank_groups = static_cast<int32_t>(n_rank_groups);
  gg.parts_max = static_cast<int32_t>(parts_max);
  gg.period = n_rank_groups > 0 ? static_cast<int32_t>(n_gather / lanes / n_rank_groups) : 1;
  gg.n_dense = static_cast<int32_t>(n_tiles);
  // The gathered rows' stores: plain (allocating) stores when the rows the
  // launch may write come to 96-256 MiB, nontemporal stores otherwise.
  // Measured on MI355X (one CSA layer at 64k, B = 64..512; the 8-layer
  // CSA/HCA step, B = 16..64): from about 100 MiB up to the 256 MiB
  // last-level cache, rows written with plain stores stay in that cache and
  // the step runs 2-8% faster; below, the nontemporal stores' smaller
  // write-back at the end of the launch wins (up to 1.5 us at B = 16); above,
  // plain stores thrash the cache (up to 7% slower).
  const int64_t out_bytes = out_rows * h->latent * 2;
  const bool wb = out_bytes >= (static_cast<int64_t>(96) << 20) && out_bytes <= (static_cast<int64_t>(256) << 20);
  int bt = 1, ck_cap = 0;
  int64_t lds = 0;
  if (n_csa > 0) {
    // LDS sized for this launch: the longest block-table row of a CSA group
    // (at most kRankBt entries) and at least the candidate lists of rows
    // whose tie bin holds 2048 keys, grown while the workgroups a CU holds
    // stay the same; rows with longer lists rank from global memory
    int64_t bt_lds = 1;
    for (int l = 0; l < h->n_layers; ++l) {
      if (h->layers[l].kind == SKV_LAYER_CSA) bt_lds = max(bt_lds, h->groups[h->layers[l].group].bt_stride);
    }
    if (bt_lds > kRankBt) bt_lds = kRankBt;
    bt = static_cast<int>(bt_lds);
    ck_cap = min(max_top_k + 2048, kTkCand);
    const int64_t per_wg = rank_lds_budget(rank_lds_bytes(bt, ck_cap), wb);
    while (ck_cap < kTkCand && rank_lds_bytes(bt, min(ck_cap + 256, kTkCand)) <= per_wg) {
      ck_cap = min(ck_cap + 256, kTkCand);
    }
    lds = rank_lds_bytes(bt, ck_cap);
  }
  if (wb) {
    hipLaunchKernelGGL(k_decode_gather<true>, dim3(static_cast<unsigned>(n_gather)), dim3(kStepThreads),
                       static_cast<size_t>(lds), s, dd, gg, rank_out, bt, ck_cap, map);
  } else {
    hipLaunchKernelGGL(k_decode_gather<false>, dim3(static_cast<unsigned>(n_gather)), dim3(kStepThreads),
                       static_cast<size_t>(lds), s, dd, gg, rank_out, bt, ck_cap, map);
  }
  return check_launch(what);
}

}  // namespace

extern "C" int skv_decode_step(const skv_decode_desc* h, const skv_decode_desc* dd, void* stream) {
  return decode_step(h, dd, stream, nullptr, nullptr, 0, "skv_decode_step");
}

extern "C" int64_t skv_decode_step_attend_workspace(const skv_decode_desc* h, const skv_attention_desc* attn) {
  if (!h || !attn || h->n_layers < 0 || h->n_layers > SKV_MAX_LAYERS || h->n_groups < 0 ||
      h->n_groups > SKV_MAX_GROUPS) {
    set_error(SKV_EINVAL, "skv_decode_step_attend_workspace: NULL or bad descriptor");
    return -1;
  }
  int64_t need = 0;
  if (decode_attend(attn, h, nullptr, nullptr, 0, nullptr, &need, false) != SKV_OK) return -1;
  return need;
}

extern "C" int skv_decode_step_attend(const skv_decode_desc* h, const skv_decode_desc* dd,
                                      const skv_attention_desc* attn, void* workspace, int64_t ws_bytes,
                                      void* stream) {
  const char* what = "skv_decode_step_attend";
  if (!attn) return set_error(SKV_EINVAL, "%s: NULL attention descriptor", what);
  return decode_step(h, dd, stream, attn, workspace, ws_bytes, what);
}
