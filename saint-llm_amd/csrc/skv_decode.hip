// Fused decode step over a stack of heterogeneous layers: four launches per
// step whatever the number of layers (plan; append/compress + top-k
// histograms; top-k filter + dense gathers; top-k rank + sparse gather).
//
// Reference: one cached decode call of SaintLLM.forward walks the blocks and
// hands each attention its cache layer (model.py:294-315); the per-layer cache
// work is SWAKVCacheLayer/HCAKVCacheLayer/CSAKVCacheLayer.append
// (kv_cache.py:63-83, 138-202, 266-322), the CSA indexer top-k
// (csa.py:377-422), the sparse gather (csa.py:326-331), the HCA dense read
// (hca.py:126-141) and the SWA window (swa.py:115-125).
#include "skv_pool_state.h"
#include "skv_topk.h"

namespace skv {

constexpr int kDecodeMaxBatch = 1024;
constexpr int kPlanThreads = 1024;
constexpr int kGatherThreadsD = 256;
#ifndef SKV_GATHER_ROWS
#define SKV_GATHER_ROWS 8
#endif
constexpr int kGatherRowsD = SKV_GATHER_ROWS;  // output rows per gather workgroup

// ---------------------------------------------------------------------------
// 1. plan: token counts +1 and page reservation of every group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kPlanThreads) void k_decode_plan(const skv_decode_desc* __restrict__ d) {
  __shared__ int off[SKV_MAX_GROUPS][kDecodeMaxBatch + 1];
  __shared__ int first[SKV_MAX_GROUPS][kDecodeMaxBatch];
  __shared__ int total[SKV_MAX_GROUPS];
  __shared__ int scan_lds[17];
  __shared__ int bad_all;
  const int tid = threadIdx.x;
  const int batch = d->batch;
  if (tid == 0) bad_all = 0;
  __syncthreads();
  int bad = 0;
  for (int g = 0; g < d->n_groups; ++g) {
    const skv_page_group& G = d->groups[g];
    int need = 0;
    if (tid < batch) {
      const int L1 = d->tok_lens[tid] + 1;
      const int cur = G.n_entries[tid];
      const int target = L1 / G.m;
      if (target < cur) {
        bad |= SKV_STATUS_BADARG;
      } else {
        const int64_t p0 = ceil_div(cur, G.block_size);
        const int64_t p1 = ceil_div(target, G.block_size);
        if (p1 > G.bt_stride) bad |= SKV_STATUS_MAX_PAGES;
        need = static_cast<int>(p1 - p0);
        first[g][tid] = static_cast<int>(p0);
      }
    }
    int tot;
    const int ex = block_exclusive_scan(need, scan_lds, &tot);
    if (tid < batch) off[g][tid] = ex;
    if (tid == 0) {
      off[g][batch] = tot;
      total[g] = tot;
    }
    const int top = *G.free_top;
    if (top < 0 || top > G.n_pages) bad |= SKV_STATUS_BADARG;
    else if (tot > top) bad |= SKV_STATUS_NOSPC;
  }
  if (bad) atomicOr(&bad_all, bad);
  __syncthreads();
  if (bad_all) {
    if (tid == 0) *d->status = bad_all;
    return;
  }
  for (int g = 0; g < d->n_groups; ++g) {
    const skv_page_group& G = d->groups[g];
    const int top = *G.free_top;
    const int tot = total[g];
    for (int t = tid; t < tot; t += kPlanThreads) {
      int lo = 0, hi = batch;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[g][mid] <= t) lo = mid; else hi = mid;
      }
      G.block_table[static_cast<int64_t>(lo) * G.bt_stride + first[g][lo] + (t - off[g][lo])] =
          G.free_stack[top - 1 - t];
    }
    __syncthreads();  // every thread has read free_top before it moves
    if (tid < batch) G.n_entries[tid] = (d->tok_lens[tid] + 1) / G.m;
    if (tid == 0) *G.free_top = top - tot;
  }
  __syncthreads();  // n_entries used the old token count
  if (tid < batch) d->tok_lens[tid] += 1;
  if (tid == 0) *d->status = 0;
}

// ---------------------------------------------------------------------------
// 2. append + top-k histograms, one launch, 256-thread workgroups:
//    blocks [0, batch*layers)        : (sequence, layer) appends — wave 0-1 fold
//                                      the main stream, wave 2 the indexer stream,
//                                      wave 3 copies the ring row;
//    blocks [batch*layers, + chunks*batch*csa) : top-k histogram chunks.
// ---------------------------------------------------------------------------
constexpr int kAppendThreads = 256;

__device__ __forceinline__ const skv_decode_layer* csa_layer(const skv_decode_desc* d, int want) {
  for (int li = 0; li < d->n_layers; ++li) {
    if (d->layers[li].kind == SKV_LAYER_CSA && want-- == 0) return &d->layers[li];
  }
  return nullptr;
}

// Fold the token into the running state of channel groups t, t + nt (8
// channels each) of one stream and emit the entry when the block completes.
// All threads t in [0, nt) of a stream must call it (fp8 amax shuffles span
// the 16 lanes of a 128-channel block, which nt = 128 keeps inside a wave).
__device__ __forceinline__ void decode_fold_part(const skv_page_group& G, int b, int64_t p, void* pool,
                                                 int64_t entry_bytes, float* state, const float* bias,
                                                 const void* c_all, const void* z_all, int channels,
                                                 int format, int fp8_main, int t, int nt) {
  const int groups = channels >> 3;
  float* sbase = state + static_cast<int64_t>(b) * 3 * channels;
  const uint16_t* crow = static_cast<const uint16_t*>(c_all) + static_cast<int64_t>(b) * channels;
  const uint16_t* zrow = static_cast<const uint16_t*>(z_all) + static_cast<int64_t>(b) * channels;
  const float* brow = bias + (p % G.m) * channels;
  const bool fresh = (p % G.m) == 0;
  const bool emit = ((p + 1) % G.m) == 0;
  uint8_t* entry = nullptr;
  if (emit) {
    const int64_t e = (p + 1) / G.m - 1;
    const int64_t pi = e / G.block_size;
    const int32_t page = (pi < G.bt_stride) ? G.block_table[b * G.bt_stride + pi] : -1;
    if (page >= 0 && page < G.n_pages) {
      entry = static_cast<uint8_t*>(pool) +
              (static_cast<int64_t>(page) * G.block_size + e % G.block_size) * entry_bytes;
    }
  }
  for (int grp = t; grp < ((groups + nt - 1) / nt) * nt; grp += nt) {
    const bool mine = grp < groups;
    float mx[8], sum[8], acc[8];
    if (mine && !fresh) {
      const u32x4* sp = reinterpret_cast<const u32x4*>(sbase + grp * 8);
      const u32x4 m0 = sp[0], m1 = sp[1];
      const u32x4 s0 = *reinterpret_cast<const u32x4*>(sbase + channels + grp * 8);
      const u32x4 s1 = *(reinterpret_cast<const u32x4*>(sbase + channels + grp * 8) + 1);
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(sbase + 2 * channels + grp * 8);
      const u32x4 a1 = *(reinterpret_cast<const u32x4*>(sbase + 2 * channels + grp * 8) + 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        mx[j] = __uint_as_float(m0[j]);
        mx[j + 4] = __uint_as_float(m1[j]);
        sum[j] = __uint_as_float(s0[j]);
        sum[j + 4] = __uint_as_float(s1[j]);
        acc[j] = __uint_as_float(a0[j]);
        acc[j + 4] = __uint_as_float(a1[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mx[j] = -INFINITY;
        sum[j] = 0.f;
        acc[j] = 0.f;
      }
    }
    float out[8];
    if (mine) {
      float c[8], z[8];
      unpack8_bf16(*reinterpret_cast<const u32x4*>(crow + grp * 8), c);
      unpack8_bf16(*reinterpret_cast<const u32x4*>(zrow + grp * 8), z);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = z[j] + brow[grp * 8 + j];
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
        out[j] = bf16_to_f32(f32_to_bf16(acc[j] / sum[j]));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) out[j] = 0.f;
    }
    if (emit) {
      if (entry) store_entry_group(entry, out, grp, groups, format, fp8_main);
    } else if (mine) {
      u32x4* sp = reinterpret_cast<u32x4*>(sbase + grp * 8);
      sp[0] = u32x4{__float_as_uint(mx[0]), __float_as_uint(mx[1]), __float_as_uint(mx[2]), __float_as_uint(mx[3])};
      sp[1] = u32x4{__float_as_uint(mx[4]), __float_as_uint(mx[5]), __float_as_uint(mx[6]), __float_as_uint(mx[7])};
      u32x4* ss = reinterpret_cast<u32x4*>(sbase + channels + grp * 8);
      ss[0] = u32x4{__float_as_uint(sum[0]), __float_as_uint(sum[1]), __float_as_uint(sum[2]), __float_as_uint(sum[3])};
      ss[1] = u32x4{__float_as_uint(sum[4]), __float_as_uint(sum[5]), __float_as_uint(sum[6]), __float_as_uint(sum[7])};
      u32x4* sa = reinterpret_cast<u32x4*>(sbase + 2 * channels + grp * 8);
      sa[0] = u32x4{__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]), __float_as_uint(acc[3])};
      sa[1] = u32x4{__float_as_uint(acc[4]), __float_as_uint(acc[5]), __float_as_uint(acc[6]), __float_as_uint(acc[7])};
    }
  }
}

__global__ __launch_bounds__(kAppendThreads) void k_decode_append(const skv_decode_desc* __restrict__ d,
                                                                  int n_chunks) {
  __shared__ TopkHistSmem hsm;
  if (*d->status) return;  // refused step: no state changes
  const int n_append = d->batch * d->n_layers;
  if (static_cast<int>(blockIdx.x) >= n_append) {
    // top-k histogram chunk (chunk, b, csa layer); chunk 0 also zeroes the
    // row's list counters, which the previous step's rank launch still read
    int u = blockIdx.x - n_append;
    const int chunk = u % n_chunks;
    u /= n_chunks;
    const int b = u % d->batch;
    const skv_decode_layer* Ly = csa_layer(d, u / d->batch);
    if (!Ly) return;
    int32_t* ws = Ly->topk_ws + static_cast<int64_t>(b) * kTkWsWords;
    if (chunk == 0 && threadIdx.x < 3) ws[kTkWsCnt + threadIdx.x] = 0;
    const int m = d->groups[Ly->group].m;
    const int L = d->tok_lens[b];
    topk_hist_chunk(hsm, Ly->scores + static_cast<int64_t>(b) * Ly->score_stride, L / m,
                    L > 0 ? (L - 1) / m : 0, Ly->top_k, chunk, ws);
    return;
  }
  const int b = blockIdx.x % d->batch;
  const skv_decode_layer& Ly = d->layers[blockIdx.x / d->batch];
  const int L = d->tok_lens[b];
  if (L <= 0) return;
  const int64_t p = L - 1;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  if (wave == 3) {
    const int row_chunks = d->latent >> 3;  // 16-byte chunks of a bf16 row
    const u32x4* src = static_cast<const u32x4*>(Ly.kv_new) + static_cast<int64_t>(b) * row_chunks;
    u32x4* dst = static_cast<u32x4*>(Ly.ring) + (static_cast<int64_t>(b) * d->window + p % d->window) * row_chunks;
    for (int c = tid - 3 * kWave; c < row_chunks; c += kWave) dst[c] = src[c];
    return;
  }
  if (Ly.kind == SKV_LAYER_SWA) return;
  const skv_page_group& G = d->groups[Ly.group];
  if (wave < 2) {
    const int fp8_main = (Ly.format == SKV_FMT_FP8) ? d->latent - SKV_FP8_ROPE_DIMS : 0;
    decode_fold_part(G, b, p, Ly.pool, Ly.entry_bytes, Ly.state, Ly.bias, Ly.c_new, Ly.z_new, d->latent,
                     Ly.format, fp8_main, tid, 2 * kWave);
  } else if (Ly.kind == SKV_LAYER_CSA && Ly.idx_pool) {
    decode_fold_part(G, b, p, Ly.idx_pool, static_cast<int64_t>(d->c_indexer) * 2, Ly.idx_state,
                     Ly.idx_bias, Ly.ci_new, Ly.zi_new, d->c_indexer, SKV_FMT_BF16, 0, tid - 2 * kWave,
                     kWave);
  }
}

// ---------------------------------------------------------------------------
// Row copies shared by the gather tiles and the top-k rank step.  Row kinds:
// 0 skip, 1 copy a bf16 row, 2 dequantize an fp8 entry to bf16, 3 zero row.
// ---------------------------------------------------------------------------
// 16 fp8 e4m3fn codes times their block scale -> 16 bf16 (two 16-byte chunks).
__device__ __forceinline__ void dequant_codes(const u32x4 codes, float scale, u32x4& o0, u32x4& o1) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float f[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) f[h] = e4m3fn_to_f32(static_cast<uint8_t>(codes[q] >> (8 * h))) * scale;
    const uint32_t lo = f32_to_bf16(f[0]) | (static_cast<uint32_t>(f32_to_bf16(f[1])) << 16);
    const uint32_t hi = f32_to_bf16(f[2]) | (static_cast<uint32_t>(f32_to_bf16(f[3])) << 16);
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

// Copies rows [0, n) with all kThreads threads; row(r) gives row r's RowRef.
// Each thread issues kUnroll loads before its stores.  The loads are
// unconditional (a lane with nothing to load reads 16 bytes at `safe`, any
// readable device address, and drops them): a load under a branch is waited
// for before the branch joins, which would serialize the memory round trips.
// `fp8` says whether any row may be of kind 2 (uniform over the workgroup).
template <int kThreads, int kUnroll, class RowFn>
__device__ __forceinline__ void copy_rows(int n, RowFn row, int latent, bool fp8, const void* safe) {
  const u32x4* safe4 = static_cast<const u32x4*>(safe);
  const int bf_chunks = latent >> 3;  // 16-byte chunks of an output row
  const int total = n * bf_chunks;
  for (int t0 = threadIdx.x; t0 < total; t0 += kThreads * kUnroll) {
    u32x4 v[kUnroll];
    RowRef rf[kUnroll];
    int c[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int t = t0 + u * kThreads;
      const int tt = (t < total) ? t : 0;
      const int rr = tt / bf_chunks;
      c[u] = tt - rr * bf_chunks;
      rf[u] = row(rr);
      if (t >= total) rf[u].kind = 0;
      const u32x4* p = (rf[u].kind == 1) ? reinterpret_cast<const u32x4*>(rf[u].src) + c[u] : safe4;
      v[u] = ld_stream(p);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (rf[u].kind == 1) st_stream(reinterpret_cast<u32x4*>(rf[u].dst) + c[u], v[u]);
      if (rf[u].kind == 3) st_stream(reinterpret_cast<u32x4*>(rf[u].dst) + c[u], u32x4{0u, 0u, 0u, 0u});
    }
  }
  if (!fp8) return;
  const int fp8_main = latent - SKV_FP8_ROPE_DIMS;
  const int code_chunks = fp8_main >> 4;  // 16 codes -> 2 output chunks
  const int fp8_tasks = code_chunks + (SKV_FP8_ROPE_DIMS >> 3);
  const int ftotal = n * fp8_tasks;
  for (int t0 = threadIdx.x; t0 < ftotal; t0 += kThreads * kUnroll) {
    u32x4 v[kUnroll];
    float scale[kUnroll];
    RowRef rf[kUnroll];
    int c[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int t = t0 + u * kThreads;
      const int tt = (t < ftotal) ? t : 0;
      const int rr = tt / fp8_tasks;
      c[u] = tt - rr * fp8_tasks;
      rf[u] = row(rr);
      if (t >= ftotal) rf[u].kind = 0;
      const bool is_code = c[u] < code_chunks;
      const uint8_t* codes = is_code ? rf[u].src + c[u] * 16
                                     : rf[u].src + fp8_main + (fp8_main >> 7) * 4 + (c[u] - code_chunks) * 16;
      const uint8_t* sc = rf[u].src + fp8_main + (c[u] >> 3) * 4;
      const bool live = rf[u].kind == 2;
      v[u] = *(live ? reinterpret_cast<const u32x4*>(codes) : safe4);
      scale[u] = *(live && is_code ? reinterpret_cast<const float*>(sc) : reinterpret_cast<const float*>(safe4));
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (rf[u].kind != 2) continue;
      u32x4* o = reinterpret_cast<u32x4*>(rf[u].dst);
      if (c[u] < code_chunks) {
        u32x4 o0, o1;
        dequant_codes(v[u], scale[u], o0, o1);
        st_stream(o + 2 * c[u], o0);
        st_stream(o + 2 * c[u] + 1, o1);
      } else {
        st_stream(o + (fp8_main >> 3) + (c[u] - code_chunks), v[u]);
      }
    }
  }
}

// Source of compressed entry e of sequence b: the row kind (1 bf16, 2 fp8)
// and its address, or 0 when e is past n_ent or its page is not mapped.
__device__ __forceinline__ int entry_source(const skv_page_group& G, const skv_decode_layer& Ly, int b, int e,
                                            int n_ent, const uint8_t** src) {
  if (e < 0 || e >= n_ent) return 0;
  const int64_t pi = e / G.block_size;
  const int32_t page = (pi < G.bt_stride) ? G.block_table[b * G.bt_stride + pi] : -1;
  if (page < 0 || page >= G.n_pages) return 0;
  *src = static_cast<const uint8_t*>(Ly.pool) +
         (static_cast<int64_t>(page) * G.block_size + e % G.block_size) * Ly.entry_bytes;
  return (Ly.format == SKV_FMT_FP8) ? 2 : 1;
}

// ---------------------------------------------------------------------------
// 3. filter launch, 256-thread workgroups:
//    blocks [0, chunks*batch*csa)  : top-k filter chunks (skv_topk.h);
//    then gather tiles             : kGatherRowsD rows of a layer's dense rows
//                                    [HCA entries (out_rows) | window].
// ---------------------------------------------------------------------------
struct GatherTileSmem {
  const uint8_t* src_row[kGatherRowsD];
  uint8_t* dst_row[kGatherRowsD];
  int row_kind[kGatherRowsD];
};

union FilterLaunchSmem {
  TopkFilterSmem filter;
  GatherTileSmem tile;
};

__device__ __forceinline__ int dense_rows(const skv_decode_desc* d, const skv_decode_layer& Ly) {
  return d->window + (Ly.kind == SKV_LAYER_HCA ? static_cast<int>(Ly.out_rows) : 0);
}

__device__ __forceinline__ void gather_tile(GatherTileSmem& sm, const skv_decode_desc* d,
                                            const skv_decode_layer& Ly, int b, int tile) {
  const int latent = d->latent;
  const int64_t out_row = static_cast<int64_t>(latent) * 2;
  const int L = d->tok_lens[b];
  const int n_dense = (Ly.kind == SKV_LAYER_HCA) ? static_cast<int>(Ly.out_rows) : 0;
  const int n_rows = n_dense + d->window;
  const int r0 = tile * kGatherRowsD;
  if (threadIdx.x < kGatherRowsD) {
    const int r = r0 + threadIdx.x;
    int kind = 0;
    const uint8_t* s = nullptr;
    uint8_t* o = nullptr;
    if (r < n_dense) {
      // dense HCA rows past the entries stay untouched
      const skv_page_group& G = d->groups[Ly.group];
      kind = entry_source(G, Ly, b, r, G.n_entries[b], &s);
      o = static_cast<uint8_t*>(Ly.out_entries) + (static_cast<int64_t>(b) * Ly.out_rows + r) * out_row;
    } else if (r < n_rows) {
      const int w = r - n_dense;
      const int cnt = min(max(L, 0), d->window);
      if (w < cnt) {
        const int64_t slot = (static_cast<int64_t>(L) - cnt + w) % d->window;
        s = static_cast<const uint8_t*>(Ly.ring) + (static_cast<int64_t>(b) * d->window + slot) * out_row;
        o = static_cast<uint8_t*>(Ly.out_window) + (static_cast<int64_t>(b) * d->window + w) * out_row;
        kind = 1;
      }
    }
    sm.src_row[threadIdx.x] = s;
    sm.dst_row[threadIdx.x] = o;
    sm.row_kind[threadIdx.x] = kind;
  }
  __syncthreads();
  copy_rows<kGatherThreadsD, 4>(
      kGatherRowsD, [&](int r) { return RowRef{sm.src_row[r], sm.dst_row[r], sm.row_kind[r]}; }, latent,
      Ly.format == SKV_FMT_FP8 && Ly.kind == SKV_LAYER_HCA, d);
}

__global__ __launch_bounds__(kTkPartThreads) void k_decode_filter(const skv_decode_desc* __restrict__ d,
                                                                  int n_chunks, int n_csa) {
  static_assert(kTkPartThreads == kGatherThreadsD, "filter and gather tiles share the launch");
  __shared__ FilterLaunchSmem sm;
  if (*d->status) return;  // refused step
  const int batch = d->batch;
  int u = blockIdx.x;
  const int n_filter = n_chunks * batch * n_csa;
  if (u < n_filter) {
    const int chunk = u % n_chunks;
    u /= n_chunks;
    const int b = u % batch;
    const skv_decode_layer* Ly = csa_layer(d, u / batch);
    if (!Ly) return;  // uniform over the workgroup
    const int m = d->groups[Ly->group].m;
    const int L = d->tok_lens[b];
    topk_filter_chunk(sm.filter, Ly->scores + static_cast<int64_t>(b) * Ly->score_stride, L / m,
                      L > 0 ? (L - 1) / m : 0, Ly->top_k, chunk,
                      Ly->topk_ws + static_cast<int64_t>(b) * kTkWsWords);
    return;
  }
  u -= n_filter;
  for (int l = 0; l < d->n_layers; ++l) {
    const skv_decode_layer& Ly = d->layers[l];
    const int tiles = static_cast<int>(ceil_div(dense_rows(d, Ly), kGatherRowsD));
    if (u < tiles * batch) {
      gather_tile(sm.tile, d, Ly, u / tiles, u % tiles);
      return;
    }
    u -= tiles * batch;
  }
}

// ---------------------------------------------------------------------------
// 4. top-k rank + sparse gather: grid (parts, batch, CSA layers), part p of a
//    row owns output positions [p*rank_out, (p+1)*rank_out), rank_out 16 or
//    32 (the host picks 16 when the rows alone give few workgroups).
//    Every part loads the row's candidate lists as 64-bit order keys
//    (key << 32 | ~index: larger means earlier in the output), ranks the sure
//    candidates p, p + parts, ... among the sure list and the tie candidates
//    p, p + parts, ... among the tie list (kRankSub lanes per candidate, each
//    counting a strided share of the list), and writes each winner's index
//    and entry at its output position; positions in [sel, top_k) it owns get
//    index -1 and entry 0 (the reference's clamp(min=0) before its gather).
//    On a tie bin too large for the lists every part runs the full select.
//    Part 0 zeroes the row's histogram for the next step; the counters are
//    zeroed by the next step's histogram launch.
// ---------------------------------------------------------------------------
constexpr int kRankThreads = 256;
constexpr int kRankOutMin = 16;  // output positions per part: 16 or 32, chosen per launch
constexpr int kRankOut = 32;
constexpr int kRankSub = 8;
constexpr int kRankCands = kRankThreads / kRankSub;  // candidates ranked per round
constexpr int kRankMaxRows = 512;  // rows one part can collect (checked below)

struct RankSmem {
  int cnt[3];  // n_sure, n_tie, tie-overflow flag
  int n_rows;
  int2 win[kRankMaxRows];         // (output position, pick)
  uintptr_t src_kind[kRankMaxRows];  // entry address | row kind (entries are 4-byte aligned)
  union {
    uint64_t ck[kTkCand];
    struct {
      TopkSmemT<kRankThreads> full;
      int32_t order[kMaxTopK];
    } f;
  } u;
};

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

__global__ __launch_bounds__(kRankThreads) void k_decode_topk_rank(const skv_decode_desc* __restrict__ d,
                                                                    int rank_out) {
  __shared__ RankSmem sm;
  if (*d->status) return;  // refused step
  const skv_decode_layer* Lp = csa_layer(d, blockIdx.z);
  if (!Lp) return;
  const skv_decode_layer& Ly = *Lp;
  const int k = Ly.top_k;
  const int parts = static_cast<int>(ceil_div(k, rank_out));
  const int part = blockIdx.x;
  if (part >= parts) return;  // the grid is sized for the largest top_k
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const skv_page_group& G = d->groups[Ly.group];
  const int L = d->tok_lens[b];
  const int n_cols = L / G.m;
  const int n_valid = L > 0 ? (L - 1) / G.m : 0;
  const int sel = topk_sel(k, n_cols, n_valid);
  int32_t* ws = Ly.topk_ws + static_cast<int64_t>(b) * kTkWsWords;
  if (part == 0) {
    for (int i = tid; i < kTkBins; i += kRankThreads) ws[kTkWsHist + i] = 0;
  }
  if (tid < 3) sm.cnt[tid] = ws[kTkWsCnt + tid];
  if (tid == 0) sm.n_rows = 0;
  __syncthreads();
  const int o0 = part * rank_out;
  const int o1 = min(k, o0 + rank_out);
  const int f0 = max(o0, sel);  // positions [f0, o1) are fills
  int n_rows;
  if (sel > 0 && sm.cnt[2]) {
    // tie bin over the list capacity: full select of the row, then this part's positions
    topk_row<kRankThreads>(sm.u.f.full, nullptr, Ly.scores + static_cast<int64_t>(b) * Ly.score_stride,
                           n_cols, n_valid, k, sm.u.f.order);
    __syncthreads();
    if (tid < o1 - o0) sm.win[tid] = make_int2(o0 + tid, sm.u.f.order[o0 + tid]);
    n_rows = o1 - o0;
  } else {
    if (sel > 0) {
      const int S = min(sm.cnt[0], kMaxTopK);
      const int C = S + min(sm.cnt[1], kTkTieCap);
      const int2* sure_list = reinterpret_cast<const int2*>(ws + kTkWsSure);
      const int2* tie_list = reinterpret_cast<const int2*>(ws + kTkWsTie);
      constexpr int kLoad = 8;  // list loads in flight per thread
      for (int c0 = tid; c0 < C; c0 += kRankThreads * kLoad) {
        int2 v[kLoad];
#pragma unroll
        for (int u = 0; u < kLoad; ++u) {
          const int c = min(c0 + u * kRankThreads, C - 1);  // unconditional: C >= sel > 0
          v[u] = (c < S ? sure_list : tie_list - S)[c];
        }
#pragma unroll
        for (int u = 0; u < kLoad; ++u) {
          const int c = c0 + u * kRankThreads;
          if (c < C) {
            sm.u.ck[c] = (static_cast<uint64_t>(static_cast<uint32_t>(v[u].x)) << 32) |
                         static_cast<uint32_t>(~v[u].y);
          }
        }
      }
      __syncthreads();
      const int sub = tid % kRankSub;
#pragma unroll 1
      for (int cls = 0; cls < 2; ++cls) {
        const int lo = cls ? S : 0;
        const int hi = cls ? C : S;
        const int n_mine = (part < hi - lo) ? static_cast<int>(ceil_div(hi - lo - part, parts)) : 0;
        for (int j0 = 0; j0 < n_mine; j0 += kRankCands) {
          const int j = j0 + tid / kRankSub;
          const bool valid = j < n_mine;
          const uint64_t mine = valid ? sm.u.ck[lo + part + j * parts] : ~0ull;
          int rank = 0;
#pragma unroll 8
          for (int q = lo + sub; q < hi; q += kRankSub) rank += sm.u.ck[q] > mine;
          rank += __shfl_xor(rank, 1);
          rank += __shfl_xor(rank, 2);
          rank += __shfl_xor(rank, 4);
          const int pos = lo + rank;
          if (valid && sub == 0 && pos < sel) {
            const uint32_t key = static_cast<uint32_t>(mine >> 32);
            const int idx = static_cast<int>(~static_cast<uint32_t>(mine));
            sm.win[atomicAdd(&sm.n_rows, 1)] = make_int2(pos, key_finite(key) ? idx : -1);
          }
        }
      }
    }
    __syncthreads();
    n_rows = sm.n_rows;
    if (tid < o1 - f0) sm.win[n_rows + tid] = make_int2(f0 + tid, -1);
    n_rows += max(0, o1 - f0);
  }
  __syncthreads();
  // indices out, entry sources, then one copy pass over every row
  const int n_ent = G.n_entries[b];
  const int64_t out_row = static_cast<int64_t>(d->latent) * 2;
  int32_t* out_idx = Ly.topk_idx + static_cast<int64_t>(b) * k;
  uint8_t* out_base = static_cast<uint8_t*>(Ly.out_entries) + static_cast<int64_t>(b) * k * out_row;
  for (int w = tid; w < n_rows; w += kRankThreads) {
    const int2 pw = sm.win[w];
    out_idx[pw.x] = pw.y;
    const uint8_t* s = nullptr;
    int kind = entry_source(G, Ly, b, pw.y < 0 ? 0 : pw.y, n_ent, &s);
    sm.src_kind[w] = reinterpret_cast<uintptr_t>(s) | static_cast<uintptr_t>(kind ? kind : 3);
  }
  __syncthreads();
  copy_rows<kRankThreads, 16>(
      n_rows,
      [&](int r) {
        const uintptr_t sk = sm.src_kind[r];
        return RowRef{reinterpret_cast<const uint8_t*>(sk & ~static_cast<uintptr_t>(3)),
                      out_base + sm.win[r].x * out_row, static_cast<int>(sk & 3)};
      },
      d->latent, Ly.format == SKV_FMT_FP8, d);
}

}  // namespace skv

using namespace skv;

extern "C" int skv_decode_desc_sizes(int64_t* out) {
  if (!out) return set_error(SKV_EINVAL, "skv_decode_desc_sizes: out is NULL");
  out[0] = sizeof(skv_decode_desc);
  out[1] = sizeof(skv_decode_layer);
  out[2] = sizeof(skv_page_group);
  return SKV_OK;
}

extern "C" int skv_decode_step(const skv_decode_desc* h, const skv_decode_desc* dd, void* stream) {
  const char* what = "skv_decode_step";
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
  if (!h->tok_lens || !h->status) return set_error(SKV_EINVAL, "%s: NULL tok_lens/status", what);
  for (int g = 0; g < h->n_groups; ++g) {
    const skv_page_group& G = h->groups[g];
    if (!G.free_stack || !G.free_top || !G.block_table || !G.n_entries || G.m <= 0 ||
        G.block_size <= 0 || G.bt_stride <= 0 || G.n_pages <= 0) {
      return set_error(SKV_EINVAL, "%s: page group %d is incomplete", what, g);
    }
  }
  int n_csa = 0, max_top_k = 0;
  int64_t max_score_cols = 1, n_tiles = 0;
  for (int l = 0; l < h->n_layers; ++l) {
    const skv_decode_layer& Ly = h->layers[l];
    if (!Ly.ring || !Ly.kv_new || !Ly.out_window) return set_error(SKV_EINVAL, "%s: layer %d lacks ring/kv_new/out_window", what, l);
    int64_t dense = h->window;
    if (Ly.kind == SKV_LAYER_HCA || Ly.kind == SKV_LAYER_CSA) {
      if (Ly.group < 0 || Ly.group >= h->n_groups) return set_error(SKV_EINVAL, "%s: layer %d group out of range", what, l);
      if (!Ly.pool || !Ly.state || !Ly.bias || !Ly.c_new || !Ly.z_new || !Ly.out_entries) {
        return set_error(SKV_EINVAL, "%s: layer %d lacks pool/state/bias/c/z/out", what, l);
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
        ++n_csa;
        max_top_k = max(max_top_k, Ly.top_k);
      } else {
        if (Ly.out_rows <= 0 || Ly.out_rows > (1 << 24)) {
          return set_error(SKV_EINVAL, "%s: HCA layer %d needs 0 < out_rows <= 2^24", what, l);
        }
        dense += Ly.out_rows;
      }
    } else if (Ly.kind != SKV_LAYER_SWA) {
      return set_error(SKV_EINVAL, "%s: layer %d has unknown kind %d", what, l, Ly.kind);
    }
    n_tiles += ceil_div(dense, kGatherRowsD) * h->batch;
  }
  if (h->batch == 0 || h->n_layers == 0) return SKV_OK;
  const int n_chunks = static_cast<int>(ceil_div(max_score_cols, kTkChunk));
  const int64_t n_append = static_cast<int64_t>(h->batch) * h->n_layers +
                           static_cast<int64_t>(n_chunks) * h->batch * n_csa;
  const int64_t n_filter = static_cast<int64_t>(n_chunks) * h->batch * n_csa + n_tiles;
  if (n_append > INT32_MAX || n_filter > INT32_MAX) {
    return set_error(SKV_EINVAL, "%s: score_stride/out_rows give a grid over 2^31 workgroups", what);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_decode_plan, dim3(1), dim3(kPlanThreads), 0, s, dd);
  int rc = check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(k_decode_append, dim3(static_cast<unsigned>(n_append)), dim3(kAppendThreads), 0, s,
                     dd, n_chunks);
  if ((rc = check_launch(what))) return rc;
  hipLaunchKernelGGL(k_decode_filter, dim3(static_cast<unsigned>(n_filter)), dim3(kTkPartThreads), 0, s,
                     dd, n_chunks, n_csa);
  if ((rc = check_launch(what))) return rc;
  if (n_csa > 0) {
    // smaller parts when the rows alone would leave most CUs idle
    const int rank_out = (static_cast<int64_t>(h->batch) * n_csa * ceil_div(max_top_k, kRankOut) < 512)
                             ? kRankOutMin : kRankOut;
    const dim3 rgrid(static_cast<unsigned>(ceil_div(max_top_k, rank_out)), h->batch, n_csa);
    hipLaunchKernelGGL(k_decode_topk_rank, rgrid, dim3(kRankThreads), 0, s, dd, rank_out);
  }
  return check_launch(what);
}
