// Fused decode step over a stack of heterogeneous layers: four launches per
// step whatever the number of layers (plan, append/compress, top-k, gather).
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
constexpr int kGatherRowsD = 8;

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
  const int n_append = d->batch * d->n_layers;
  if (static_cast<int>(blockIdx.x) >= n_append) {
    // top-k histogram chunk (chunk, b, csa layer)
    int u = blockIdx.x - n_append;
    const int chunk = u % n_chunks;
    u /= n_chunks;
    const int b = u % d->batch;
    const skv_decode_layer* Ly = csa_layer(d, u / d->batch);
    if (!Ly) return;
    const int m = d->groups[Ly->group].m;
    const int L = d->tok_lens[b];
    topk_hist_chunk(hsm, Ly->scores + static_cast<int64_t>(b) * Ly->score_stride, L / m,
                    L > 0 ? (L - 1) / m : 0, Ly->top_k, chunk,
                    Ly->topk_ws + static_cast<int64_t>(b) * kTkWsWords);
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
// 3. top-k filter (grid chunks, batch, CSA layers) and final (grid batch, CSA
//    layers); see skv_topk.h.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kTkPartThreads) void k_decode_topk_filter(const skv_decode_desc* __restrict__ d) {
  __shared__ TopkFilterSmem sm;
  const skv_decode_layer* Ly = csa_layer(d, blockIdx.z);
  if (!Ly) return;  // uniform over the workgroup
  const int b = blockIdx.y;
  const int m = d->groups[Ly->group].m;
  const int L = d->tok_lens[b];
  topk_filter_chunk(sm, Ly->scores + static_cast<int64_t>(b) * Ly->score_stride, L / m,
                    L > 0 ? (L - 1) / m : 0, Ly->top_k, blockIdx.x,
                    Ly->topk_ws + static_cast<int64_t>(b) * kTkWsWords);
}

__global__ __launch_bounds__(kTopkThreads) void k_decode_topk_final(const skv_decode_desc* __restrict__ d) {
  __shared__ TopkFinalSmem sm;
  const skv_decode_layer* Ly = csa_layer(d, blockIdx.y);
  if (!Ly) return;
  const int b = blockIdx.x;
  const int m = d->groups[Ly->group].m;
  const int L = d->tok_lens[b];
  topk_final_row(sm, Ly->scores + static_cast<int64_t>(b) * Ly->score_stride, L / m,
                 L > 0 ? (L - 1) / m : 0, Ly->top_k, Ly->topk_ws + static_cast<int64_t>(b) * kTkWsWords,
                 Ly->topk_idx + static_cast<int64_t>(b) * Ly->top_k);
}

// ---------------------------------------------------------------------------
// 4. gather: grid (tiles, batch, layers); a tile is 8 output rows of the
//    layer's row space [entries (top_k or out_rows) | window].
// ---------------------------------------------------------------------------
__device__ __forceinline__ void dequant_chunk(const uint8_t* entry, int fp8_main, int c, u32x4& o0, u32x4& o1) {
  const u32x4 codes = *(reinterpret_cast<const u32x4*>(entry) + c);
  const float scale = *reinterpret_cast<const float*>(entry + fp8_main + (c >> 3) * 4);
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

__global__ __launch_bounds__(kGatherThreadsD) void k_decode_gather(const skv_decode_desc* __restrict__ d) {
  __shared__ const uint8_t* src_row[kGatherRowsD];
  __shared__ uint8_t* dst_row[kGatherRowsD];
  __shared__ int row_kind[kGatherRowsD];  // 0 skip, 1 copy bf16 row, 2 dequant fp8 entry, 3 zero row
  const int b = blockIdx.y;
  const skv_decode_layer& Ly = d->layers[blockIdx.z];
  const int latent = d->latent;
  const int64_t out_row = static_cast<int64_t>(latent) * 2;
  const int L = d->tok_lens[b];
  int n_entry_rows = 0;
  if (Ly.kind == SKV_LAYER_CSA) n_entry_rows = Ly.top_k;
  else if (Ly.kind == SKV_LAYER_HCA) n_entry_rows = static_cast<int>(Ly.out_rows);
  const int n_rows = n_entry_rows + d->window;
  const int r0 = blockIdx.x * kGatherRowsD;
  if (r0 >= n_rows) return;
  if (threadIdx.x < kGatherRowsD) {
    const int r = r0 + threadIdx.x;
    int kind = 0;
    const uint8_t* s = nullptr;
    uint8_t* o = nullptr;
    if (r < n_entry_rows) {
      const skv_page_group& G = d->groups[Ly.group];
      const int n_ent = G.n_entries[b];
      int e;
      if (Ly.kind == SKV_LAYER_CSA) {
        e = Ly.topk_idx[static_cast<int64_t>(b) * Ly.top_k + r];
        if (e < 0) e = 0;  // clamp(min=0): a -1 pick reads entry 0
        o = static_cast<uint8_t*>(Ly.out_entries) + (static_cast<int64_t>(b) * Ly.top_k + r) * out_row;
        kind = 3;
      } else {
        e = r;
        o = static_cast<uint8_t*>(Ly.out_entries) + (static_cast<int64_t>(b) * Ly.out_rows + r) * out_row;
        kind = 0;  // dense rows past the entries stay untouched
      }
      if (e < n_ent) {
        const int64_t pi = e / G.block_size;
        const int32_t page = (pi < G.bt_stride) ? G.block_table[b * G.bt_stride + pi] : -1;
        if (page >= 0 && page < G.n_pages) {
          s = static_cast<const uint8_t*>(Ly.pool) +
              (static_cast<int64_t>(page) * G.block_size + e % G.block_size) * Ly.entry_bytes;
          kind = (Ly.format == SKV_FMT_FP8) ? 2 : 1;
        }
      }
    } else if (r < n_rows) {
      const int w = r - n_entry_rows;
      const int cnt = min(max(L, 0), d->window);
      if (w < cnt) {
        const int64_t slot = (static_cast<int64_t>(L) - cnt + w) % d->window;
        s = static_cast<const uint8_t*>(Ly.ring) + (static_cast<int64_t>(b) * d->window + slot) * out_row;
        o = static_cast<uint8_t*>(Ly.out_window) + (static_cast<int64_t>(b) * d->window + w) * out_row;
        kind = 1;
      }
    }
    src_row[threadIdx.x] = s;
    dst_row[threadIdx.x] = o;
    row_kind[threadIdx.x] = kind;
  }
  __syncthreads();
  const int bf_chunks = latent >> 3;                 // 16-byte chunks of an output row
  const int fp8_main = latent - SKV_FP8_ROPE_DIMS;
  const int code_chunks = fp8_main >> 4;             // 16 codes -> 2 output chunks
  const int rope_chunks = SKV_FP8_ROPE_DIMS >> 3;
  const int fp8_tasks = code_chunks + rope_chunks;
  // bf16 copies and zero rows: one task per output chunk
  for (int t = threadIdx.x; t < kGatherRowsD * bf_chunks; t += kGatherThreadsD) {
    const int rr = t / bf_chunks;
    const int c = t - rr * bf_chunks;
    const int kind = row_kind[rr];
    if (kind == 1) {
      st_stream(reinterpret_cast<u32x4*>(dst_row[rr]) + c, *(reinterpret_cast<const u32x4*>(src_row[rr]) + c));
    } else if (kind == 3) {
      st_stream(reinterpret_cast<u32x4*>(dst_row[rr]) + c, u32x4{0u, 0u, 0u, 0u});
    }
  }
  // fp8 entries: one task per 16 codes (two output chunks) or per rope chunk
  for (int t = threadIdx.x; t < kGatherRowsD * fp8_tasks; t += kGatherThreadsD) {
    const int rr = t / fp8_tasks;
    if (row_kind[rr] != 2) continue;
    const int c = t - rr * fp8_tasks;
    const uint8_t* s = src_row[rr];
    u32x4* o = reinterpret_cast<u32x4*>(dst_row[rr]);
    if (c < code_chunks) {
      u32x4 o0, o1;
      dequant_chunk(s, fp8_main, c, o0, o1);
      st_stream(o + 2 * c, o0);
      st_stream(o + 2 * c + 1, o1);
    } else {
      const int rc = c - code_chunks;
      st_stream(o + (fp8_main >> 3) + rc,
                *reinterpret_cast<const u32x4*>(s + fp8_main + (fp8_main >> 7) * 4 + rc * 16));
    }
  }
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
  int n_csa = 0, max_rows = 0;
  int64_t max_score_cols = 1;
  for (int l = 0; l < h->n_layers; ++l) {
    const skv_decode_layer& Ly = h->layers[l];
    if (!Ly.ring || !Ly.kv_new || !Ly.out_window) return set_error(SKV_EINVAL, "%s: layer %d lacks ring/kv_new/out_window", what, l);
    int rows = h->window;
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
        rows += Ly.top_k;
      } else {
        if (Ly.out_rows <= 0) return set_error(SKV_EINVAL, "%s: HCA layer %d needs out_rows > 0", what, l);
        rows += static_cast<int>(Ly.out_rows);
      }
    } else if (Ly.kind != SKV_LAYER_SWA) {
      return set_error(SKV_EINVAL, "%s: layer %d has unknown kind %d", what, l, Ly.kind);
    }
    max_rows = max(max_rows, rows);
  }
  if (h->batch == 0 || h->n_layers == 0) return SKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_decode_plan, dim3(1), dim3(kPlanThreads), 0, s, dd);
  int rc = check_launch(what);
  if (rc) return rc;
  const int n_chunks = static_cast<int>(ceil_div(max_score_cols, kTkChunk));
  const int64_t n_blocks = static_cast<int64_t>(h->batch) * h->n_layers +
                           static_cast<int64_t>(n_chunks) * h->batch * n_csa;
  hipLaunchKernelGGL(k_decode_append, dim3(static_cast<unsigned>(n_blocks)), dim3(kAppendThreads), 0, s,
                     dd, n_chunks);
  if ((rc = check_launch(what))) return rc;
  if (n_csa > 0) {
    hipLaunchKernelGGL(k_decode_topk_filter, dim3(n_chunks, h->batch, n_csa), dim3(kTkPartThreads), 0, s, dd);
    if ((rc = check_launch(what))) return rc;
    hipLaunchKernelGGL(k_decode_topk_final, dim3(h->batch, n_csa), dim3(kTopkThreads), 0, s, dd);
    if ((rc = check_launch(what))) return rc;
  }
  const dim3 ggrid(static_cast<unsigned>(ceil_div(max_rows, kGatherRowsD)), h->batch, h->n_layers);
  hipLaunchKernelGGL(k_decode_gather, ggrid, dim3(kGatherThreadsD), 0, s, dd);
  return check_launch(what);
}
