/*
 * saintkv.h — C ABI of the MI355X (gfx950) heterogeneous KV-cache library.
 *
 * Plain C: raw device pointers, int64 sizes, a hipStream_t (passed as void*).
 * Every entry point returns 0 on success or a negative SKV_E* code; the text
 * of the last error on the calling thread is available from skv_last_error().
 * The library allocates nothing: every buffer is owned by the caller (the
 * one static device array is the unit table of
 * skv_decode_append_gather_noalloc, 2 MiB per GPU).
 *
 * Page-indexed entry points take n_pages: a block-table entry outside
 * [0, n_pages) is treated as unmapped and never dereferenced.
 *
 * Storage model (all device memory):
 *   pool         n_pages pages; page p holds block_size rows of row_bytes
 *                bytes at pool + p*block_size*row_bytes.  row_bytes is a
 *                multiple of 16.  One row = one token (raw KV) or one
 *                compressed entry.
 *   block_table  int32 [batch, bt_stride]; entry (b, j) = physical page of
 *                logical page j of sequence b (-1 when unmapped).
 *   seq_lens     int32 [batch]; rows held by each sequence.
 *   free_stack   int32 [n_pages] + free_top int32[1]: a LIFO stack of free
 *                page ids; a pop returns free_stack[free_top-1].
 *
 * The reference keeps contiguous per-layer tensors with a single host cursor
 * (packages/inference/src/saint_llm_inference/kv_cache.py:59-83); this ABI is
 * the paged, ragged replacement for the tensor ops those classes perform.
 */
#ifndef SAINTKV_H_
#define SAINTKV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SKV_ABI_VERSION 1

/* Status codes.  SKV_EINVAL maps to Python ValueError, the rest to
 * RuntimeError (the exception types of kv_cache.py:54-55, 69-79). */
#define SKV_OK 0
#define SKV_EINVAL (-1)     /* bad argument (shape, size, alignment)        */
#define SKV_EOVERFLOW (-2)  /* append past a sequence's capacity            */
#define SKV_ENOSPC (-3)     /* page pool exhausted                          */
#define SKV_EHIP (-4)       /* HIP runtime error (launch / memcpy)          */
#define SKV_ESTATE (-5)     /* illegal state transition (double free, sink) */

/* Entry formats of compressed caches. */
#define SKV_FMT_BF16 0 /* entry = channels bf16 values (2*channels bytes) */
#define SKV_FMT_FP8 1  /* entry = e4m3fn codes of the main dims, one fp32 scale
                        * per 128 main dims, then SKV_FP8_ROPE_DIMS bf16 dims */
#define SKV_FMT_F32 2  /* entry = channels fp32 values (4*channels bytes), with fp32
                        * c/z rows: skv_compress_append only (fp32 caches) */
#define SKV_FMT_IN_F32 0x100 /* or'd into skv_compress_append's format: the c/z rows
                              * are fp32 (pooled unrounded) for bf16 or fp8 entries */
#define SKV_FP8_ROPE_DIMS 64
#define SKV_FP8_ENTRY_BYTES(channels) \
  (((channels) - SKV_FP8_ROPE_DIMS) + ((channels) - SKV_FP8_ROPE_DIMS) / 128 * 4 + 2 * SKV_FP8_ROPE_DIMS)

/* Device-side status words written by kernels that can refuse work
 * (bit flags, 0 = success). */
#define SKV_STATUS_MAX_PAGES 1 /* a sequence would exceed bt_stride pages   */
#define SKV_STATUS_NOSPC 2     /* not enough free pages                     */
#define SKV_STATUS_BADARG 4    /* negative count                            */
#define SKV_STATUS_STACK 8     /* release would overfill the free stack     */
#define SKV_STATUS_UNITS 16    /* page-unit table too small                 */

/* ABI version tag (SKV_ABI_VERSION) and the last error on this thread. */
int skv_abi_version(void);
const char* skv_last_error(void);

/* ---- free list ---------------------------------------------------------
 * Initialise the free stack.  order == NULL: free_stack[i] = n_pages-1-i so
 * pops return 0,1,2,...; otherwise order[0..n_pages) is a device array whose
 * element i is the i-th page to be popped.  free_top = n_pages.
 * No reference counterpart: block tables and the free list exist only as a
 * plan in the reference (saint_llm_inference/__init__.py:5-9). */
int skv_free_stack_init(int32_t* free_stack, int32_t* free_top, const int32_t* order,
                        int64_t n_pages, void* stream);

/* Reserve pages so that sequence b can hold seq_lens[b] + n_new[b] rows, then
 * advance seq_lens[b] by n_new[b] (n_new == NULL: n_new_uniform for all).
 * Pages are popped in ascending b, and within b in logical-page order.
 * All-or-nothing: if any sequence would exceed max_pages or the pool lacks
 * pages, nothing is written and *status receives SKV_STATUS_* bits (status
 * may be NULL).  Replaces the cursor advance + capacity check of
 * kv_cache.py:74-82.  batch <= 4096 (all batched entry points). */
int skv_reserve(int32_t* free_stack, int32_t* free_top, int64_t n_pages, int32_t* block_table,
                int64_t bt_stride, int64_t max_pages, int32_t* seq_lens, const int32_t* n_new,
                int32_t n_new_uniform, int64_t batch, int64_t block_size, int32_t* status,
                void* stream);

/* ---- paged append / gather ---------------------------------------------
 * skv_paged_append: write the n_new[b] newest rows of each sequence (rows
 * [seq_lens[b]-n_new[b], seq_lens[b]); seq_lens already advanced by
 * skv_reserve) from src into the pool.  Source row i of sequence b is at
 * src + b*src_seq_stride + i*src_row_stride (bytes); rows i >= src_len are
 * never read.  Replaces self.k[:, L:L+n] = k_new (kv_cache.py:80-81). */
int skv_paged_append(void* pool, int64_t row_bytes, int64_t block_size, int64_t n_pages,
                     const int32_t* block_table, int64_t bt_stride, const int32_t* seq_lens,
                     const int32_t* n_new, int32_t n_new_uniform, const void* src,
                     int64_t src_seq_stride, int64_t src_row_stride, int64_t src_len,
                     int64_t batch, void* stream);

/* skv_paged_gather: copy rows [0, seq_lens[b]) of every sequence, in order,
 * into dst.  Row r of sequence b lands at dst row dst_row_offsets[b] + r
 * (dst_row_offsets == NULL: b*dst_seq_stride_rows); a page whose rows would
 * land at or past dst_capacity_rows is skipped.
 * Replaces the contiguous view self.k[:, :L] (kv_cache.py:83). */
int skv_paged_gather(void* dst, const int64_t* dst_row_offsets, int64_t dst_seq_stride_rows,
                     int64_t dst_capacity_rows, const void* pool, int64_t row_bytes,
                     int64_t block_size, int64_t n_pages, const int32_t* block_table,
                     int64_t bt_stride, const int32_t* seq_lens, int64_t batch, void* stream);

/* skv_append_gather: skv_paged_append + skv_paged_gather in one launch; new
 * rows go from src to both the pool and dst.  One decode step of
 * SWAKVCacheLayer.append (kv_cache.py:63-83) on paged storage. */
int skv_append_gather(void* dst, const int64_t* dst_row_offsets, int64_t dst_seq_stride_rows,
                      int64_t dst_capacity_rows, void* pool, int64_t row_bytes,
                      int64_t block_size, int64_t n_pages, const int32_t* block_table,
                      int64_t bt_stride, const int32_t* seq_lens, const int32_t* n_new,
                      int32_t n_new_uniform, const void* src, int64_t src_seq_stride,
                      int64_t src_row_stride, int64_t src_len, int64_t batch, void* stream);

/* skv_decode_append_gather: skv_reserve + skv_append_gather as one decode
 * step in two launches, the copy cut into 4 KB slices of page units (one
 * 256-thread workgroup per slice).  units: int32 workspace of
 * 8 + 8*max_units words where max_units >= sum over b of
 * ceil((seq_lens[b] + n_new[b]) / block_size); the launch covers max_units
 * units (pass the exact count when the host knows it).  On a refusal
 * (SKV_STATUS_* in *status, including SKV_STATUS_UNITS) nothing changes and
 * nothing is copied.  Same results as skv_reserve followed by
 * skv_append_gather (kv_cache.py:63-83 on paged storage). */
int skv_decode_append_gather(int32_t* free_stack, int32_t* free_top, int64_t n_pages,
                             int32_t* block_table, int64_t bt_stride, int32_t* seq_lens,
                             const int32_t* n_new, int32_t n_new_uniform, int32_t* status, void* dst,
                             const int64_t* dst_row_offsets, int64_t dst_seq_stride_rows,
                             int64_t dst_capacity_rows, void* pool, int64_t row_bytes,
                             int64_t block_size, const void* src, int64_t src_seq_stride,
                             int64_t src_row_stride, int64_t src_len, int32_t* units,
                             int64_t max_units, int64_t batch, void* stream);

/* The two launches of skv_decode_append_gather as separate calls:
 * skv_plan_units reserves the pages, advances seq_lens and writes the unit
 * table; skv_copy_slices performs the copy the table describes (new rows
 * [seq_lens-n_new, seq_lens) of each unit from src, the rest from the pool). */
int skv_plan_units(int32_t* free_stack, int32_t* free_top, int64_t n_pages, int32_t* block_table,
                   int64_t bt_stride, int32_t* seq_lens, const int32_t* n_new,
                   int32_t n_new_uniform, int32_t* status, const int64_t* dst_row_offsets,
                   int64_t dst_seq_stride_rows, int64_t block_size, int32_t* units,
                   int64_t max_units, int64_t batch, void* stream);
int skv_copy_slices(void* dst, int64_t dst_capacity_rows, void* pool, int64_t row_bytes,
                    int64_t block_size, int64_t n_pages, const void* src, int64_t src_seq_stride,
                    int64_t src_row_stride, int64_t src_len, const int32_t* units,
                    int64_t max_units, void* stream);

/* Allocation-free form of skv_decode_append_gather: the same two launches
 * and results, with the page-unit table in a static device array of
 * SKV_NOALLOC_MAX_UNITS units (2 MiB, one per GPU the library runs on, held
 * until the process ends) instead of the caller's `units` workspace.  It
 * calls no hipMalloc/hipFree and allocates nothing; max_units above
 * SKV_NOALLOC_MAX_UNITS is refused with SKV_EINVAL.  The stream must belong
 * to the calling thread's current device.  Every call on one GPU shares that
 * GPU's table, which keeps the last call's contents: calls that overlap on
 * one GPU (concurrent streams, or threads) race.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
#define SKV_NOALLOC_MAX_UNITS 65536
int skv_decode_append_gather_noalloc(int32_t* free_stack, int32_t* free_top, int64_t n_pages,
                                     int32_t* block_table, int64_t bt_stride, int32_t* seq_lens,
                                     const int32_t* n_new, int32_t n_new_uniform, int32_t* status,
                                     void* dst, const int64_t* dst_row_offsets,
                                     int64_t dst_seq_stride_rows, int64_t dst_capacity_rows,
                                     void* pool, int64_t row_bytes, int64_t block_size,
                                     const void* src, int64_t src_seq_stride,
                                     int64_t src_row_stride, int64_t src_len, int64_t max_units,
                                     int64_t batch, void* stream);

/* ---- SWA ring -------------------------------------------------------------
 * ring: [batch, window, row_bytes]; token at position p of sequence b lives
 * in slot p % window.  skv_ring_append writes the n_new[b] newest tokens
 * (positions [seq_lens[b]-n_new[b], seq_lens[b]); seq_lens already include
 * them); when n_new > window only the last window tokens are written.
 * skv_ring_read copies the last min(window, seq_lens[b]) tokens in position
 * order to dst row b*dst_seq_stride_rows + r.  Replaces the window mask over
 * the full history (swa.py:115-125, csa.py:352-360). */
int skv_ring_append(void* ring, int64_t window, int64_t row_bytes, const int32_t* seq_lens,
                    const int32_t* n_new, int32_t n_new_uniform, const void* src,
                    int64_t src_seq_stride, int64_t src_row_stride, int64_t src_len,
                    int64_t batch, void* stream);
int skv_ring_read(void* dst, int64_t dst_seq_stride_rows, int64_t dst_capacity_rows,
                  const void* ring, int64_t window, int64_t row_bytes, const int32_t* seq_lens,
                  int64_t batch, void* stream);

/* ---- compression ----------------------------------------------------------
 * Append n_new tokens' compressor projections (c, z: bf16 [batch, T, channels]
 * with byte strides in_seq_stride / in_row_stride, T = in_len) of sequences
 * whose token counts are now seq_lens.  Every block of m tokens completed by
 * this call is pooled, out[j] = sum_i softmax_i(z[i,j] + bias[i,j]) * c[i,j]
 * (bias fp32 [m, channels]; fp32 math, rounded to bf16), and written as entry
 * floor(p/m) of the paged compressed cache (format SKV_FMT_BF16 or
 * SKV_FMT_FP8, quantized on write).  With SKV_FMT_F32 the c/z rows are fp32
 * and the entries the unrounded fp32 results (fp32 caches); SKV_FMT_IN_F32
 * or'd into a bf16 or fp8 format takes fp32 c/z rows (an fp32 compressor
 * module feeding a bf16 cache: the entry is rounded once, as the
 * reference's copy into its cache rounds it).  The incomplete block is carried in
 * tail_state (fp32 [batch, 3, channels]: running max, sum of weights and
 * weighted sum of its tokens' online softmax), so a block split over several
 * calls pools to the same value as one call.  Pages for the new entries must
 * be reserved beforehand.
 * Replaces TokenLevelCompressor pooling (csa.py:79-87) and the block-emission
 * state machine of HCAKVCacheLayer/CSAKVCacheLayer.append
 * (kv_cache.py:170-195, 291-315). */
int skv_compress_append(void* pool, int64_t entry_bytes, int64_t block_size, int64_t n_pages,
                        const int32_t* block_table, int64_t bt_stride, float* tail_state,
                        const void* c_new, const void* z_new, int64_t in_seq_stride,
                        int64_t in_row_stride, int64_t in_len, const float* bias,
                        const int32_t* seq_lens, const int32_t* n_new, int32_t n_new_uniform,
                        int64_t m, int64_t channels, int32_t format, int64_t batch, void* stream);

/* ---- FP8 quantize-on-write --------------------------------------------------
 * skv_paged_append for SKV_FMT_FP8 entries: bf16 source rows of `channels`
 * dims are quantized per 1x128 block on the way into the pool
 * (cast_to_fp8, quant/reference.py:75-111; rope dims kept bf16). */
int skv_fp8_quant_append(void* pool, int64_t entry_bytes, int64_t block_size, int64_t n_pages,
                         const int32_t* block_table, int64_t bt_stride, const int32_t* seq_lens,
                         const int32_t* n_new, int32_t n_new_uniform, const void* src,
                         int64_t src_seq_stride, int64_t src_row_stride, int64_t src_len,
                         int64_t channels, int64_t batch, void* stream);

/* Host-side access to the e4m3fn codec the kernels use (CPU, no GPU), for
 * exhaustive codec checks.  No reference counterpart. */
int skv_fp8_encode_host(const float* x, uint8_t* codes, int64_t n);
int skv_fp8_decode_host(const uint8_t* codes, float* x, int64_t n);

/* ---- top-k selection --------------------------------------------------------
 * Row r of fp32 scores (row stride score_stride elements) has n_cols[r]
 * columns (n_cols == NULL: n_cols_uniform) of which the first n_valid[r] are
 * causally valid.  Writes k indices per row (row stride out_stride): the
 * min(k, n_cols, n_valid) best valid columns ordered by score descending,
 * ties by ascending index; a pick whose score is not finite is -1, and ranks
 * past that count are -1.  Replaces the mask + topk + isfinite of
 * CSA._indexer_topk_cached (csa.py:411-422).  k <= 2048, rows <= 65535. */
int skv_topk_select(const float* scores, int64_t score_stride, int64_t rows,
                    const int32_t* n_valid, const int32_t* n_cols, int32_t n_cols_uniform,
                    int64_t k, int32_t* out_idx, int64_t out_stride, int32_t* workspace,
                    void* stream);

/* Decode form: row b is the query at position seq_lens[b]-1 of sequence b,
 * n_cols = seq_lens[b] / m and n_valid = (seq_lens[b]-1) / m (a block s is
 * visible iff s*m + m - 1 < q_pos; kernels/attention.py:53-57). */
int skv_topk_select_decode(const float* scores, int64_t score_stride, int64_t batch,
                           const int32_t* seq_lens, int64_t m, int64_t k, int32_t* out_idx,
                           int64_t out_stride, int32_t* workspace, void* stream);

/* Top-k workspace size in int32 words per row.  workspace == NULL selects one
 * workgroup per row; otherwise each row is cut into 2048-score chunks (one
 * workgroup each, two launches) using rows * skv_topk_workspace_words() words
 * that must be zero before the first call and are left zero by every call.
 * Calls that share a workspace must not overlap. */
int64_t skv_topk_workspace_words(void);

/* ---- top-k gather -----------------------------------------------------------
 * dst[r, j] = entry max(idx[r*idx_stride + j], 0) of sequence row_seq[r]
 * (row_seq == NULL: r) from the paged compressed cache; a -1 pick reads
 * entry 0 (clamp(min=0), csa.py:328-331).  Picks at or past n_entries[b]
 * (including every pick of a sequence with no entries) produce zero rows.
 * SKV_FMT_BF16 copies entries; SKV_FMT_FP8 dequantizes them to bf16
 * (code * scale rounded to bf16; quant/reference.py:114-116).
 * dst: [rows, k, out_row] with out_row = entry_bytes (bf16) or 2*channels. */
int skv_topk_gather(void* dst, const void* pool, int64_t entry_bytes, int64_t block_size,
                    int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                    const int32_t* n_entries, const int32_t* idx, int64_t idx_stride, int64_t k,
                    int64_t rows, const int32_t* row_seq, int64_t channels, int32_t format,
                    void* stream);

/* ---- lightning-indexer scores -------------------------------------------------
 * scores[r, s] = sum_h w[r, h] * max(0, q[r, h, :] . k[b, s, :]) for query row
 * r = b * t_per_seq + t and every entry s < min(n_entries[b], max_entries) of
 * sequence b; k is the paged compressed indexer cache (bf16 [n_pages,
 * block_size, channels], block_table [batch, bt_stride]).  q: bf16 [rows,
 * n_heads, channels]; w: fp32 [rows, n_heads]; scores: fp32 [rows,
 * score_stride], unmasked (the top-k applies the causal block mask), -inf for
 * an entry whose page is not mapped; columns past the entry count are left
 * untouched.  Bf16 products accumulate in fp32 (MFMA).  Replaces the einsum +
 * clamp + weighted head sum of lightning_indexer_scores_reference
 * (kernels/attention.py:33-50) and CSA._indexer_topk_cached (csa.py:405-409);
 * no visual bias (the cached path ignores it, csa.py:396-399).
 * n_heads <= 64, channels a multiple of 8 up to 128, rows <= 65535. */
int skv_indexer_scores(const void* q, const float* w, const void* idx_pool, int64_t block_size,
                       int64_t n_pages, const int32_t* block_table, int64_t bt_stride,
                       const int32_t* n_entries, float* scores, int64_t score_stride, int64_t batch,
                       int64_t t_per_seq, int64_t n_heads, int64_t channels, int64_t max_entries,
                       void* stream);

/* ---- eviction and compaction --------------------------------------------------
 * skv_release: push every page of each sequence with release_mask[b] != 0 back
 * on the free stack (ascending b; within b from the last logical page to the
 * first), set its block-table row to -1 and its length to 0.  Refuses
 * (status SKV_STATUS_STACK / BADARG, nothing written) if the stack would
 * overflow or a released page id is invalid.  No reference counterpart. */
int skv_release(int32_t* free_stack, int32_t* free_top, int64_t n_pages, int32_t* block_table,
                int64_t bt_stride, int32_t* seq_lens, const uint8_t* release_mask, int64_t batch,
                int64_t block_size, int32_t* status, void* stream);

/* A pool whose pages share one block table (e.g. the main and indexer streams
 * of a CSA cache); page p of the pool is at base + p*page_bytes. */
typedef struct skv_pool_ref {
  void* base;
  int64_t page_bytes;
} skv_pool_ref;

/* skv_compact: defragment up to 16 pools sharing one block table.  Live pages
 * with id >= n_live move into the free ids < n_live (both ascending), the
 * tables are rewritten and the free stack rebuilt so pops return n_live,
 * n_live+1, ...  workspace: int32 [3*n_pages] whose first n_pages words are
 * zero before the first call and are left zero by every call (the rest is
 * scratch); info: int32 [2] receives {n_live, n_moved}.  Calls that share a
 * workspace must not overlap.  n_pages < 2^24, batch * bt_stride < 2^24.  No
 * reference counterpart. */
int skv_compact(const skv_pool_ref* pools, int32_t n_pools, int32_t* block_table,
                int64_t bt_stride, const int32_t* seq_lens, int64_t batch, int64_t block_size,
                int64_t n_pages, int32_t* free_stack, int32_t* free_top, int32_t* workspace,
                int32_t* info, void* stream);

/* ---- fused decode step ----------------------------------------------------
 * One decode step (one new token per sequence) of a stack of heterogeneous
 * layers in three launches, whatever the layer count:
 *   histogram : per CSA layer the 11-bit key histogram of the score row
 *            (with idx_q set: the scores themselves, computed from the
 *            indexer stream and written to scores, and their histogram);
 *            no launch without CSA layers.
 *   append : every workgroup computes the step's page plan (for each page
 *            group, the page of any compressed entry this token completes,
 *            popped in skv_reserve order: groups in order, ascending
 *            sequence; all-or-nothing: on a refusal nothing changes and
 *            *status gets SKV_STATUS_* bits); per layer, the token's latent
 *            row goes into its SWA ring; HCA/CSA layers fold (c, z) into the
 *            running pooling state and emit the entry when the block
 *            completes (bf16 or fp8); CSA layers do the same for the indexer
 *            stream (bf16 entries).  Beside it, per CSA layer, the top-k
 *            candidate lists (skv_topk_select_decode semantics).  New
 *            lengths and free-stack tops go to step_lens / step_top.
 *   gather : per CSA layer the ordered top_k picks and their gather (fp8
 *            dequantized to bf16; -1 reads entry 0, picks without an entry
 *            give zero rows); HCA layers copy all their entries (dense read,
 *            rows past the sequence's entries are left untouched); every
 *            layer copies the last min(window, L) tokens of its ring in
 *            position order; the step's lengths and tops are committed.
 *            A layer whose out_entries / out_window is NULL skips that copy
 *            (a consumer that reads the picks, entries and ring rows in
 *            place, as skv_decode_attention does, needs none of them).
 * skv_decode_step_launches returns the launches a step of the descriptor
 * takes (2 without CSA layers, else 3; 0 for an empty step; negative on a
 * bad descriptor).
 * Mirrors one cached step of CSA/HCA/SWAttention.forward over a
 * KVCacheBundle (model.py:294-315; csa.py:299-331; hca.py:110-141;
 * swa.py:107-125).  The kernels read the descriptor from device memory:
 * device_desc must hold a copy of *host_desc (uploaded by the caller).
 * batch <= 1024, up to 16 layers and 4 page groups. */
#define SKV_MAX_LAYERS 16
#define SKV_MAX_GROUPS 4
#define SKV_LAYER_SWA 0
#define SKV_LAYER_HCA 1
#define SKV_LAYER_CSA 2

typedef struct skv_page_group {
  int32_t* free_stack;  /* [n_pages] */
  int32_t* free_top;    /* [1] */
  int64_t n_pages;
  int32_t* block_table; /* [batch, bt_stride] */
  int64_t bt_stride;
  int32_t* n_entries;   /* [batch] compressed entries per sequence */
  int32_t m;            /* compression rate of every layer of the group */
  int32_t block_size;   /* entries per page */
} skv_page_group;

typedef struct skv_decode_layer {
  int32_t kind;           /* SKV_LAYER_* */
  int32_t group;          /* page group of an HCA/CSA layer */
  int32_t format;         /* SKV_FMT_* of the main compressed stream */
  int32_t top_k;          /* CSA: picks per query (<= 2048) */
  void* ring;             /* [batch, window, latent] bf16 */
  void* pool;             /* main stream pages: [n_pages, block_size, entry_bytes] */
  int64_t entry_bytes;
  float* state;           /* [batch, 3, latent] fp32 pooling state */
  const float* bias;      /* [m, latent] fp32 */
  void* idx_pool;         /* CSA indexer stream: [n_pages, block_size, c_indexer] bf16 */
  float* idx_state;       /* [batch, 3, c_indexer] */
  const float* idx_bias;  /* [m, c_indexer] */
  const void* kv_new;     /* [batch, latent] bf16: the new token's latent row */
  const void* c_new;      /* [batch, latent] bf16: compressor projections */
  const void* z_new;
  const void* ci_new;     /* [batch, c_indexer] bf16: indexer compressor projections */
  const void* zi_new;
  const float* scores;    /* CSA: [batch, score_stride] fp32 indexer scores */
  int64_t score_stride;
  int32_t* topk_idx;      /* CSA out: [batch, top_k] */
  int32_t* topk_ws;       /* CSA: [batch, skv_topk_workspace_words()] int32, zeroed once */
  void* out_entries;      /* CSA: [batch, top_k, latent]; HCA: [batch, out_rows, latent] bf16;
                           * NULL: no copy (a CSA layer still writes topk_idx) */
  int64_t out_rows;       /* HCA: rows per sequence of out_entries */
  void* out_window;       /* [batch, window, latent] bf16; NULL: no copy */
  /* CSA with an indexer stream, optional: the step's indexer query.  When
   * idx_q is set, the step computes the layer's scores itself (written to
   * scores, as skv_indexer_scores would over the entries before the step)
   * in its first launch, fused with the top-k histogram; the caller's
   * separate score launch and the histogram's read of the scores go away.
   * Either every CSA layer of the step sets it or none does. */
  const void* idx_q;      /* [batch, idx_heads, c_indexer] bf16 */
  const float* idx_w;     /* [batch, idx_heads] fp32 head weights */
  int32_t idx_heads;      /* 1..64 (c_indexer <= 128) */
  int32_t idx_pad_;
} skv_decode_layer;

typedef struct skv_decode_desc {
  int32_t batch;
  int32_t n_layers;
  int32_t n_groups;
  int32_t latent;         /* channels of the ring rows and main entries (multiple of 8) */
  int32_t c_indexer;      /* channels of the indexer stream (multiple of 8) */
  int32_t window;         /* SWA ring rows */
  int32_t* tok_lens;      /* [batch] tokens per sequence */
  int32_t* status;        /* [1] */
  int32_t* step_lens;     /* [batch] scratch: lengths after the step in flight */
  int32_t* step_top;      /* [SKV_MAX_GROUPS] scratch: free-stack tops after the step */
  skv_page_group groups[SKV_MAX_GROUPS];
  skv_decode_layer layers[SKV_MAX_LAYERS];
} skv_decode_desc;

int skv_decode_step(const skv_decode_desc* host_desc, const skv_decode_desc* device_desc,
                    void* stream);
int skv_decode_step_launches(const skv_decode_desc* host_desc);

/* Decode attention of one layer over the paged cache (T query tokens per
 * sequence, MQA: one K/V head, n_heads query heads of head_dim), the gather
 * fused in: replaces the cached-step attention of CSA.forward
 * (csa.py:324-373: sparse branch over the top-k picks + window branch),
 * HCA.forward (hca.py:126-169: dense branch over the visible entries + window
 * branch) and SWAttention.forward (swa.py:115-137: window branch), with
 * scaled_dot_product / softmax_with_sink / RMSNorm of common.py:12-124.
 * Query token t of sequence b (q, out: [batch, T, n_heads, head_dim]; T = 1
 * is [batch, n_heads, head_dim]) is the cache's position q_pos = lens[b] - T
 * + t: the T tokens were appended last, as the cached forward of csa.py:276-
 * 281 and hca.py:127-131 sees them (cache_offset = lens[b] - T).  It sees the
 * first L_t = q_pos + 1 positions:
 *   out[b,t,h,:] = compressed(b,t,h) + window(b,t,h), each its own softmax
 *   with scores q.k / sqrt(head_dim):
 *   compressed: K = V = k_norm(entry) = knorm_w * e * rsqrt(mean(e^2) + eps);
 *     CSA: the picks picks[b, t, j] >= 0 (rows of pick_stride; j < top_k;
 *     picks >= n_entries[b] are masked), no sink; HCA: entries s <
 *     floor(q_pos/m) (s*m + m-1 < q_pos, hca.py:128-130), at most
 *     n_entries[b], with the sink; SWA: none.  No live key: adds 0.
 *   window: keys win_k and values win_v of positions [L_t - min(W, L_t),
 *     L_t) (k_pos <= q_pos and q_pos - k_pos < W, swa.py:121-124), ring slot
 *     pos % ring ([batch, ring, head_dim] bf16, keys already normed and roped
 *     as the reference caches them), the sink, and the softcap c*tanh(s/c)
 *     when softcap > 0.  The ring must hold the last min(W + T - 1,
 *     lens[b]) positions: a ring of W + T - 1 slots or more always does, and
 *     so does a contiguous cache of the sequence's whole capacity (slot pos
 *     = pos), such as SWAKVCacheLayer's.
 * The pool's entries are bf16 or fp8 (dequantized to bf16 as the gathers
 * do).  Two launches: per (sequence, split, 64 heads) partial softmax
 * statistics and outputs into `workspace` (16-byte aligned), then the merge
 * into `out` (fp32).
 * skv_attention_workspace returns the workspace bytes (or -1 on a bad
 * descriptor). */
typedef struct skv_attention_desc {
  int32_t kind;             /* SKV_LAYER_SWA / SKV_LAYER_HCA / SKV_LAYER_CSA */
  int32_t format;           /* SKV_FMT_* of the pool's entries */
  int64_t batch, n_heads, head_dim; /* n_heads <= 256; head_dim a multiple of 32, <= 576 */
  const void* q;            /* [batch, n_heads, head_dim] bf16 (roped, q_norm applied) */
  float* out;               /* [batch, n_heads, head_dim] fp32 */
  const int32_t* lens;      /* [batch] tokens after the step's append */
  const void* pool;         /* compressed entries of head_dim channels */
  int64_t entry_bytes, block_size, n_pages;
  const int32_t* block_table;
  int64_t bt_stride;        /* bt_stride * block_size < 2^24 */
  const int32_t* n_entries; /* [batch] */
  int64_t m;                /* HCA compression rate */
  int64_t max_entries;      /* HCA: bound on entries per sequence (0: the table's capacity) */
  const int32_t* picks;     /* CSA: [batch, pick_stride] */
  int64_t pick_stride, top_k;
  const float* knorm_w;     /* [head_dim] */
  float eps;
  float softcap;            /* <= 0: none */
  const float* sink;        /* [n_heads] or NULL */
  const void* win_k;        /* [batch, ring] slots of head_dim bf16, win_stride apart */
  const void* win_v;        /* the same for values (may equal win_k) */
  int64_t window;
  int64_t splits;           /* 0: chosen by the library */
  int64_t n_queries;        /* query tokens per sequence, T (0: 1; at most 4096) */
  int64_t ring;             /* window slots per sequence (0: window), >= window; see above */
  int64_t win_stride;       /* bytes from one window slot to the next (0: head_dim * 2; a
                               multiple of 16), e.g. 4 * head_dim for [K | V] rows */
} skv_attention_desc;

int64_t skv_attention_workspace(const skv_attention_desc* desc);
/* sizeof(skv_attention_desc), so bindings can check their struct layout. */
int64_t skv_attention_desc_size(void);
int skv_decode_attention(const skv_attention_desc* desc, void* workspace, int64_t ws_bytes, void* stream);

/* One decode step of a one-layer stack followed by that layer's decode
 * attention, in the launches of skv_decode_step with its gather launch
 * replaced by the attention's: what one layer of a model's cached forward
 * does (model.py:294-315: the block's attention appends to its cache layer,
 * csa.py:299-373 / hca.py:110-169 / swa.py:107-137, then attends over it).
 *   hist, append : as skv_decode_step;
 *   attention    : per (sequence, split, 64 heads) units as
 *                  skv_decode_attention's; a CSA unit ranks its share of the
 *                  row's top-k candidates (the ordering of skv_decode_step's
 *                  gather launch), writes those positions of topk_idx and
 *                  attends over its picks in place; the step's lengths, entry
 *                  counts and tops are committed;
 *   merge        : as skv_decode_attention's.
 * The results equal skv_decode_step followed by skv_decode_attention over
 * the cache (topk_idx, lengths, pages and rings bit for bit; the attention
 * output up to its partial sums' order).  The layer writes no gathered
 * copies (out_entries and out_window NULL).  `attn` supplies q, out,
 * knorm_w (HCA/CSA), eps, softcap, sink, win_v (NULL: the layer's ring),
 * n_heads, head_dim (= latent), batch (= the step's), max_entries and
 * splits; the cache fields (kind, format, lens, pool, block table, entry
 * counts, m, picks, top_k, win_k, window) are taken from the step's
 * descriptor.  skv_decode_step_attend_workspace returns the workspace bytes
 * (16-byte aligned, as skv_decode_attention's), or -1 on bad descriptors. */
int64_t skv_decode_step_attend_workspace(const skv_decode_desc* host_desc, const skv_attention_desc* attn);
int skv_decode_step_attend(const skv_decode_desc* host_desc, const skv_decode_desc* device_desc,
                           const skv_attention_desc* attn, void* workspace, int64_t ws_bytes, void* stream);

/* sizeof(skv_decode_desc), sizeof(skv_decode_layer), sizeof(skv_page_group)
 * written to out[0..2], so bindings can check their struct layout. */
int skv_decode_desc_sizes(int64_t* out);

#ifdef __cplusplus
}
#endif

#endif /* SAINTKV_H_ */
