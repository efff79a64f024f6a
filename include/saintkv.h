/*
 * saintkv.h — C ABI of the MI355X (gfx950) heterogeneous KV-cache library.
 *
 * Plain C: raw device pointers, int64 sizes, a hipStream_t (passed as void*).
 * Every entry point returns 0 on success or a negative SKV_E* code; the text
 * of the last error on the calling thread is available from skv_last_error().
 * The library allocates nothing: every buffer is owned by the caller.
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

/* Device-side status words written by kernels that can refuse work
 * (bit flags, 0 = success). */
#define SKV_STATUS_MAX_PAGES 1 /* a sequence would exceed bt_stride pages   */
#define SKV_STATUS_NOSPC 2     /* not enough free pages                     */
#define SKV_STATUS_BADARG 4    /* negative count                            */
#define SKV_STATUS_STACK 8     /* release would overfill the free stack     */

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

#ifdef __cplusplus
}
#endif

#endif /* SAINTKV_H_ */
