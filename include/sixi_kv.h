/*
 * sixi_kv.h -- C ABI of the KV-cache writes around the attention hot path (gfx950).
 *
 * The attention of include/sixi_attn.h reads each stream's K/V cells; these calls put the
 * cells there and move them between streams, in the same ggml view convention
 * (sixi_view, ggml type ids, status codes of sixi_attn.h).
 *
 * Reference interfaces these replace (file:line in the reference tree):
 *   - sixi_kv_write: the K/V store of each new token that upstream llama.cpp runs inside
 *     every llama_decode the engine makes (src/core/core_execution.cpp:2074 verify,
 *     :3536 prefill chunk, :3811 decode): ggml_set_rows of the step's K (or V) rows into
 *     the cache view, converting f32 to the cache type.  Conversions are the reference's
 *     codecs, src/core/numeric.cpp:28-106 (f16, round to nearest even) and :349-384
 *     (q8_0 blocks of include/sixi_asi/numeric.hpp:32-38).
 *   - sixi_kv_copy: the data movement of llama_memory_seq_cp between two sequences held
 *     in separate streams (src/core/core_execution.cpp:3215-3216 snapshot save,
 *     :3245-3246 restore).
 *   - Rollback (src/core/core_execution.cpp:4021-4062, llama_memory_seq_rm) needs no call:
 *     the caller shortens kv_len, and the attention never reads past it.
 *
 * Ownership and threading as in sixi_attn.h: the caller owns every buffer, a call
 * allocates nothing and is asynchronous on `stream`.
 */
#ifndef SIXI_KV_H
#define SIXI_KV_H

#include "sixi_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sixi_kv_write_params {
    sixi_view src;          /* [D, n_rows, Hkv, S] f32 or f16: the new K (or V) rows; rows
                               contiguous (nb[0] = element size), 16-byte aligned          */
    sixi_view dst;          /* [D, n_cells, Hkv, S] f16 or q8_0: the cache; same D, Hkv, S;
                               f16 rows 16-byte aligned, q8_0 rows 2-byte aligned;
                               paged (page_table != NULL): the page pool
                               [D, SIXI_KV_PAGE_CELLS, Hkv, n_pages], nb[3] = page stride   */
    const int32_t* kv_len;  /* device [S]: cell of row 0 in stream s, or NULL (cell 0)      */
    const int32_t* q_len;   /* device [S]: rows of stream s (<= n_rows), or NULL (= n_rows) */
    int32_t flags;          /* reserved, must be 0                                          */
    int32_t reserved;
    void* stream;           /* hipStream_t; NULL = the null stream                          */
    /* Paged cache (optional, as sixi_attn_params): cell c of stream s is cell c % 256 of page
     * page_table[s * page_table_stride + c / 256] of dst; a stream has
     * n_cells = page_table_stride * 256 cells.  Entries are clamped to [0, n_pages). */
    const int32_t* page_table;
    int64_t page_table_stride;
} sixi_kv_write_params;

/* Writes row j < q_len[s] of stream s to cell kv_len[s] + j of dst, for every kv-head.
 * A row whose cell falls outside [0, n_cells) is not written; no other cell changes. */
int sixi_kv_write(const sixi_kv_write_params* p);

/* Host-side validation only (no device access): SIXI_OK or the error sixi_kv_write returns. */
int sixi_kv_write_validate(const sixi_kv_write_params* p);

typedef struct sixi_kv_copy_params {
    sixi_view cache;        /* [D, n_cells, Hkv, S] f16 or q8_0 (K or V of one layer)      */
    int32_t src_stream;
    int32_t dst_stream;
    int64_t src_cell;       /* first cell read in src_stream                               */
    int64_t dst_cell;       /* first cell written in dst_stream                            */
    int64_t n_cells;        /* cells copied (every kv-head); 0 copies nothing              */
    void* stream;           /* hipStream_t; NULL = the null stream                          */
} sixi_kv_copy_params;

/* Copies cells [src_cell, src_cell + n_cells) of src_stream to [dst_cell, dst_cell + n_cells)
 * of dst_stream.  Both ranges must lie inside the view; overlapping ranges are rejected
 * (SIXI_E_INVALID_ARGUMENT). */
int sixi_kv_copy(const sixi_kv_copy_params* p);

/* ---- Page pool: 256-cell pages shared between streams ----
 *
 * Host-side bookkeeping of a paged KV cache: which pages of the K/V pools (views
 * [D, SIXI_KV_PAGE_CELLS, Hkv, n_pages] of every layer) hold the cells of each stream, in the
 * page-table form that sixi_attn_params and sixi_kv_write_params read.  Streams own a prefix
 * of their page-table row; a page may be held by several streams (reference counted).
 *
 * Reference interfaces these replace (file:line in the reference tree): the KV memory
 * operations llama.cpp runs for the engine -- page_size_tokens = 256
 * (include/sixi_asi/manifest.hpp:124); llama_memory_seq_cp, which shares the source's cells
 * with the destination sequence (src/core/core_execution.cpp:3215-3216 snapshot save,
 * :3245-3246 restore); llama_memory_seq_rm, truncation (:4021-4062 rollback, and the
 * whole-sequence drop before a copy at :3215 and :3245).  Copies move no cell data: a stream
 * that then writes into a shared page first gets a private copy of that page
 * (sixi_kv_pool_prepare_write), one page per write boundary.
 *
 * Pool calls are host-side and thread-safe (one lock per pool); only
 * sixi_kv_pool_prepare_write (page copies) and sixi_kv_pool_upload touch the device. */
typedef struct sixi_kv_pool sixi_kv_pool;

/* n_pages pages for n_streams streams of at most max_pages pages each.  *out is NULL on error. */
int sixi_kv_pool_create(int32_t n_pages, int32_t n_streams, int32_t max_pages, sixi_kv_pool** out);
void sixi_kv_pool_destroy(sixi_kv_pool* pool);

/* Registers a pool view (K or V of one layer: [D, SIXI_KV_PAGE_CELLS, Hkv, n_pages], f16 or
 * q8_0, nb[3] the page stride) whose pages copy-on-write duplicates.  At most 256 views. */
int sixi_kv_pool_attach(sixi_kv_pool* pool, const sixi_view* pages);

/* Before stream s writes cells [first, first + n): gives it pages through cell first + n - 1
 * (new pages for a longer stream), and replaces each page of that range that another stream
 * also holds by a private copy (every attached view's page copied on `stream`, ordered before
 * the caller's later work there).  SIXI_E_OUT_OF_BOUNDS when the stream would exceed
 * max_pages or the pool has too few free pages; nothing changes then. */
int sixi_kv_pool_prepare_write(sixi_kv_pool* pool, int32_t s, int64_t first, int64_t n, void* stream);

/* llama_memory_seq_rm(s, p0, -1): stream s keeps cells [0, p0) (p0 < 0: none); the pages past
 * them are released (freed when no stream holds them). */
int sixi_kv_pool_seq_rm(sixi_kv_pool* pool, int32_t s, int64_t p0);

/* llama_memory_seq_cp(src, dst): dst drops its pages, then holds src's pages of cells [0, n)
 * (n < 0: all of src's pages).  O(pages) bookkeeping, no cell data moves.  src == dst is a
 * no-op; n beyond src's pages is SIXI_E_OUT_OF_BOUNDS. */
int sixi_kv_pool_seq_cp(sixi_kv_pool* pool, int32_t src, int32_t dst, int64_t n);

/* The page table, n_streams rows of max_pages int32 entries (-1: no page), into host memory. */
int sixi_kv_pool_page_table(const sixi_kv_pool* pool, int32_t* host_dst);
/* The same into device memory (n_streams * max_pages int32), copied on `stream` and ordered
 * with the caller's work there; later pool changes do not reach this copy.  The call does
 * not wait for the stream: it copies from one of two pinned snapshots of the pool (waiting
 * only, if at all, for the copy two uploads earlier that read the same snapshot).  Under
 * HIP graph capture it records kernel launches that carry the table in their arguments, so
 * every replay stores the table as it was at capture. */
int sixi_kv_pool_upload(const sixi_kv_pool* pool, int32_t* dev_dst, void* stream);

int32_t sixi_kv_pool_free_pages(const sixi_kv_pool* pool);             /* < 0: error */
int32_t sixi_kv_pool_stream_pages(const sixi_kv_pool* pool, int32_t s);  /* pages s holds */
int32_t sixi_kv_pool_page_refs(const sixi_kv_pool* pool, int32_t page);  /* streams holding it */

#ifdef __cplusplus
}
#endif
#endif /* SIXI_KV_H */
