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
                               f16 rows 16-byte aligned, q8_0 rows 2-byte aligned           */
    const int32_t* kv_len;  /* device [S]: cell of row 0 in stream s, or NULL (cell 0)      */
    const int32_t* q_len;   /* device [S]: rows of stream s (<= n_rows), or NULL (= n_rows) */
    int32_t flags;          /* reserved, must be 0                                          */
    int32_t reserved;
    void* stream;           /* hipStream_t; NULL = the null stream                          */
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

#ifdef __cplusplus
}
#endif
#endif /* SIXI_KV_H */
