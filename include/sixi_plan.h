/*
 * sixi_plan.h -- host-side former of a multi-stream verify batch (no device access).
 *
 * The engine verifies the drafted blocks of several streams in one forward pass.  The
 * reference forms that pass in LlamaCppBackend::Impl::exec_verify_group
 * (src/core/core_execution.cpp:2016-2212): rows are stream-major, every stream is padded to
 * the longest block R by repeating its last token (pad rows are computed, stored in the KV
 * cache and removed again by settle_pads, :1990-2010), and a stream with less room than R
 * left in its context runs in a pass of its own (:2037-2045), because llama.cpp keeps
 * sequences in one ubatch only when they contribute equally many tokens.
 *
 * With per-stream lengths (sixi_attn.h: kv_len, q_len) the attention needs no padding: one
 * pass takes every stream with its own row count.  sixi_verify_plan gives both forms:
 *   SIXI_PAD_REFERENCE  the reference's parts, offsets and padded row counts, exactly;
 *   SIXI_PAD_NONE       one part, each stream with its real rows (q_len = real, pads never
 *                       computed or stored, nothing to settle afterwards).
 * For either, the attention and KV-store calls of part p take, at the stream's index i in
 * that part: kv_len[i] = cached, q_len[i] = rows (REFERENCE, pads included) or real (NONE).
 */
#ifndef SIXI_PLAN_H
#define SIXI_PLAN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { SIXI_PAD_REFERENCE = 0, SIXI_PAD_NONE = 1 };

typedef struct sixi_verify_stream {
    int32_t stream;  /* the engine's stream id                                     */
    int32_t cached;  /* N: tokens already in the stream's KV cache (>= 0)           */
    int32_t real;    /* rows of the block: anchor + drafts (>= 1)                   */
} sixi_verify_stream;

typedef struct sixi_verify_slot {
    int32_t part;        /* forward pass that carries the stream                    */
    int32_t index;       /* the stream's position inside its part                   */
    int32_t row_offset;  /* first row of the stream in its part (stream-major rows) */
    int32_t rows;        /* rows it occupies: real + pad rows                       */
} sixi_verify_slot;

/* Plans the verify pass(es) of n streams.  out[i] describes in[i]; *n_parts receives the
 * number of passes (parts are numbered in order of first appearance, streams keep their
 * input order inside a part).  n_ctx_seq is the context of one sequence (the reference's
 * n_ctx / n_seq_max; 0 means 4096 as in the reference).  Returns 0 or SIXI_E_INVALID_ARGUMENT
 * (-1) for a NULL pointer, n < 0, an unknown pad mode, cached < 0 or real < 1. */
int sixi_verify_plan(const sixi_verify_stream* in, int32_t n, int64_t n_ctx_seq, int32_t pad_mode,
                     sixi_verify_slot* out, int32_t* n_parts);

#ifdef __cplusplus
}
#endif
#endif /* SIXI_PLAN_H */
