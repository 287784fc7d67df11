/*
 * sixi_gdn.h -- C ABI of the gated-delta-rule (GDN) recurrent verify (gfx950): every token of
 * every stream's block through the recurrent state of one linear-attention layer, in one call.
 *
 * Reference interfaces this replaces (file:line in the reference tree):
 *   - GdnOperator::step_token (src/core/core_execution.cpp:254-335) and its CUDA twin
 *     kernel_gdn_step_fp32 (src/cuda/sixi_kernels.cu:241-281, host wrapper cuda_gdn_step_fp32
 *     :602-660): one token, one stream.  Per group g and state row h (a value index):
 *       sk    = sum_s S[g][h][s] * k[g][s]            (the state before the step)
 *       delta = beta[g] * (v[g][h] - sk)
 *       S[g][h][s] = alpha[g] * S[g][h][s] + delta * k[g][s]
 *       y[g][h]    = sum_s S[g][h][s] * q[g][s]        (the state after the step)
 *     The reference verifies a block by calling it once per token (core_execution.cpp:823);
 *     here one launch runs q_len[s] tokens of every stream with the state held on chip.
 *   - The engine's GDN verify inside llama_decode (upstream ggml_gated_delta_net; the sequential
 *     per-row scan of src/core/core_execution.cpp:4072-4074, patches 0006/0007), whose decay
 *     acts before the state is read: SIXI_GDN_DECAY_FIRST uses sk = alpha * sum_s S*k.  The
 *     snapshot position (snap) plays the part of patch 0007's snap-back: the state written is
 *     the one after snap[s] tokens, so a rejected draft suffix needs no rollback copy.
 *
 * Shapes (ggml order, ne[0] innermost): G groups (value heads), K state size (key dim),
 * Hd head dim (value dim), n_rows rows per stream, S streams.
 *   q, k    [K, G, n_rows, S] f32       v, y   [Hd, G, n_rows, S] f32
 *   alpha, beta [G, n_rows, S, 1] f32   state_in, state_out [K, Hd, G, S] f32
 * Ownership and threading as in sixi_attn.h.
 */
#ifndef SIXI_GDN_H
#define SIXI_GDN_H

#include "sixi_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { SIXI_GDN_DECAY_FIRST = 1 };

typedef struct sixi_gdn_params {
    sixi_view q;
    sixi_view k;
    sixi_view v;
    sixi_view alpha;        /* per-token decay of each group                                    */
    sixi_view beta;         /* per-token write strength of each group                           */
    sixi_view y;            /* output, rows j < q_len[s]                                       */
    sixi_view state_in;     /* the state before row 0 of each stream                           */
    sixi_view state_out;    /* the state after snap[s] rows; may be state_in itself (in place)  */
    const int32_t* q_len;   /* device [S]: rows of stream s (<= n_rows), or NULL (= n_rows)     */
    const int32_t* snap;    /* device [S]: rows before the state written (clamped to
                               [0, q_len[s]]), or NULL (= q_len[s])                            */
    int32_t flags;          /* 0 (the reference's step) or SIXI_GDN_DECAY_FIRST                 */
    int32_t reserved;
    void* stream;
} sixi_gdn_params;

/* Runs rows j < q_len[s] of every stream through its state: y of each row, and the state after
 * snap[s] rows written to state_out (every stream's state is written).  (K, Hd) is (64, 64),
 * (64, 128), (128, 64) or (128, 128); rows contiguous and 16-byte aligned. */
int sixi_gdn_verify(const sixi_gdn_params* p);

#ifdef __cplusplus
}
#endif
#endif /* SIXI_GDN_H */
