/*
 * sixi_layer.h -- C ABI of the work fused around the attention op of one Qwen3.8 full-attention
 * layer (gfx950): the Q/K prologue with the KV store, and the output gate.
 *
 * Reference geometry (configs/qwen3.8-27b-ud-q4-k-xl.sixi): key/value length 256, 24 q-heads,
 * 4 kv-heads, rms_norm_eps 1e-6, rope_dim_count 64, rope_freq_base 1e7; the layer carries
 * attn_q (24 * 256 * 2 outputs: per head the query, then its gate), attn_q_norm, attn_k_norm
 * and attn_output (blk.3 tensors of that file).  The graph that uses them is upstream
 * llama.cpp's (not in the reference tree), reached through every llama_decode of
 * src/core/core_execution.cpp:2074, :3536 and :3811:
 *   q, gate = split(attn_q(x)) per head;  k = attn_k(x);  v = attn_v(x)
 *   q = rope(rmsnorm(q) * attn_q_norm);   k = rope(rmsnorm(k) * attn_k_norm)
 *   store k, v in the cache;  o = attention(q, cache);  o = o * sigmoid(gate)
 * RoPE is the NEOX form on the first n_rot dims: pair (i, i + n_rot/2), angle
 * pos * base^(-2i/n_rot) with the angles of a row taken by repeated multiplication as ggml
 * does; dims >= n_rot pass unchanged.
 *
 * Ownership and threading as in sixi_attn.h.
 */
#ifndef SIXI_LAYER_H
#define SIXI_LAYER_H

#include "sixi_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sixi_qk_prologue_params {
    sixi_view qg;           /* [2D, H, n_rows, S] f32: attn_q output, per head D query then D gate */
    sixi_view k;            /* [D, Hkv, n_rows, S] f32: attn_k output                             */
    sixi_view v;            /* [D, Hkv, n_rows, S] f32: attn_v output                             */
    const float* q_norm;    /* device [D], 16-byte aligned: attn_q_norm weight                    */
    const float* k_norm;    /* device [D], 16-byte aligned: attn_k_norm weight                    */
    float eps;              /* RMS norm epsilon                                                   */
    float rope_base;        /* RoPE frequency base                                                */
    int32_t n_rot;          /* RoPE dims: even, a multiple of D/32, at most D                     */
    int32_t flags;          /* reserved, must be 0                                                */
    const int32_t* kv_len;  /* device [S]: cells cached before the block = position of row 0       */
    const int32_t* q_len;   /* device [S]: rows of stream s (<= n_rows), or NULL (= n_rows)        */
    sixi_view q_out;        /* [D, n_rows, H, S] f32, or f16 (rounded to nearest even) with an f16
                               cache: the attention's Q (sixi_attn_params.q); f16 halves its bytes
                               and leaves the attention's result the same bit for bit (it rounds Q
                               to f16 itself); a q8_0 cache needs f32 (ggml converts Q to the q8_0
                               dot type from its f32 values)                                      */
    sixi_view k_cache;      /* [D, n_cells, Hkv, S] f16 or q8_0; paged: the page pool
                               [D, SIXI_KV_PAGE_CELLS, Hkv, n_pages], nb[3] = page stride           */
    sixi_view v_cache;      /* same shape and type as k_cache                                     */
    void* stream;
    /* Paged caches (optional, as sixi_attn_params): cell c of stream s is cell c % 256 of page
     * page_table[s * page_table_stride + c / 256]; n_cells = page_table_stride * 256. */
    const int32_t* page_table;
    int64_t page_table_stride;
} sixi_qk_prologue_params;

/* For row j < q_len[s] of stream s (position kv_len[s] + j): writes the normed, rotated query of
 * every q-head to q_out, and stores the normed, rotated key and the value of every kv-head in
 * cell kv_len[s] + j of the caches (the codecs of sixi_kv_write; cells outside the cache are
 * skipped).  D is 128 or 256. */
int sixi_qk_prologue(const sixi_qk_prologue_params* p);

typedef struct sixi_attn_gate_params {
    sixi_view out;          /* [D, H, n_rows, S] f32: the attention output, gated in place         */
    sixi_view qg;           /* the prologue's qg: the gate is elements D .. 2D-1 of each head      */
    const int32_t* q_len;   /* device [S] or NULL                                                 */
    void* stream;
} sixi_attn_gate_params;

/* out *= sigmoid(gate) for rows j < q_len[s]. */
int sixi_attn_gate(const sixi_attn_gate_params* p);

#ifdef __cplusplus
}
#endif
#endif /* SIXI_LAYER_H */
