/*
 * sixi_attn.h -- C ABI of the MI355X (gfx950) GQA attention hot path.
 *
 * One operator: O = softmax(scale * Q K^T + mask) V per (stream, query head, row) over
 * each stream's KV cache, with grouped-query heads (q-heads g*G .. g*G+G-1 share
 * kv-head g, G = H / Hkv).  It covers the three modes the engine drives:
 *   - single-token decode           (q_len = 1),
 *   - speculative verify of a block (q_len = 1 + k <= 16, block-causal),
 *   - chunked causal prefill        (q_len = chunk, causal over cache + chunk).
 *
 * Reference interface this replaces (file:line in the reference tree):
 *   - upstream ggml's ggml_flash_attn_ext(ctx, q, k, v, mask, scale, max_bias,
 *     logit_softcap), reached through llama_decode() at
 *     src/core/core_execution.cpp:2074 (multi-stream verify), :3536 (prefill chunk),
 *     :3811 (single-stream decode); flash attention is switched on at
 *     src/core/core_execution.cpp:2600-2608 and scripts/build_llamacpp.sh:41-45.
 *     The view layout (ne/nb, ggml type ids) and the permuted output [D, H, n_q, S]
 *     are ggml's; the per-stream lengths replace the host-built KQ mask that llama.cpp
 *     derives from the positions set at src/core/core_execution.cpp:2047-2062, and such a
 *     mask handed over as EXPLICIT is recognised on the device and run as those lengths.
 *   - status codes are the negated sixi_asi::ErrorCode values of
 *     include/sixi_asi/common.hpp:40-67 (no abort, no throw).
 *
 * Ownership and threading: the caller owns every buffer.  A call writes only `out` and
 * `workspace`, allocates nothing, and is asynchronous on `stream`.  Calls are reentrant;
 * two calls that share a workspace must be ordered on one stream.
 */
#ifndef SIXI_ATTN_H
#define SIXI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIXI_ATTN_ABI_VERSION 3

/* Cells per page of a paged KV cache (include/sixi_asi/manifest.hpp:124 page_size_tokens). */
#define SIXI_KV_PAGE_CELLS 256

/* ggml type ids (include/sixi_asi/common.hpp:170-180 QuantType: F32 0, F16 1, Q8_0 8) */
enum {
    SIXI_TYPE_F32 = 0,
    SIXI_TYPE_F16 = 1,
    SIXI_TYPE_Q8_0 = 8
};

/* Which cells a row sees (cells of stream s are numbered 0 .. n_kv-1 in its view):
 *  NONE          row j sees cells [0, kv_len[s] + q_len[s]); with kv_len == NULL, all
 *                n_kv cells (ggml with mask == NULL).
 *  BLOCK_CAUSAL  row j sees cells [0, kv_len[s] + j]  (the block's own K/V sit at cells
 *                kv_len[s] .. kv_len[s] + q_len[s] - 1, as llama.cpp stores them).
 *  EXPLICIT      ggml semantics: add the f16 `mask` view; -inf cells are skipped.  With
 *                kv_len != NULL only cells [0, kv_len[s] + q_len[s]) are scanned.  A cell
 *                that no row of its stream sees may hold any bits, NaN included. */
enum {
    SIXI_MASK_NONE = 0,
    SIXI_MASK_BLOCK_CAUSAL = 1,
    SIXI_MASK_EXPLICIT = 2
};

/* Status codes: 0 or -ErrorCode (include/sixi_asi/common.hpp:40-67). */
enum {
    SIXI_OK = 0,
    SIXI_E_INVALID_ARGUMENT = -1,   /* ErrorCode::InvalidArgument  */
    SIXI_E_OUT_OF_BOUNDS = -2,      /* ErrorCode::OutOfBounds (e.g. workspace too small) */
    SIXI_E_INTEGER_OVERFLOW = -3,   /* ErrorCode::IntegerOverflow  */
    SIXI_E_ALIGNMENT = -15,         /* ErrorCode::AlignmentError   */
    SIXI_E_BACKEND = -23,           /* ErrorCode::BackendError (HIP launch failed) */
    SIXI_E_UNSUPPORTED = -24        /* ErrorCode::UnsupportedHardware (shape/type not built) */
};

/* sixi_attn_params.flags.  BOUNDED_WORKSPACE: never stage a q8_0 cache as f16 in the
 * workspace, so the workspace does not grow with the cache.  Without it, prefill-sized
 * blocks over a q8_0 cache stage K and V as f16 operands (the prefill kernel converts Q to
 * the q8_0 dot type itself; split-K calls of unaligned 256-dim rows also stage Q) while that
 * copy takes at most
 * SIXI_ATTN_STAGE_CAP_BYTES (a separate pass, then the f16 kernel: faster than converting
 * every tile in LDS, which repeats the conversion in every work-group that reads the tile),
 * and convert the q8_0 tiles in LDS beyond it.  256-dim q8_0 rows that are not 16-byte
 * aligned are always staged (the in-LDS path loads rows by 16-byte DMA).  No counterpart in
 * the reference (ggml's kernels take no workspace). */
#define SIXI_ATTN_FLAG_BOUNDED_WORKSPACE 1
#define SIXI_ATTN_STAGE_CAP_BYTES ((size_t)64 << 20)
/* GATE (ABI version 3): multiply every written output element by sigmoid(gate), the output
 * gate of Qwen3.8's full-attention layers (o = attention * sigmoid(gate); the layer graph in
 * include/sixi_layer.h), with the gate read from `gate_qg` (the prologue's qg tensor: elements
 * D .. 2D-1 of each head's row).  The result equals sixi_attn_forward followed by
 * sixi_attn_gate bit for bit, without that second pass over the output.  No counterpart in
 * ggml_flash_attn_ext (upstream runs the gate as a separate graph node). */
#define SIXI_ATTN_FLAG_GATE 2

/* ggml-compatible strided view.  ne[0] is the innermost extent (elements); nb[] are byte
 * strides; for q8_0, nb[0] = 34 (one 32-element block) and a row of ne[0] elements takes
 * ne[0]/32*34 bytes. */
typedef struct sixi_view {
    const void* data;
    int32_t type;
    int32_t reserved;
    int64_t ne[4];
    int64_t nb[4];
} sixi_view;

typedef struct sixi_attn_params {
    sixi_view q;            /* [D, n_q, H, S]    f32 or f16                                */
    sixi_view k;            /* [D, n_kv, Hkv, S] f16 or q8_0; nb[1] cell, nb[2] head,
                               nb[3] stream (a 256-cell page multiple in the engine);
                               paged (page_table != NULL): the page pool
                               [D, SIXI_KV_PAGE_CELLS, Hkv, n_pages], nb[3] = page stride  */
    sixi_view v;            /* [D, n_kv, Hkv, S] f16 or q8_0, same D as k (paged: the same
                               pool shape as k)                                            */
    sixi_view out;          /* [D, H, n_q, S]    f32 (ggml's permuted output)             */
    const int32_t* kv_len;  /* device [S]: cells cached before the block, or NULL          */
    const int32_t* q_len;   /* device [S]: rows of stream s (<= n_q), or NULL (= n_q)      */
    int32_t mask_mode;      /* SIXI_MASK_*                                                 */
    int32_t flags;          /* SIXI_ATTN_FLAG_* bits; 0 by default                         */
    sixi_view mask;         /* EXPLICIT only: f16 [n_kv, >= n_q, 1, 1 or S]                */
    float scale;            /* 1/sqrt(D) for the engine's models                           */
    float max_bias;         /* ALiBi; 0 = off                                              */
    float logit_softcap;    /* 0 = off                                                     */
    float reserved_f;
    void* workspace;        /* device scratch of >= sixi_attn_workspace_bytes() bytes,
                               256-byte aligned; its contents need no initialisation       */
    size_t workspace_bytes;
    void* stream;           /* hipStream_t; NULL = the null stream                         */
    /* Paged KV (optional).  NULL: k and v hold each stream's cells as one range.  Otherwise
     * cell c of stream s is cell c % SIXI_KV_PAGE_CELLS of page
     * page_table[s * page_table_stride + c / SIXI_KV_PAGE_CELLS] of the k and v pools, and a
     * stream has n_kv = page_table_stride * SIXI_KV_PAGE_CELLS cells.  Device memory, int32,
     * 4-byte aligned; only the entries of cells a row can see are read, each clamped to
     * [0, n_pages) on the device.  Streams may share pages (sixi_kv_pool_seq_cp). */
    const int32_t* page_table;
    int64_t page_table_stride;
    /* SIXI_ATTN_FLAG_GATE only (ABI version 3; not read otherwise): f32 [2D, H, >= n_q, S],
     * per head D query values then D gate values (sixi_qk_prologue_params.qg); nb[0] = 4,
     * 16-byte aligned rows; must not overlap `out` */
    sixi_view gate_qg;
} sixi_attn_params;

/* Launches the attention for every stream, head and row.  Rows j >= q_len[s] are not
 * written.  kv_len[s] is clamped to [0, n_kv - q_len[s]] on the device. */
int sixi_attn_forward(const sixi_attn_params* p);

/* sixi_attn_forward without a caller workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The call allocates nothing: its scratch is a fixed
 * SIXI_ATTN_NOALLOC_SCRATCH_BYTES array in the library's device code, one per GPU, held
 * until the process ends; `workspace` and `workspace_bytes` are ignored.  q8_0 caches are
 * staged only while the staging fits the scratch (as with SIXI_ATTN_FLAG_BOUNDED_WORKSPACE
 * beyond that).  A description whose scratch (split-K partials, a q8_0 staging that cannot
 * be avoided) exceeds that size returns SIXI_E_OUT_OF_BOUNDS before any launch.  The scratch needs no initialisation, but every
 * call on a GPU shares it: calls that may overlap on one GPU (different streams, or
 * threads without ordering) race; order them on one stream. */
#define SIXI_ATTN_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int sixi_attn_forward_noalloc(const sixi_attn_params* p);

/* Workspace the call needs for this description (depends on S, H, Hkv, D, n_q, n_kv and
 * the device's CU count; not on the device-side lengths). */
int sixi_attn_workspace_bytes(const sixi_attn_params* p, size_t* bytes);

/* Host-side validation only (no device access): SIXI_OK or the error forward() returns. */
int sixi_attn_validate(const sixi_attn_params* p);

const char* sixi_attn_strerror(int code);
int sixi_attn_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* SIXI_ATTN_H */
