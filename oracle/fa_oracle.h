/*
 * fa_oracle.h -- CPU restatement of the attention hot path, used ONLY as a checker.
 *
 * This is test infrastructure.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path (libsixi_attn.so) never links it.
 *
 * What it restates:
 *  - fp16 codec of the reference (src/core/numeric.cpp:28-106): exact f16->f32,
 *    f32->f16 round-to-nearest-even with subnormals, overflow to inf, quiet NaN.
 *  - q8_0 block codec (include/sixi_asi/numeric.hpp:32-38, src/core/numeric.cpp:349-384):
 *    34-byte block {f16 d; int8 qs[32]}, d = f16(amax/127), id = 127/amax,
 *    q = clamp(round_half_away(x*id), -127, 127).
 *  - ggml CPU flash_attn_ext row kernel (upstream llama.cpp/ggml at a691b234, not in the
 *    reference tree; enabled by scripts/build_llamacpp.sh:41-45 and
 *    src/core/core_execution.cpp:2600-2608): per (stream, head, row) a serial online
 *    softmax over the KV cells; Q converted to K's dot type (f16 or q8_0); mask value
 *    -inf skips the cell; V accumulated in f16 (upstream's one-row kernel) or f32.
 *  - the llama KQ mask for stream-major multi-sequence batches
 *    (src/core/core_execution.cpp:2047-2062: row j of stream s has pos N_s + j and sees
 *    the cells of its own sequence with pos <= N_s + j).
 *  - PCG32 XSH-RR (src/core/core_execution.cpp:33-62) with Box-Muller normals in float64.
 *
 * Parity pins (what checks each function; see tests/test_oracle_*.py):
 *  - fp16 codec: exhaustive over all 65536 halves against the compiled reference
 *    numeric.cpp (oracle/_ref) and against an independent numpy rounding.
 *  - q8_0 codec: bit-exact against the compiled reference numeric.cpp on random and
 *    hand-made tie blocks; closed form per block.
 *  - PCG32: bit-exact against the compiled reference DeterministicRng is not possible
 *    (core_execution.cpp pulls in the whole engine), so it is pinned by the published
 *    PCG32 known-answer vector (pcg32-demo, seed 42 / seq 54).
 *  - attention: float64 brute force on small shapes, textbook special cases (one
 *    dominant key, equal scores, single cell), invariances (key permutation, Q/scale
 *    reciprocity), and mask equivalence against the llama-style mask builder.
 */
#ifndef SIXI_FA_ORACLE_H
#define SIXI_FA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_Q8_0 = 8 };

/* ggml-style strided 4-d view: ne[0] innermost; nb[] in bytes (nb[0] = element size;
 * for q8_0 nb[0] = 34 and ne[0] counts elements, a multiple of 32). */
typedef struct oracle_view {
    const void* data;
    int32_t type;
    int64_t ne[4];
    int64_t nb[4];
} oracle_view;

/* AVX2/F16C/FMA loops (same association order as the scalar code): on/off, available */
int      oracle_set_simd(int on);
int      oracle_have_simd(void);

/* ---- codecs ---- */
float    oracle_fp16_to_fp32(uint16_t h);
uint16_t oracle_fp32_to_fp16(float f);
void     oracle_fp32_to_fp16_row(const float* x, uint16_t* y, int64_t n);
void     oracle_fp16_to_fp32_row(const uint16_t* x, float* y, int64_t n);
/* n multiple of 32; dst holds n/32 blocks of 34 bytes. Returns 0, or -1 on bad n. */
int      oracle_quantize_row_q8_0(const float* x, void* dst, int64_t n);
void     oracle_dequantize_row_q8_0(const void* src, float* y, int64_t n);

/* ---- dots (ggml CPU vec_dot restatements, x86 AVX2 association order) ---- */
float oracle_vec_dot_f16(int64_t n, const uint16_t* x, const uint16_t* y);
float oracle_vec_dot_q8_0(int64_t n, const void* x, const void* y);

/* ---- the op ----
 * q    : [D, n_q, H, S]   f32
 * k, v : [D, n_kv, Hkv, S] f16 or q8_0 (k and v may differ)
 * mask : f16 [n_kv, >= n_q, 1|H, 1|S] or NULL (no mask)
 * out  : f32, contiguous [D, H, n_q, S] (ggml permuted layout: out[s][i][h][d])
 * v_acc_f16: 1 = upstream f16 V accumulator (only when v is f16), 0 = f32 accumulator.
 * n_threads: OpenMP threads (<= 0: library default).
 * Returns 0 on success, negative on an invalid description. */
int oracle_flash_attn_ext(const oracle_view* q, const oracle_view* k, const oracle_view* v,
                          const oracle_view* mask, float scale, float max_bias,
                          float logit_softcap, float* out, int v_acc_f16, int n_threads);

/* Builds the llama-style f16 KQ mask for a stream-major batch whose stream s has
 * kv_len[s] cached cells and q_len[s] new rows at cells kv_len[s]..kv_len[s]+q_len[s]-1.
 * mask is [n_kv, n_q_pad, 1, S] contiguous f16.  causal = 1: row j sees cells
 * <= kv_len[s] + j; causal = 0: row j sees all kv_len[s] + q_len[s] cells.  Rows j >=
 * q_len[s] and cells >= kv_len[s] + q_len[s] are -inf.  Returns -1 if a stream's cells
 * exceed n_kv. */
int oracle_build_kq_mask(uint16_t* mask, int64_t n_kv, int64_t n_q_pad, int64_t S,
                         const int32_t* kv_len, const int32_t* q_len, int causal);

/* ---- deterministic generator ---- */
typedef struct oracle_pcg32 { uint64_t state, inc; } oracle_pcg32;
void     oracle_pcg32_seed(oracle_pcg32* r, uint64_t seed, uint64_t seq);
uint32_t oracle_pcg32_next(oracle_pcg32* r);
double   oracle_pcg32_uniform01(oracle_pcg32* r);   /* 53-bit: (u64 >> 11) * 2^-53 */
/* n N(0,1) draws (Box-Muller in float64, both outputs used), times `mul`, cast to f32 */
void     oracle_fill_normal_f32(uint64_t seed, uint64_t seq, float mul, float* out, int64_t n);

/* Gated-delta-rule recurrent verify (restates GdnOperator::step_token,
 * src/core/core_execution.cpp:254-335, applied token by token as the reference's verify does,
 * :823): dense arrays q, k [S][n_rows][G][K], v, y [S][n_rows][G][HD], alpha, beta
 * [S][n_rows][G], state [S][G][HD][K] (updated in place to the state after snap[s] rows;
 * NULL q_len / snap = n_rows / q_len).  decay_first multiplies sk by alpha (ggml's order).
 * Sums run serially over the K columns in index order, as the reference's loops do. */
void oracle_gdn_verify(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                       float* state, float* y, int64_t S, int64_t n_rows, int64_t G, int64_t K, int64_t HD,
                       const int32_t* q_len, const int32_t* snap, int decay_first);

#ifdef __cplusplus
}
#endif
#endif
