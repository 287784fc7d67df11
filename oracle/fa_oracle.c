/*
 * fa_oracle.c -- CPU restatement of the attention hot path (test infrastructure only).
 *
 * Nothing in the product library links or calls this file; it is the checker that the
 * HIP path is compared against, and the CPU baseline that bench.py times.  See
 * fa_oracle.h for what each function restates and how it is pinned.
 */
#include "fa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__AVX2__) && defined(__F16C__) && defined(__FMA__)
#include <immintrin.h>
#define ORACLE_HAVE_SIMD 1
#else
#define ORACLE_HAVE_SIMD 0
#endif

/* 1 = use the AVX2/F16C/FMA loops where compiled in.  They keep the scalar code's
 * association order, so both settings give bitwise-identical results (tested). */
static int g_use_simd = ORACLE_HAVE_SIMD;
int oracle_set_simd(int on) { g_use_simd = on && ORACLE_HAVE_SIMD; return g_use_simd; }
int oracle_have_simd(void) { return ORACLE_HAVE_SIMD; }

/* ------------------------------------------------------------------------------------
 * fp16 codec -- semantics of src/core/numeric.cpp:28-106 (fp16_to_fp32 / fp32_to_fp16).
 * ---------------------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in f32 */
        float mag = ldexpf((float)m, -24);
        return u2f(f2u(mag) | sign);
    }
    if (e == 31) {
        /* inf, or NaN with the quiet bit forced as numeric.cpp:50-53 does */
        return u2f(sign | 0x7f800000u | (m ? 0x00400000u : 0u) | (m << 13));
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        const uint32_t payload = (ax >> 13) & 0x3ffu;
        return (uint16_t)(sign | 0x7e00u | (payload ? payload : 1u));
    }
    if (ax < 0x00800000u) return sign; /* f32 subnormal: far below half the f16 subnormal */
    const int32_t e = (int32_t)(ax >> 23) - 112;   /* f16 biased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    const uint32_t sig = (ax & 0x7fffffu) | 0x800000u; /* 24-bit significand */
    uint32_t h, rem, half;
    if (e >= 1) {
        /* normal: (e-1)<<10 plus the 11-bit significand (hidden bit carries into e) */
        h = ((uint32_t)(e - 1) << 10) + (sig >> 13);
        rem = sig & 0x1fffu;
        half = 0x1000u;
    } else {
        const int32_t shift = 14 - e;               /* 14..24 for e in [0, -10] */
        if (shift > 24) return sign;
        h = sig >> shift;
        rem = sig & ((1u << shift) - 1u);
        half = 1u << (shift - 1);
    }
    if (rem > half || (rem == half && (h & 1u))) ++h;   /* carry may reach inf: correct */
    return (uint16_t)(sign | h);
}

void oracle_fp32_to_fp16_row(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_fp32_to_fp16(x[i]);
}
void oracle_fp16_to_fp32_row(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------------------------
 * q8_0 codec -- include/sixi_asi/numeric.hpp:32-38 (34-byte block) and
 * src/core/numeric.cpp:349-384 (d = amax/127 stored as f16, id = 127/amax,
 * q = clamp(round(x*id)), round = half away from zero).
 * ---------------------------------------------------------------------------------- */
#define QK8_0 32
#define Q8_0_BYTES 34

int oracle_quantize_row_q8_0(const float* x, void* dst, int64_t n) {
    if (n < 0 || (n % QK8_0) != 0) return -1;
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        const float* xb = x + b * QK8_0;
        float amax = 0.0f;
        for (int i = 0; i < QK8_0; ++i) {
            const float a = fabsf(xb[i]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const uint16_t dh = oracle_fp32_to_fp16(d);
        const float id = (d != 0.0f) ? (127.0f / amax) : 0.0f;
        uint8_t* blk = out + b * Q8_0_BYTES;
        memcpy(blk, &dh, 2);
        for (int i = 0; i < QK8_0; ++i) {
            float r = roundf(xb[i] * id);
            int32_t q = (int32_t)r;
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            blk[2 + i] = (uint8_t)(int8_t)q;
        }
    }
    return 0;
}

void oracle_dequantize_row_q8_0(const void* src, float* y, int64_t n) {
    const uint8_t* in = (const uint8_t*)src;
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        const uint8_t* blk = in + b * Q8_0_BYTES;
        uint16_t dh;
        memcpy(&dh, blk, 2);
        const float d = oracle_fp16_to_fp32(dh);
        for (int i = 0; i < QK8_0; ++i) y[b * QK8_0 + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* ------------------------------------------------------------------------------------
 * Dots.  ggml's x86 AVX2/F16C/FMA vec_dot_f16 keeps 4 accumulators of 8 f32 lanes over
 * steps of 32 elements, reduces acc0+=acc2, acc1+=acc3, acc0+=acc1, then lane pairs
 * (i, i+4), then two horizontal adds; the tail is summed in double.  vec_dot_q8_0_q8_0
 * keeps 8 f32 lanes, each the FMA of (d_x*d_y) with the exact int sum of 4 byte products,
 * and reduces them as hsum_float_8.  Both are restated scalar with the same association
 * so the result does not depend on the build's SIMD flags.
 * ---------------------------------------------------------------------------------- */
float oracle_vec_dot_f16(int64_t n, const uint16_t* x, const uint16_t* y) {
    float acc[4][8];
    memset(acc, 0, sizeof(acc));
    const int64_t np = n & ~(int64_t)31;
    for (int64_t i = 0; i < np; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l) {
                const int64_t t = i + 8 * j + l;
                acc[j][l] = fmaf(oracle_fp16_to_fp32(x[t]), oracle_fp16_to_fp32(y[t]), acc[j][l]);
            }
    for (int l = 0; l < 8; ++l) { acc[0][l] += acc[2][l]; acc[1][l] += acc[3][l]; }
    for (int l = 0; l < 8; ++l) acc[0][l] += acc[1][l];
    float t0[4];
    for (int l = 0; l < 4; ++l) t0[l] = acc[0][l] + acc[0][l + 4];
    const float t1a = t0[0] + t0[1], t1b = t0[2] + t0[3];
    double sum = (double)(t1a + t1b);
    for (int64_t t = np; t < n; ++t)
        sum += (double)(oracle_fp16_to_fp32(x[t]) * oracle_fp16_to_fp32(y[t]));
    return (float)sum;
}

float oracle_vec_dot_q8_0(int64_t n, const void* xv, const void* yv) {
    const uint8_t* x = (const uint8_t*)xv;
    const uint8_t* y = (const uint8_t*)yv;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        const uint8_t* xb = x + b * Q8_0_BYTES;
        const uint8_t* yb = y + b * Q8_0_BYTES;
        uint16_t dx, dy;
        memcpy(&dx, xb, 2);
        memcpy(&dy, yb, 2);
        const float d = oracle_fp16_to_fp32(dx) * oracle_fp16_to_fp32(dy);
        for (int l = 0; l < 8; ++l) {
            int32_t s = 0;
            for (int t = 0; t < 4; ++t)
                s += (int32_t)(int8_t)xb[2 + 4 * l + t] * (int32_t)(int8_t)yb[2 + 4 * l + t];
            acc[l] = fmaf(d, (float)s, acc[l]);
        }
    }
    float r[4];
    for (int l = 0; l < 4; ++l) r[l] = acc[l + 4] + acc[l];
    r[0] = r[0] + r[2];
    r[1] = r[1] + r[3];
    return r[0] + r[1];
}

#if ORACLE_HAVE_SIMD
static float dot_f16_simd(int64_t n, const uint16_t* x, const uint16_t* y) {
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    const int64_t np = n & ~(int64_t)31;
    for (int64_t i = 0; i < np; i += 32)
        for (int j = 0; j < 4; ++j) {
            const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + i + 8 * j)));
            const __m256 b = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(y + i + 8 * j)));
            acc[j] = _mm256_fmadd_ps(a, b, acc[j]);
        }
    acc[0] = _mm256_add_ps(acc[0], acc[2]);
    acc[1] = _mm256_add_ps(acc[1], acc[3]);
    acc[0] = _mm256_add_ps(acc[0], acc[1]);
    const __m128 t0 = _mm_add_ps(_mm256_castps256_ps128(acc[0]), _mm256_extractf128_ps(acc[0], 1));
    const __m128 t1 = _mm_hadd_ps(t0, t0);
    const __m128 t2 = _mm_hadd_ps(t1, t1);
    double sum = (double)_mm_cvtss_f32(t2);
    for (int64_t t = np; t < n; ++t)
        sum += (double)(oracle_fp16_to_fp32(x[t]) * oracle_fp16_to_fp32(y[t]));
    return (float)sum;
}
#endif

/* VKQ16 = f16(f32(VKQ16) * ms) elementwise */
static void scale_f16(int64_t n, uint16_t* y, float v) {
    int64_t i = 0;
#if ORACLE_HAVE_SIMD
    if (g_use_simd) {
        const __m256 vv = _mm256_set1_ps(v);
        for (; i + 8 <= n; i += 8) {
            __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(y + i)));
            a = _mm256_mul_ps(a, vv);
            _mm_storeu_si128((__m128i*)(y + i), _mm256_cvtps_ph(a, _MM_FROUND_TO_NEAREST_INT));
        }
    }
#endif
    for (; i < n; ++i) y[i] = oracle_fp32_to_fp16(oracle_fp16_to_fp32(y[i]) * v);
}

/* VKQ16 = f16(fma(v_f16, vs, VKQ16)) elementwise */
static void mad_f16(int64_t n, uint16_t* y, const uint16_t* x, float v) {
    int64_t i = 0;
#if ORACLE_HAVE_SIMD
    if (g_use_simd) {
        const __m256 vv = _mm256_set1_ps(v);
        for (; i + 8 <= n; i += 8) {
            const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + i)));
            __m256 b = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(y + i)));
            b = _mm256_fmadd_ps(a, vv, b);
            _mm_storeu_si128((__m128i*)(y + i), _mm256_cvtps_ph(b, _MM_FROUND_TO_NEAREST_INT));
        }
    }
#endif
    for (; i < n; ++i) y[i] = oracle_fp32_to_fp16(fmaf(oracle_fp16_to_fp32(x[i]), v, oracle_fp16_to_fp32(y[i])));
}

static void f16_row_to_f32(const uint16_t* x, float* y, int64_t n) {
    int64_t i = 0;
#if ORACLE_HAVE_SIMD
    if (g_use_simd)
        for (; i + 8 <= n; i += 8)
            _mm256_storeu_ps(y + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + i))));
#endif
    for (; i < n; ++i) y[i] = oracle_fp16_to_fp32(x[i]);
}

static void scale_f32(int64_t n, float* y, float v) {
    for (int64_t i = 0; i < n; ++i) y[i] *= v;
}

static void mad_f32(int64_t n, float* y, const float* x, float v) {
    int64_t i = 0;
#if ORACLE_HAVE_SIMD
    if (g_use_simd) {
        const __m256 vv = _mm256_set1_ps(v);
        for (; i + 8 <= n; i += 8)
            _mm256_storeu_ps(y + i, _mm256_fmadd_ps(_mm256_loadu_ps(x + i), vv, _mm256_loadu_ps(y + i)));
    }
#endif
    for (; i < n; ++i) y[i] = fmaf(x[i], v, y[i]);
}

static float dot_f16(int64_t n, const uint16_t* x, const uint16_t* y) {
#if ORACLE_HAVE_SIMD
    if (g_use_simd) return dot_f16_simd(n, x, y);
#endif
    return oracle_vec_dot_f16(n, x, y);
}

/* ------------------------------------------------------------------------------------
 * flash_attn_ext (ggml CPU one-row kernel restated; upstream ggml-cpu ops.cpp,
 * ggml_compute_forward_flash_attn_ext_f16_one_chunk).
 * ---------------------------------------------------------------------------------- */
static inline const uint8_t* vptr(const oracle_view* t, int64_t i1, int64_t i2, int64_t i3) {
    return (const uint8_t*)t->data + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
}

static int valid_kv_type(int32_t t) { return t == ORACLE_F16 || t == ORACLE_Q8_0; }

int oracle_flash_attn_ext(const oracle_view* q, const oracle_view* k, const oracle_view* v,
                          const oracle_view* mask, float scale, float max_bias,
                          float logit_softcap, float* out, int v_acc_f16, int n_threads) {
    if (!q || !k || !v || !out) return -1;
    if (q->type != ORACLE_F32 || !valid_kv_type(k->type) || !valid_kv_type(v->type)) return -2;
    const int64_t DK = k->ne[0], DV = v->ne[0];
    const int64_t N = q->ne[1], H = q->ne[2], S = q->ne[3];
    const int64_t NKV = k->ne[1];
    if (q->ne[0] != DK || v->ne[1] != NKV) return -3;
    if (H % k->ne[2] || H % v->ne[2] || S % k->ne[3] || S % v->ne[3]) return -3;
    if ((k->type == ORACLE_Q8_0 && DK % QK8_0) || (v->type == ORACLE_Q8_0 && DV % QK8_0)) return -3;
    if (mask) {
        if (mask->type != ORACLE_F16 || mask->ne[0] < NKV || mask->ne[1] < N) return -4;
        if (H % mask->ne[2] || S % mask->ne[3]) return -4;
    }
    const int64_t rk2 = H / k->ne[2], rk3 = S / k->ne[3];
    const int64_t rv2 = H / v->ne[2], rv3 = S / v->ne[3];

    if (logit_softcap != 0.0f) scale /= logit_softcap;
    const uint32_t n_head = (uint32_t)H;
    uint32_t n_head_log2 = 1;
    while (n_head_log2 * 2 <= n_head) n_head_log2 *= 2;
    const float m0 = powf(2.0f, -(max_bias) / (float)n_head_log2);
    const float m1 = powf(2.0f, -(max_bias / 2.0f) / (float)n_head_log2);

    const int64_t n_rows = S * H * N;
    const int use_f16_acc = (v->type == ORACLE_F16) && v_acc_f16;
    int nt = 1;
#ifdef _OPENMP
    nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#else
    (void)n_threads;
#endif

#ifdef _OPENMP
#pragma omp parallel num_threads(nt)
#endif
    {
        float* VKQ32 = (float*)malloc(sizeof(float) * (size_t)DV);
        float* V32 = (float*)malloc(sizeof(float) * (size_t)DV);
        uint16_t* VKQ16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)DV);
        float* qrow = (float*)malloc(sizeof(float) * (size_t)DK);
        void* Qq = malloc((size_t)DK * 2 + 64);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
        for (int64_t ir = 0; ir < n_rows; ++ir) {
            const int64_t iq3 = ir / (H * N);
            const int64_t iq2 = (ir - iq3 * H * N) / N;
            const int64_t iq1 = ir - iq3 * H * N - iq2 * N;
            const uint32_t h = (uint32_t)iq2;
            const float slope = (max_bias > 0.0f)
                ? (h < n_head_log2 ? powf(m0, (float)(h + 1)) : powf(m1, (float)(2 * (h - n_head_log2) + 1)))
                : 1.0f;
            float Ssum = 0.0f;
            float M = -INFINITY;
            if (use_f16_acc) memset(VKQ16, 0, sizeof(uint16_t) * (size_t)DV);
            else memset(VKQ32, 0, sizeof(float) * (size_t)DV);

            const uint16_t* mp = mask
                ? (const uint16_t*)((const uint8_t*)mask->data + iq1 * mask->nb[1] +
                                    (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3])
                : NULL;
            const int64_t ik2 = iq2 / rk2, ik3 = iq3 / rk3;
            const int64_t iv2 = iq2 / rv2, iv3 = iq3 / rv3;

            /* Q row (f32, element stride nb[0]) converted to K's dot type */
            const uint8_t* pq = vptr(q, iq1, iq2, iq3);
            for (int64_t d = 0; d < DK; ++d) memcpy(&qrow[d], pq + d * q->nb[0], 4);
            if (k->type == ORACLE_F16) oracle_fp32_to_fp16_row(qrow, (uint16_t*)Qq, DK);
            else oracle_quantize_row_q8_0(qrow, Qq, DK);

            for (int64_t ic = 0; ic < NKV; ++ic) {
                const float mv = mp ? slope * oracle_fp16_to_fp32(mp[ic]) : 0.0f;
                if (mv == -INFINITY) continue;
                const uint8_t* kd = vptr(k, ic, ik2, ik3);
                float s = (k->type == ORACLE_F16)
                    ? dot_f16(DK, (const uint16_t*)kd, (const uint16_t*)Qq)
                    : oracle_vec_dot_q8_0(DK, kd, Qq);
                s = s * scale;
                if (logit_softcap != 0.0f) s = logit_softcap * tanhf(s);
                s += mv;
                const float Mold = M;
                float ms = 1.0f, vs = 1.0f;
                const uint8_t* vd = vptr(v, ic, iv2, iv3);
                if (use_f16_acc) {
                    if (s > M) {
                        M = s;
                        ms = expf(Mold - M);
                        scale_f16(DV, VKQ16, ms);
                    } else {
                        vs = expf(s - M);
                    }
                    mad_f16(DV, VKQ16, (const uint16_t*)vd, vs);
                } else {
                    if (s > M) {
                        M = s;
                        ms = expf(Mold - M);
                        scale_f32(DV, VKQ32, ms);
                    } else {
                        vs = expf(s - M);
                    }
                    if (v->type == ORACLE_F16) f16_row_to_f32((const uint16_t*)vd, V32, DV);
                    else oracle_dequantize_row_q8_0(vd, V32, DV);
                    mad_f32(DV, VKQ32, V32, vs);
                }
                Ssum = Ssum * ms + vs;
            }
            if (use_f16_acc) f16_row_to_f32(VKQ16, VKQ32, DV);
            const float S_inv = (Ssum == 0.0f) ? 0.0f : 1.0f / Ssum;
            float* dst = out + ((iq3 * N + iq1) * H + iq2) * DV;
            for (int64_t d = 0; d < DV; ++d) dst[d] = VKQ32[d] * S_inv;
        }
        free(VKQ32);
        free(V32);
        free(VKQ16);
        free(qrow);
        free(Qq);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------
 * llama-style KQ mask for a stream-major multi-sequence batch
 * (src/core/core_execution.cpp:2047-2062 positions N_s + j, one seq id per stream).
 * ---------------------------------------------------------------------------------- */
int oracle_build_kq_mask(uint16_t* mask, int64_t n_kv, int64_t n_q_pad, int64_t S,
                         const int32_t* kv_len, const int32_t* q_len, int causal) {
    const uint16_t NEG_INF = 0xfc00u;
    for (int64_t s = 0; s < S; ++s) {
        const int64_t L = kv_len[s], Q = q_len[s];
        if (L < 0 || Q < 0 || L + Q > n_kv || Q > n_q_pad) return -1;
        for (int64_t j = 0; j < n_q_pad; ++j) {
            uint16_t* row = mask + (s * n_q_pad + j) * n_kv;
            for (int64_t i = 0; i < n_kv; ++i) {
                int vis = (j < Q) && (i < L + Q) && (!causal || i <= L + j);
                row[i] = vis ? 0u : NEG_INF;
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------
 * PCG32 XSH-RR (O'Neill's published pcg32; the reference's DeterministicRng at
 * src/core/core_execution.cpp:33-62 is the same generator) and Box-Muller normals.
 * ---------------------------------------------------------------------------------- */
uint32_t oracle_pcg32_next(oracle_pcg32* r) {
    const uint64_t old = r->state;
    r->state = old * 6364136223846793005ULL + r->inc;
    const uint32_t xs = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    const uint32_t rot = (uint32_t)(old >> 59u);
    return (xs >> rot) | (xs << ((0u - rot) & 31u));
}

void oracle_pcg32_seed(oracle_pcg32* r, uint64_t seed, uint64_t seq) {
    r->state = 0u;
    r->inc = (seq << 1u) | 1u;
    (void)oracle_pcg32_next(r);
    r->state += seed;
    (void)oracle_pcg32_next(r);
}

double oracle_pcg32_uniform01(oracle_pcg32* r) {
    const uint64_t hi = oracle_pcg32_next(r);
    const uint64_t lo = oracle_pcg32_next(r);
    return (double)(((hi << 32) | lo) >> 11) * (1.0 / 9007199254740992.0);
}

void oracle_fill_normal_f32(uint64_t seed, uint64_t seq, float mul, float* out, int64_t n) {
    oracle_pcg32 r;
    oracle_pcg32_seed(&r, seed, seq);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = oracle_pcg32_uniform01(&r);
        const double u2 = oracle_pcg32_uniform01(&r);
        if (u1 < 1e-300) u1 = 1e-300;
        const double rad = sqrt(-2.0 * log(u1));
        out[i] = (float)(rad * cos(two_pi * u2) * (double)mul);
        if (i + 1 < n) out[i + 1] = (float)(rad * sin(two_pi * u2) * (double)mul);
    }
}

/* ---------------------------------------------------------------------------------------
 * Gated-delta-rule recurrent verify: GdnOperator::step_token (src/core/core_execution.cpp:
 * 254-335) for every row of every stream.  Per group g and state row h:
 *   sk = sum_s S[h][s] k[s] (serial, :314-317), delta = beta (v[h] - sk) (:318),
 *   S[h][s] = alpha S[h][s] + delta k[s], y[h] = sum_s S[h][s] q[s] (:319-329).
 * The state kept is the one after snap rows: a copy is taken when that row is reached. */
void oracle_gdn_verify(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                       float* state, float* y, int64_t S, int64_t n_rows, int64_t G, int64_t K, int64_t HD,
                       const int32_t* q_len, const int32_t* snap, int decay_first) {
    float* work = (float*)malloc((size_t)(G * HD * K) * sizeof(float));
    if (!work) return;
    for (int64_t s = 0; s < S; ++s) {
        int64_t ql = q_len ? q_len[s] : n_rows;
        ql = ql < 0 ? 0 : (ql > n_rows ? n_rows : ql);
        int64_t sn = snap ? snap[s] : ql;
        sn = sn < 0 ? 0 : (sn > ql ? ql : sn);
        float* st = state + s * G * HD * K;
        memcpy(work, st, (size_t)(G * HD * K) * sizeof(float));
        for (int64_t t = 0; t < ql; ++t) {
            const int64_t row = s * n_rows + t;
            for (int64_t g = 0; g < G; ++g) {
                const float* qg = q + (row * G + g) * K;
                const float* kg = k + (row * G + g) * K;
                const float* vg = v + (row * G + g) * HD;
                const float a = alpha[row * G + g], b = beta[row * G + g];
                float* yg = y + (row * G + g) * HD;
                for (int64_t h = 0; h < HD; ++h) {
                    float* rs = work + (g * HD + h) * K;
                    float sk = 0.0f;
                    for (int64_t c = 0; c < K; ++c) sk += rs[c] * kg[c];
                    if (decay_first) sk *= a;
                    const float delta = b * (vg[h] - sk);
                    float acc = 0.0f;
                    for (int64_t c = 0; c < K; ++c) {
                        const float upd = a * rs[c] + delta * kg[c];
                        rs[c] = upd;
                        acc += upd * qg[c];
                    }
                    yg[h] = acc;
                }
            }
            if (t + 1 == sn) memcpy(st, work, (size_t)(G * HD * K) * sizeof(float));
        }
    }
    free(work);
}
