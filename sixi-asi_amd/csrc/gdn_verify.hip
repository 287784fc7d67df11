// gdn_verify.hip -- the gated-delta-rule recurrent verify: q_len[s] tokens of every stream
// through that stream's state of one linear-attention layer, in one launch.
//
// Per token, per group g and state row h (src/core/core_execution.cpp:254-335, the reference's
// GdnOperator::step_token; src/cuda/sixi_kernels.cu:241-281 is its CUDA twin):
//   sk = sum_s S[h][s] k[s]    (times alpha first with SIXI_GDN_DECAY_FIRST, ggml's order)
//   delta = beta * (v[h] - sk);   S[h][s] = alpha S[h][s] + delta k[s];   y[h] = sum_s S[h][s] q[s]
// The reference runs one launch per token and stream with the state in HBM; here the state of a
// (stream, group) is read once and written once (at the snapshot row), and a block of rows runs on
// chip.  Two kernels:
//
// gdn_verify_chunked_kernel (128-dim keys, states of 128 or 64 rows: the model's linear-attention
// layers hold 128 x 128) runs 16 rows at a time in the closed ("WY") form of the delta rule, on the f32 matrix
// cores; its comment below has the algebra and layout.  It is persistent: each work-group runs
// several (stream, group, 64-row half) items and reads half of the next item's state while it
// computes the current one.  Qwen verify batch (32 streams x 16 rows, 48 groups): 52.1-52.8 us
// against 64-65 us for the step by step kernel below; launching one item per work-group it
// measured 63.7 us (every work-group of a CU then loads, computes and stores in step), and without
// the XCD pairing of the two halves of a state 60.5 us.
//
// gdn_verify_kernel (64-dim keys) steps token by token on the VALU with the state in registers;
// the decay alpha goes into a scalar factor of the carried state (S = cs * st, below), not into
// every element.  Two work-groups share each (stream, group) when the state has 128 rows, each
// owning half of the rows (the rows update independently; q, k, alpha and beta are staged by
// both).  At 128 x 128 this form took 101 registers (four waves per SIMD) and 62.9 us on the
// Qwen verify batch (the scalar factor took the element update from a multiply and an FMA to one
// FMA: 65.2 -> 62.9 us).
//
// Mapping of gdn_verify_kernel (256 threads): a thread holds R consecutive state rows x C = 16
// consecutive columns; the TPR = K/16 lanes that share the rows form a row group (adjacent lanes),
// whose partial dot products are summed by DPP lane moves (ds_bpermute shuffles measured 94
// against 83 us).  The block's tokens are staged through LDS TC at a time (q, k, v, alpha, beta of
// TC rows); every lane of a row group reads the same q/k columns, so those LDS reads are
// broadcasts.  y leaves from the row group's first lane as R floats.
//
// Roofline: the state dominates the bytes (2 * 4 Hd K per group and stream: read + write); each
// row adds 3 Hd K FMAs, so a block of n rows does 3n/8 FMA per state byte moved -- 6 FMA per byte
// for a 16-row verify block: above the 4.9 FMA per HBM byte of the unpacked FP32 VALU (78.6
// TFLOP/s against 8 TB/s), below the 9.8 of the f32 matrix cores (157.3 TFLOP/s).  Rounding differs from the step by
// step recurrence (sums in another order, the scalar factor, the closed form) at the level of f32
// rounding.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gdn_internal.hpp"

namespace sixi {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kC = 16;   // state columns per thread
constexpr int kTC = 16;  // tokens staged per pass

// SPLIT work-groups share the HD rows of one (stream, group) state: the delta rule updates
// every row from its own values and the shared k, q, so the rows are independent.
template <int K, int HD, int SPLIT>
struct GdnShape {
    static constexpr int TPR = K / kC;         // lanes per row group
    static constexpr int GROUPS = 256 / TPR;   // row groups per block
    static constexpr int R = HD / SPLIT / GROUPS;  // state rows per thread
    static_assert(R >= 1 && GROUPS * R * SPLIT == HD, "shape");
};

// DPP lane moves (GFX9 encodings): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror (lane i of
// each 8-lane half-row reads lane 7 - i)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the TPR (4 or 8) adjacent lanes of a row group, the total in every lane of it: two quad
// swaps give each quad its sum, and for 8 lanes the half-row mirror adds the other quad's.
template <int TPR>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(TPR == 4 || TPR == 8, "row groups of 4 or 8 lanes");
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    if constexpr (TPR == 8) v += dpp<0x141>(v);
    return v;
}

template <int K, int HD, int SPLIT, bool DECAY_FIRST>
__global__ __launch_bounds__(256) void gdn_verify_kernel(GdnArgs a) {
    using Sh = GdnShape<K, HD, SPLIT>;
    constexpr int R = Sh::R, TPR = Sh::TPR;
    constexpr int HR = HD / SPLIT;  // state rows of this work-group
    __shared__ f32x4 lq[kTC][K / 4], lk[kTC][K / 4];
    __shared__ float lv[kTC][HR], la[kTC], lb[kTC];

    const int g = (int)((blockIdx.x / SPLIT) % (unsigned)a.G);
    const int s = (int)((blockIdx.x / SPLIT) / (unsigned)a.G);
    const int hr0 = (int)(blockIdx.x % SPLIT) * HR;  // first state row of the work-group
    const int tid = threadIdx.x;
    const int part = tid % TPR;           // column block: columns part*16 .. part*16+15
    const int rw = (tid / TPR) * R;       // first state row of the thread, in the work-group's rows
    const int row0 = hr0 + rw;            // ... in the state
    int ql = a.q_len ? a.q_len[s] : a.n_rows;
    ql = ql < 0 ? 0 : (ql > a.n_rows ? a.n_rows : ql);
    int snap = a.snap ? a.snap[s] : ql;
    snap = snap < 0 ? 0 : (snap > ql ? ql : snap);

    // The state is carried as S = cs * st: a token's decay multiplies the scalar cs (the same in
    // every lane) instead of every element, and the element update is st += (delta / cs) k^T --
    // one FMA per element instead of a multiply and an FMA.  A token that takes cs outside
    // [2^-30, 2^30] (a gate near 0 or above 1, or not finite) folds it into st first.
    float st[R][kC];
    float cs = 1.0f;
    const char* sin_base = a.s_in + (int64_t)g * a.si_nb2 + (int64_t)s * a.si_nb3 + part * kC * 4;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < kC / 4; ++u) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(sin_base + (int64_t)(row0 + r) * a.si_nb1 + 16 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) st[r][4 * u + e] = x[e];
        }
    char* sout_base = a.s_out + (int64_t)g * a.so_nb2 + (int64_t)s * a.so_nb3 + part * kC * 4;
    auto write_state = [&]() {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int u = 0; u < kC / 4; ++u)
                *reinterpret_cast<f32x4*>(sout_base + (int64_t)(row0 + r) * a.so_nb1 + 16 * u) =
                    f32x4{st[r][4 * u], st[r][4 * u + 1], st[r][4 * u + 2], st[r][4 * u + 3]} * cs;
    };
    if (snap == 0) write_state();

    for (int t0 = 0; t0 < ql; t0 += kTC) {
        const int nt = ql - t0 < kTC ? ql - t0 : kTC;
        // stage q, k (K/4 vectors per row), v (HD/4), alpha, beta of rows t0 .. t0+nt-1
        for (int i = tid; i < nt * (K / 4); i += 256) {
            const int t = i / (K / 4), c = i % (K / 4);
            const int64_t off = (int64_t)g * a.q_nb1 + (int64_t)(t0 + t) * a.q_nb2 + (int64_t)s * a.q_nb3 + 16 * c;
            lq[t][c] = *reinterpret_cast<const f32x4*>(a.q + off);
            const int64_t offk = (int64_t)g * a.k_nb1 + (int64_t)(t0 + t) * a.k_nb2 + (int64_t)s * a.k_nb3 + 16 * c;
            lk[t][c] = *reinterpret_cast<const f32x4*>(a.k + offk);
        }
        for (int i = tid; i < nt * (HR / 4); i += 256) {
            const int t = i / (HR / 4), c = i % (HR / 4);
            const f32x4 x = *reinterpret_cast<const f32x4*>(a.v + (int64_t)g * a.v_nb1 + (int64_t)(t0 + t) * a.v_nb2 +
                                                            (int64_t)s * a.v_nb3 + 4 * hr0 + 16 * c);
#pragma unroll
            for (int e = 0; e < 4; ++e) lv[t][4 * c + e] = x[e];
        }
        if (tid < nt) {
            la[tid] = *reinterpret_cast<const float*>(a.alpha + (int64_t)g * a.a_nb0 + (int64_t)(t0 + tid) * a.a_nb1 +
                                                      (int64_t)s * a.a_nb2);
            lb[tid] = *reinterpret_cast<const float*>(a.beta + (int64_t)g * a.b_nb0 + (int64_t)(t0 + tid) * a.b_nb1 +
                                                      (int64_t)s * a.b_nb2);
        }
        __syncthreads();
#pragma unroll 1
        for (int t = 0; t < nt; ++t) {
            float kv[kC], qv[kC];
#pragma unroll
            for (int u = 0; u < kC / 4; ++u) {
                const f32x4 x = lk[t][part * (kC / 4) + u];
#pragma unroll
                for (int e = 0; e < 4; ++e) kv[4 * u + e] = x[e];
            }
            const float al = la[t], be = lb[t];
            // the factor after the token's decay; outside [2^-30, 2^30] (or not finite) the token
            // folds it into st and the factor returns to 1 (the same in every lane)
            const float cn = cs * al;
            const bool fold = !(cn >= 0x1p-30f && cn <= 0x1p30f);
            // S k with the state before the token (decayed first: after it)
            float sk[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float x = 0.0f;
#pragma unroll
                for (int c = 0; c < kC; ++c) x += st[r][c] * kv[c];
                sk[r] = group_sum<TPR>(x) * (DECAY_FIRST ? cn : cs);
            }
            if (fold) {
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int c = 0; c < kC; ++c) st[r][c] *= cn;
            }
            cs = fold ? 1.0f : cn;
            const float bi = be / cs;
            // (q is read once the fold is done: fewer registers live across it)
#pragma unroll
            for (int u = 0; u < kC / 4; ++u) {
                const f32x4 y = lq[t][part * (kC / 4) + u];
#pragma unroll
                for (int e = 0; e < 4; ++e) qv[4 * u + e] = y[e];
            }
            float yo[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float dn = bi * (lv[t][rw + r] - sk[r]);
                float yv = 0.0f;
#pragma unroll
                for (int c = 0; c < kC; ++c) {
                    st[r][c] = fmaf(dn, kv[c], st[r][c]);
                    yv += st[r][c] * qv[c];
                }
                yo[r] = group_sum<TPR>(yv) * cs;
            }
            if (part == 0) {
                char* yp = a.y + (int64_t)g * a.y_nb1 + (int64_t)(t0 + t) * a.y_nb2 + (int64_t)s * a.y_nb3 + row0 * 4;
                if constexpr (R == 4)
                    *reinterpret_cast<f32x4*>(yp) = f32x4{yo[0], yo[1], yo[2], yo[3]};
                else
#pragma unroll
                    for (int r = 0; r < R; ++r) reinterpret_cast<float*>(yp)[r] = yo[r];
            }
            if (t0 + t + 1 == snap) write_state();
        }
        __syncthreads();  // the next pass overwrites the staged rows
    }
}

// ---------------------------------------------------------------------------------------------
// Chunked form on the f32 matrix cores (128-dim keys).  Over a chunk of T = 16 rows the T steps
// of the recurrence are one closed form (the "WY" / "UT" form of the delta rule; every quantity
// below is exact in exact arithmetic, the step by step loop is the definition):
//   A_t = alpha_0 ... alpha_t,   E[t][s] = alpha_{s+1} ... alpha_t (s <= t, 1 at s = t)
//   P = S0 k^T, Z = S0 q^T       (S0 the state before the chunk; P, Z are Hd x T)
//   c_t = A_{t-1} (A_{-1} = 1), or A_t when the decay comes first (ggml's order)
//   L[t][s] = beta_t e(t, s) (k_s . k_t) for s < t, e(t, s) = E[t-1][s] (E[t][s] decay-first)
//   R[h][t] = beta_t (v_t[h] - c_t P[h][t]);  U = R (I + L)^-T  (U[h][t] is token t's delta)
//   y_t[h] = A_t Z[h][t] + sum_{s<=t} U[h][s] E[t][s] (k_s . q_t)
//   S_sigma = A_sigma S0 + sum_{s<=sigma} E[sigma][s] U[:, s] k_s^T
// so a chunk costs the products P and Z (Hd x 128 by 128 x 16 each), one Hd x 16 by 16 x 128
// product per state it writes or carries, k k^T and k q^T (16 x 128 by 128 x 16, shared by the
// work-group) and 16 x 16 work -- the step by step form's 3 Hd K FMAs per row, on the matrix cores
// at twice the unpacked VALU rate.  No gate product spans more than one chunk (the carried state
// is the plain matrix), so the gates' range is that of the step by step recurrence.
//
// Layout: a work-group owns 64 state rows (HD / 64 work-groups per state), wave w rows 16w ..
// 16w+15.  v_mfma_f32_16x16x4f32: lane l supplies A[l%16][l/16] and B[l/16][l%16] and holds
// D[4(l/16) + r][l%16] in register r.  Lane l = 16 gl + lr holds state row lr of its wave, columns
// 16 m + 4 gl + j in register 4 m + j (m = 0..7, j = 0..3): read as eight 16-byte pieces, and at the
// same time the B operand of P^T = k S0^T (k-index 16 m + 4 gl + j at step (m, j)) and the output
// layout of S^T = k^T U'^T whose tile m covers columns 16 m .. 16 m + 15 -- so the state never
// leaves registers between chunks.
constexpr int kCT = 16;    // rows per chunk
constexpr int kCP = 132;   // LDS pitch (floats) of staged k, q rows: 16-byte reads of 8 rows hit distinct banks

__device__ __forceinline__ f32x4 mma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int HD, bool DECAY_FIRST>
__global__ __launch_bounds__(256) void gdn_verify_chunked_kernel(GdnArgs a, int n_items, int pair) {
    constexpr int K = 128, HR = 64, SPLIT = HD / HR, T = kCT;
    static_assert(HD % HR == 0, "64 state rows per work-group");
    __shared__ __align__(16) float lk[T][kCP], lq[T][kCP];
    __shared__ __align__(16) float lv[T][HR];
    __shared__ __align__(16) float la[T], lb[T];
    __shared__ __align__(16) float lE[T][T];          // E[t][s], 0 for s > t
    __shared__ __align__(16) float lred[4][2][T][T];  // per wave: partial k k^T, k q^T over 32 columns
    __shared__ __align__(16) float lLT[T][T];         // lLT[s][t] = L[t][s]
    __shared__ __align__(16) float lWT[T][T];         // lWT[t][s] = E[t][s] (k_s . q_t)

    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gl0 = (tid >> 4) & 3;  // the lane's group: columns 16 m + 4 gl0 .. + 3 of its state row
    // Work item x = 64 rows of one (stream, group) state.  With pair set (two items per state,
    // states a multiple of 8) items x and x + 8 are the two halves of one state: launched
    // round-robin over the 8 XCDs by work-groups b and b + 8, they share the XCD's L2 for the
    // state's q and k rows.
    auto locate = [&](int x, int& g, int& s, int& hr0) {
        int state, half;
        if (pair) {
            state = ((x >> 3) >> 1) * 8 + (x & 7);
            half = (x >> 3) & 1;
        } else {
            state = x / SPLIT;
            half = x % SPLIT;
        }
        g = state % a.G;
        s = state / a.G;
        hr0 = half * HR;
    };
    auto load_state = [&](int x, float (&dst)[32]) {
        int g, s, hr0;
        locate(x, g, s, hr0);
        const char* p = a.s_in + (int64_t)g * a.si_nb2 + (int64_t)s * a.si_nb3 +
                        (int64_t)(hr0 + 16 * wv + (tid & 15)) * a.si_nb1 + 16 * gl0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const f32x4 v4 = *reinterpret_cast<const f32x4*>(p + 64 * m);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[4 * m + j] = v4[j];
        }
    };
    // columns 16 m0 .. 16 m0 + 63 of item x's state rows (registers 4 m0 .. 4 m0 + 15 of st)
    auto load_half = [&](int x, int m0, float* dst) {
        int g, s, hr0;
        locate(x, g, s, hr0);
        const char* p = a.s_in + (int64_t)g * a.si_nb2 + (int64_t)s * a.si_nb3 +
                        (int64_t)(hr0 + 16 * wv + (tid & 15)) * a.si_nb1 + 16 * gl0;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const f32x4 v4 = *reinterpret_cast<const f32x4*>(p + 64 * (m0 + m));
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[4 * m + j] = v4[j];
        }
    };

    // A work-group runs items blockIdx.x, + gridDim.x, ...: the first half of the next item's state
    // (columns 0 .. 63) is read into nst while this item's chunks run, so a work-group's state
    // transfers overlap its own matrix-core work (launched one item per work-group, all of a CU's
    // work-groups load, compute and store in step: 63.7 against 55 us on the verify batch).  The
    // other half is read at the item's start: registers for all of it (148 VGPRs) leave three
    // work-groups per CU, with half of it (125) four fit (54.5 -> 52.8 us).
    float st[32], nst[16];
    load_state(blockIdx.x, st);
    bool first = true;
    for (int x = blockIdx.x; x < n_items; x += gridDim.x) {
        if (!first) load_half(x, 4, st + 16);  // the half not read ahead
        first = false;
        int g, s, hr0;
        locate(x, g, s, hr0);
        const int xn = x + (int)gridDim.x;
        const int h = hr0 + 16 * wv + (tid & 15);  // this lane's state row
        int ql = a.q_len ? a.q_len[s] : a.n_rows;
        ql = ql < 0 ? 0 : (ql > a.n_rows ? a.n_rows : ql);
        int snap = a.snap ? a.snap[s] : ql;
        snap = snap < 0 ? 0 : (snap > ql ? ql : snap);

        char* const sout = a.s_out + (int64_t)g * a.so_nb2 + (int64_t)s * a.so_nb3 + (int64_t)h * a.so_nb1 + 16 * gl0;
        if (snap == 0) {
#pragma unroll
            for (int m = 0; m < 8; ++m)
                *reinterpret_cast<f32x4*>(sout + 64 * m) =
                    f32x4{st[4 * m], st[4 * m + 1], st[4 * m + 2], st[4 * m + 3]};
        }
        if (ql == 0 && xn < n_items) load_half(xn, 0, nst);

        for (int t0 = 0; t0 < ql; t0 += T) {
            const int nt = ql - t0 < T ? ql - t0 : T;
            // the lane's LDS addresses and constants are derived anew in every chunk (an opaque copy
            // of the thread index): hoisted out of the loop they would hold some 60 VGPRs
            int tx;
            asm volatile("v_mov_b32 %0, %1" : "=v"(tx) : "v"(tid));
            const int lr = tx & 15, gl = (tx >> 4) & 3, hw = 16 * wv + lr;
            // stage rows t0 .. t0+nt-1; rows past nt are zero keys, queries and values with gate 1 and
            // beta 0, which leave the state and every other row's result unchanged
            for (int i = tx; i < T * (K / 4); i += 256) {
                const int t = i / (K / 4), c = i % (K / 4);
                f32x4 kx = {0.0f, 0.0f, 0.0f, 0.0f}, qx = kx;
                if (t < nt) {
                    kx = *reinterpret_cast<const f32x4*>(a.k + (int64_t)g * a.k_nb1 + (int64_t)(t0 + t) * a.k_nb2 +
                                                         (int64_t)s * a.k_nb3 + 16 * c);
                    qx = *reinterpret_cast<const f32x4*>(a.q + (int64_t)g * a.q_nb1 + (int64_t)(t0 + t) * a.q_nb2 +
                                                         (int64_t)s * a.q_nb3 + 16 * c);
                }
                *reinterpret_cast<f32x4*>(&lk[t][4 * c]) = kx;
                *reinterpret_cast<f32x4*>(&lq[t][4 * c]) = qx;
            }
            for (int i = tx; i < T * (HR / 4); i += 256) {
                const int t = i / (HR / 4), c = i % (HR / 4);
                f32x4 vx = {0.0f, 0.0f, 0.0f, 0.0f};
                if (t < nt)
                    vx = *reinterpret_cast<const f32x4*>(a.v + (int64_t)g * a.v_nb1 + (int64_t)(t0 + t) * a.v_nb2 +
                                                         (int64_t)s * a.v_nb3 + 4 * hr0 + 16 * c);
                *reinterpret_cast<f32x4*>(&lv[t][4 * c]) = vx;
            }
            if (tx < T) {
                const int64_t ra = (int64_t)g * a.a_nb0 + (int64_t)(t0 + tx) * a.a_nb1 + (int64_t)s * a.a_nb2;
                const int64_t rb = (int64_t)g * a.b_nb0 + (int64_t)(t0 + tx) * a.b_nb1 + (int64_t)s * a.b_nb2;
                la[tx] = tx < nt ? *reinterpret_cast<const float*>(a.alpha + ra) : 1.0f;
                lb[tx] = tx < nt ? *reinterpret_cast<const float*>(a.beta + rb) : 0.0f;
            }
            __syncthreads();
            if (t0 == 0 && xn < n_items) load_half(xn, 0, nst);  // in flight during this item's work

            // E[t][s], one entry per thread, multiplied in row order
            {
                const int et = tx >> 4, es = tx & 15;
                f32x4 a4[T / 4];  // every gate of the chunk (the same address in every lane)
#pragma unroll
                for (int u = 0; u < T / 4; ++u) a4[u] = *reinterpret_cast<const f32x4*>(&la[4 * u]);
                float e = 1.0f;
#pragma unroll
                for (int r = 1; r < T; ++r)
                    if (r > es && r <= et) e *= a4[r / 4][r % 4];
                lE[et][es] = es <= et ? e : 0.0f;
            }
            // P^T = k S0^T and Z^T = q S0^T (lane: P[h][4 gl + j] in register j); wave w also sums
            // k k^T and k q^T over columns 32 w .. 32 w + 31
            f32x4 pt = {0.0f, 0.0f, 0.0f, 0.0f}, zt = pt, gk = pt, gq = pt;
            // (raised wave priority while this wave issues the products: 55.0 -> 53.6-53.9 us on the
            // verify batch; raised around the state's product as well, 54.5 us)
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const f32x4 kx = *reinterpret_cast<const f32x4*>(&lk[lr][16 * m + 4 * gl]);
                const f32x4 qx = *reinterpret_cast<const f32x4*>(&lq[lr][16 * m + 4 * gl]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    pt = mma4(kx[j], st[4 * m + j], pt);
                    zt = mma4(qx[j], st[4 * m + j], zt);
                }
                if ((m >> 1) == wv) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        gk = mma4(kx[j], kx[j], gk);
                        gq = mma4(kx[j], qx[j], gq);
                    }
                }
            }
            __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                lred[wv][0][4 * gl + r][lr] = gk[r];  // k_{4gl+r} . k_lr, partial
                lred[wv][1][4 * gl + r][lr] = gq[r];  // k_{4gl+r} . q_lr, partial
            }
            __syncthreads();

            // L and W, one entry per thread: row ta, column tb
            {
                const int ta = tx >> 4, tb = tx & 15;
                const float kk = lred[0][0][tb][ta] + lred[1][0][tb][ta] + lred[2][0][tb][ta] + lred[3][0][tb][ta];
                const float kq = lred[0][1][tb][ta] + lred[1][1][tb][ta] + lred[2][1][tb][ta] + lred[3][1][tb][ta];
                float l = 0.0f;
                if (tb < ta) l = lb[ta] * (DECAY_FIRST ? lE[ta][tb] : lE[ta - 1][tb]) * kk;
                lLT[tb][ta] = l;                  // L[ta][tb]
                lWT[ta][tb] = lE[ta][tb] * kq;    // E[ta][tb] (k_tb . q_ta), 0 for tb > ta
            }
            __syncthreads();

            // row lr of M = (I + L)^-1 by back substitution: M[s][t] = [s = t] - sum_{r>t} M[s][r] L[r][t]
            // (row t - 1 of lLT is read while row t is used; the empty asm pins each step in place,
            // else the compiler reads all 36 pieces up front into 144 VGPRs)
            float mr[T];
            mr[T - 1] = lr == T - 1 ? 1.0f : 0.0f;
            f32x4 cur[T / 4], nxt[T / 4];
#pragma unroll
            for (int c = (T - 1) / 4; c < T / 4; ++c) cur[c] = *reinterpret_cast<const f32x4*>(&lLT[T - 2][4 * c]);
#pragma unroll
            for (int t = T - 2; t >= 0; --t) {
                if (t > 0) {
#pragma unroll
                    for (int c = t / 4; c < T / 4; ++c) nxt[c] = *reinterpret_cast<const f32x4*>(&lLT[t - 1][4 * c]);
                }
                float x = lr == t ? 1.0f : 0.0f;
#pragma unroll
                for (int c = (t + 1) / 4; c < T / 4; ++c)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (4 * c + e > t) x = fmaf(-mr[4 * c + e], cur[c][e], x);
                asm volatile("" : "+v"(x) : : "memory");
                mr[t] = x;
#pragma unroll
                for (int c = 0; c < T / 4; ++c) cur[c] = nxt[c];
            }
            // R[h][4 gl + j] and U^T = M R^T (lane: U[h][4 gl + j] in register j)
            const float a0 = la[0];
            f32x4 ut = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = 4 * gl + j;
                const float ct = DECAY_FIRST ? lE[t][0] * a0 : (t ? lE[t - 1][0] * a0 : 1.0f);
                const float rv = lb[t] * (lv[t][hw] - ct * pt[j]);
                const float mv = gl == 0 ? mr[j] : gl == 1 ? mr[4 + j] : gl == 2 ? mr[8 + j] : mr[12 + j];
                ut = mma4(mv, rv, ut);
            }
            // y^T = diag(A) Z^T + W^T U^T
            {
                f32x4 yt;
#pragma unroll
                for (int j = 0; j < 4; ++j) yt[j] = lE[4 * gl + j][0] * a0 * zt[j];
                const f32x4 wx = *reinterpret_cast<const f32x4*>(&lWT[lr][4 * gl]);
#pragma unroll
                for (int j = 0; j < 4; ++j) yt = mma4(wx[j], ut[j], yt);
                char* yp = a.y + (int64_t)g * a.y_nb1 + (int64_t)(t0 + 4 * gl) * a.y_nb2 + (int64_t)s * a.y_nb3 + h * 4;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (4 * gl + j < nt) *reinterpret_cast<float*>(yp + (int64_t)j * a.y_nb2) = yt[j];
            }
            // S_sigma = A_sigma S0 + k^T (U E[sigma])^T, tile by tile; written to the snapshot and/or
            // kept as the next chunk's S0
            const bool more = t0 + T < ql;
            const bool snap_here = snap > t0 && snap <= t0 + nt;
            auto advance = [&](int sig, bool write, bool keep) {
                const float as = lE[sig][0] * a0;
                float ub[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) ub[j] = ut[j] * lE[sig][4 * gl + j];
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    f32x4 acc = f32x4{st[4 * m], st[4 * m + 1], st[4 * m + 2], st[4 * m + 3]} * as;
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc = mma4(lk[4 * gl + j][16 * m + lr], ub[j], acc);
                    if (write) *reinterpret_cast<f32x4*>(sout + 64 * m) = acc;
                    if (keep) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) st[4 * m + j] = acc[j];
                    }
                }
            };
            if (snap_here) advance(snap - 1 - t0, true, more && snap == t0 + T);
            if (more && !(snap_here && snap == t0 + T)) advance(T - 1, false, true);
            if (more) __syncthreads();  // the next chunk overwrites the staged rows
        }
        __syncthreads();  // the next item overwrites the staged rows
#pragma unroll
        for (int i = 0; i < 16; ++i) st[i] = nst[i];
    }
}

// Work-groups of the chunked kernel that fit the device at once (each then runs several items).
template <int HD, bool DECAY_FIRST>
int chunked_resident_groups() {
    static int cached = -1;
    if (cached < 0) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gdn_verify_chunked_kernel<HD, DECAY_FIRST>, 256, 0) ==
                hipSuccess &&
            cus > 0 && per_cu > 0)
            cached = cus * per_cu;
        else
            cached = 0;  // unknown: one item per work-group
    }
    return cached;
}

template <int HD, bool DECAY_FIRST>
hipError_t launch_chunked_df(const GdnArgs& a, hipStream_t stream) {
    const int64_t items = (int64_t)a.S * a.G * (HD / 64);
    if (items > INT32_MAX) return hipErrorInvalidValue;
    const int resident = chunked_resident_groups<HD, DECAY_FIRST>();
    const int64_t groups = resident > 0 && resident < items ? resident : items;
    const int pair = HD == 128 && ((int64_t)a.S * a.G) % 8 == 0;
    hipLaunchKernelGGL((gdn_verify_chunked_kernel<HD, DECAY_FIRST>), dim3((unsigned)groups), dim3(256), 0, stream, a,
                       (int)items, pair);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_chunked(const GdnArgs& a, hipStream_t stream) {
    return a.decay_first ? launch_chunked_df<HD, true>(a, stream) : launch_chunked_df<HD, false>(a, stream);
}

template <int K, int HD, int SPLIT>
hipError_t launch_split(const GdnArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)((int64_t)a.S * a.G * SPLIT)), block(256);
    if (a.decay_first)
        hipLaunchKernelGGL((gdn_verify_kernel<K, HD, SPLIT, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((gdn_verify_kernel<K, HD, SPLIT, false>), grid, block, 0, stream, a);
    return hipGetLastError();
}
template <int K, int HD>
hipError_t launch_shape(const GdnArgs& a, hipStream_t stream) {
    if constexpr (HD / (256 / (K / kC)) >= 2) return launch_split<K, HD, 2>(a, stream);
    else return launch_split<K, HD, 1>(a, stream);
}

}  // namespace

hipError_t launch_gdn_verify(const GdnArgs& a, hipStream_t stream) {
    if ((int64_t)a.S * a.G == 0) return hipSuccess;
    if (a.K == 128 && a.HD == 128) return launch_chunked<128>(a, stream);
    if (a.K == 128 && a.HD == 64) return launch_chunked<64>(a, stream);
    if (a.K == 64 && a.HD == 128) return launch_shape<64, 128>(a, stream);
    if (a.K == 64 && a.HD == 64) return launch_shape<64, 64>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace sixi
