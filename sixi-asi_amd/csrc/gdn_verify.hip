// gdn_verify.hip -- the gated-delta-rule recurrent verify: q_len[s] tokens of every stream
// through that stream's state of one linear-attention layer, in one launch.
//
// Per token, per group g and state row h (src/core/core_execution.cpp:254-335, the reference's
// GdnOperator::step_token; src/cuda/sixi_kernels.cu:241-281 is its CUDA twin):
//   sk = sum_s S[h][s] k[s]    (times alpha first with SIXI_GDN_DECAY_FIRST, ggml's order)
//   delta = beta * (v[h] - sk);   S[h][s] = alpha S[h][s] + delta k[s];   y[h] = sum_s S[h][s] q[s]
// The reference runs one launch per token and stream with the state in HBM; here one work-group
// owns the Hd x K state of one (stream, group) in registers for the whole block, so the state is
// read once and written once (at the snapshot row), and each token costs 3 Hd K FMAs on chip:
// the decay alpha goes into a scalar factor of the carried state (S = cs * st, below), not into
// every element.
//
// Two work-groups share each (stream, group), each owning half of the HD state rows (the rows
// update independently; q, k, alpha and beta are staged by both): 101 instead of 136 registers
// at 128 x 128, four waves per SIMD instead of three, so more work-groups' state loads overlap
// other work-groups' token steps (Qwen verify batch 79 -> 68 us; a four-way split measured
// slower).  The scalar factor took the element update from a multiply and an FMA to one FMA
// (65.2 -> 62.9 us) at the cost of 7 registers, i.e. of the fifth wave per SIMD.
//
// Mapping (256 threads): a thread holds R consecutive state rows x C = 16 consecutive columns;
// the TPR = K/16 lanes that share the rows form a row group (adjacent lanes), whose partial
// dot products are summed by DPP lane moves (ds_bpermute shuffles measured 94 against 83 us).  The block's tokens are staged through LDS TC at a
// time (q, k, v, alpha, beta of TC rows); every lane of a row group reads the same q/k columns,
// so those LDS reads are broadcasts.  y leaves from the row group's first lane as R floats.
//
// Roofline: the state dominates the bytes (2 * 4 Hd K per group and stream: read + write);
// each token adds 3 Hd K FMAs, so a block of n rows does 3n/8 FMA per state byte moved --
// a 16-row verify block is VALU-bound on gfx950's FP32 rate (packed FP32 is not used).
// Rounding differs from the step-by-step recurrence (S is cs * st, sums run over 16 columns
// then a lane tree) at the level of f32 rounding.
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
    if (a.K == 128 && a.HD == 128) return launch_shape<128, 128>(a, stream);
    if (a.K == 128 && a.HD == 64) return launch_shape<128, 64>(a, stream);
    if (a.K == 64 && a.HD == 128) return launch_shape<64, 128>(a, stream);
    if (a.K == 64 && a.HD == 64) return launch_shape<64, 64>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace sixi
