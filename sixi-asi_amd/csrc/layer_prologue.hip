// layer_prologue.hip -- the element-wise work of a Qwen3.8 full-attention layer that sits on
// either side of the attention op: the Q/K prologue (RMS norm, weight, RoPE) fused with the
// KV store, and the sigmoid output gate.
//
// Per row j of stream s (position p = kv_len[s] + j), following the graph upstream llama.cpp
// builds for the qwen35 architecture (configs/qwen3.8-27b-ud-q4-k-xl.sixi: heads of 256, 24
// q-heads, 4 kv-heads, eps 1e-6, 64 rotated dims, base 1e7), reached through every
// llama_decode of src/core/core_execution.cpp:2074, :3536 and :3811:
//   RMS norm   y = x * (1 / sqrt(mean(x^2) + eps)), then y * weight (ggml_rms_norm, ggml_mul);
//   RoPE       pairs (i, i + n_rot/2) for i < n_rot/2 (the NEOX pairing; the model's
//              multi-section form reduces to it for text, whose section positions are equal):
//                y_i = x_i cos t_i - x_{i+h} sin t_i,  y_{i+h} = x_i sin t_i + x_{i+h} cos t_i,
//              t_0 = p and t_{i+1} = t_i * theta_scale in f32, one product at a time, as
//              ggml's CPU rope cache forms them; dims >= n_rot pass unchanged;
//   K, V store K after norm and RoPE, V as given, into cell p of the stream's cache with the
//              codecs of kv_write.hip (f16 round to nearest even, or q8_0 blocks);
//   gate       out *= 1 / (1 + exp(-g)) (ggml_sigmoid, ggml_mul), g the second half of the
//              head's attn_q output.
//
// One block per (stream, row); a wave holds one head row at a time with D/64 consecutive
// elements per lane: the head's sum of squares and the q8_0 block maxima are wave shuffles,
// the RoPE partner of an element sits n_rot/2 elements away, in the same register of another
// lane, and each wave forms the row's cos/sin pairs once for all the heads it takes.
// Both kernels are HBM-bound byte work (f32 in, f32 or f16/q8_0 out) with no reuse.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "layer_internal.hpp"

namespace sixi {
namespace {

template <int E>
struct Vec;
template <>
struct Vec<2> {
    typedef float f __attribute__((ext_vector_type(2)));
};
template <>
struct Vec<4> {
    typedef float f __attribute__((ext_vector_type(4)));
};

template <int E>
__device__ __forceinline__ void load_row(const char* p, int lane, float (&x)[E]) {
    const typename Vec<E>::f v = *reinterpret_cast<const typename Vec<E>::f*>(p + (int64_t)lane * E * 4);
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = v[e];
}

template <int E>
__device__ __forceinline__ void store_row(char* p, int lane, const float (&x)[E]) {
    typename Vec<E>::f v;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = x[e];
    *reinterpret_cast<typename Vec<E>::f*>(p + (int64_t)lane * E * 4) = v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// RMS norm with weight, then RoPE on the first n_rot dims; c/s hold the cos/sin of the pairs
// of the lane's elements (whole wave, uniform control flow).
template <int E>
__device__ __forceinline__ void norm_rope(float (&x)[E], int lane, const float (&w)[E], float eps, int D, int n_rot,
                                          const float (&c)[E], const float (&sn)[E]) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += x[e] * x[e];
    ss = wave_sum(ss);
    const float mean = ss / (float)D;
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float y = x[e] * scale;
        x[e] = y * w[e];
    }
    if (n_rot == 0) return;
    const int lane_off = n_rot / 2 / E;  // lanes between an element and its partner
    const bool first = lane < lane_off;
    const bool rotated = lane < 2 * lane_off;
    const int partner = !rotated ? lane : (first ? lane + lane_off : lane - lane_off);
    float other[E];
#pragma unroll
    for (int e = 0; e < E; ++e) other[e] = __shfl(x[e], partner, 64);
    if (!rotated) return;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (first)
            x[e] = x[e] * c[e] - other[e] * sn[e];
        else
            x[e] = other[e] * sn[e] + x[e] * c[e];
    }
}

// cos/sin of the pairs of this lane's elements at position pos: lane p forms pairs p and p + 64
// (angle p * theta_scale^i, multiplied out one step at a time), then each lane gathers its own.
template <int E>
__device__ __forceinline__ void rope_angles(int lane, int n_rot, float theta_scale, float pos, float (&c)[E],
                                            float (&sn)[E]) {
    const int half = n_rot / 2;
    float c0 = 1.0f, s0 = 0.0f, c1 = 1.0f, s1 = 0.0f;
    if (lane < half) {
        float theta = pos;
        for (int i = 0; i < lane; ++i) theta *= theta_scale;
        sincosf(theta, &s0, &c0);
        if (lane + 64 < half) {
            for (int i = 0; i < 64; ++i) theta *= theta_scale;
            sincosf(theta, &s1, &c1);
        }
    }
    const int lane_off = half / E;
    const int i0 = (lane < lane_off ? lane : lane - lane_off) * E;  // first pair of the lane's elements
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = i0 + e;
        const float a0 = __shfl(c0, i & 63, 64), b0 = __shfl(s0, i & 63, 64);
        const float a1 = __shfl(c1, i & 63, 64), b1 = __shfl(s1, i & 63, 64);
        c[e] = i < 64 ? a0 : a1;
        sn[e] = i < 64 ? b0 : b1;
    }
}

template <int E>
__device__ __forceinline__ void store_f16(char* row, int lane, const float (&x)[E]) {
    _Float16 h[E];
#pragma unroll
    for (int e = 0; e < E; ++e) h[e] = (_Float16)x[e];
    if constexpr (E == 4) {
        uint32_t w0 = (uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16);
        uint32_t w1 = (uint32_t)__builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16);
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(row + lane * 8) = u32x2{w0, w1};
    } else {
        *reinterpret_cast<uint32_t*>(row + lane * 4) =
            (uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16);
    }
}

// q8_0 blocks of 32 elements = 32/E lanes: d = amax/127 (f16), q = clamp(round(x * 127/amax))
template <int E>
__device__ __forceinline__ void store_q8(char* row, int lane, const float (&x)[E]) {
    constexpr int LB = 32 / E;  // lanes per block
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) am = fmaxf(am, fabsf(x[e]));
#pragma unroll
    for (int o = LB / 2; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 127.0f / am : 0.0f;
    const int t = lane % LB;
    char* blk = row + (lane / LB) * 34;
    if (t == 0) *reinterpret_cast<uint16_t*>(blk) = __builtin_bit_cast(uint16_t, (_Float16)d);
    uint16_t* qs = reinterpret_cast<uint16_t*>(blk + 2 + t * E);
#pragma unroll
    for (int e = 0; e < E; e += 2) {
        const int q0 = (int)fminf(fmaxf(roundf(x[e] * id), -127.0f), 127.0f);
        const int q1 = (int)fminf(fmaxf(roundf(x[e + 1] * id), -127.0f), 127.0f);
        qs[e / 2] = (uint16_t)((uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8));
    }
}

constexpr int kBatch = 8;  // head rows a wave loads before it computes

// One block of four waves per (stream, row).  Wave w takes the slots w, w+4, ... of the row
// (q-heads, k-heads, v-heads in that order), kBatch at a time.  The first batch is loaded
// before the row's q_len is read (every row of the view is in bounds; a row past q_len is
// dropped afterwards), and each wave forms the row's RoPE angles in its own registers while
// those loads are in flight: no LDS, no barrier.
template <int D, bool Q8>
__global__ __launch_bounds__(256) void qk_prologue(QkPrologueArgs a) {
    constexpr int E = D / 64;
    const int j = (int)(blockIdx.x % (unsigned)a.n_rows);
    const int s = (int)(blockIdx.x / (unsigned)a.n_rows);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar address math
    const int slots = a.H + 2 * a.Hkv;
    const char* qrow = a.qg + (int64_t)j * a.qg_nb2 + (int64_t)s * a.qg_nb3;
    const char* krow = a.k + (int64_t)j * a.k_nb2 + (int64_t)s * a.k_nb3;
    const char* vrow = a.v + (int64_t)j * a.v_nb2 + (int64_t)s * a.v_nb3;
    float x[kBatch][E], wq[E], wk[E];
    auto load_batch = [&](int first) {
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int slot = first + 4 * b;
            if (slot >= slots) break;
            const char* src = slot < a.H             ? qrow + (int64_t)slot * a.qg_nb1
                              : slot < a.H + a.Hkv ? krow + (int64_t)(slot - a.H) * a.k_nb1
                                                   : vrow + (int64_t)(slot - a.H - a.Hkv) * a.v_nb1;
            load_row<E>(src, lane, x[b]);
        }
    };
    const int64_t pos = (int64_t)(a.kv_len ? a.kv_len[s] : 0) + j;
    load_batch(wave);
    load_row<E>(reinterpret_cast<const char*>(a.q_norm), lane, wq);
    load_row<E>(reinterpret_cast<const char*>(a.k_norm), lane, wk);
    float c[E], sn[E];
    if (a.n_rot > 0) rope_angles<E>(lane, a.n_rot, a.theta_scale, (float)pos, c, sn);
    if (j >= (a.q_len ? a.q_len[s] : a.n_rows)) return;
    const bool in_cache = pos >= 0 && pos < a.n_cells;  // outside the stream's cells: not stored
    char* qo_row = a.q_out + (int64_t)j * a.qo_nb1 + (int64_t)s * a.qo_nb3;
    // the cell's rows: in the stream's range, or (paged) in its page
    int64_t page = s, cell = pos;
    if (a.pt && in_cache) {
        page = min(max(a.pt[(int64_t)s * a.pt_stride + (pos >> 8)], 0), a.n_pages - 1);
        cell = pos & 255;
    }
    char* kc_row = a.kc + cell * a.kc_nb1 + page * a.kc_nb3;
    char* vc_row = a.vc + cell * a.vc_nb1 + page * a.vc_nb3;
    // per batch: every row is computed before the first store, since a store in flight makes
    // the next load's wait a full drain (one counter covers loads and stores)
    for (int first = wave; first < slots; first += 4 * kBatch) {
        if (first != wave) load_batch(first);
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int slot = first + 4 * b;
            if (slot >= slots) break;
            if (slot < a.H)
                norm_rope<E>(x[b], lane, wq, a.eps, D, a.n_rot, c, sn);
            else if (slot < a.H + a.Hkv && in_cache)
                norm_rope<E>(x[b], lane, wk, a.eps, D, a.n_rot, c, sn);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int slot = first + 4 * b;
            if (slot >= slots) break;
            if (slot < a.H) {
                if (a.q_out_f16)
                    store_f16<E>(qo_row + (int64_t)slot * a.qo_nb2, lane, x[b]);
                else
                    store_row<E>(qo_row + (int64_t)slot * a.qo_nb2, lane, x[b]);
                continue;
            }
            if (!in_cache) continue;
            char* row = slot < a.H + a.Hkv ? kc_row + (int64_t)(slot - a.H) * a.kc_nb2
                                           : vc_row + (int64_t)(slot - a.H - a.Hkv) * a.vc_nb2;
            if constexpr (Q8)
                store_q8<E>(row, lane, x[b]);
            else
                store_f16<E>(row, lane, x[b]);
        }
    }
}

// One block of four waves per (stream, row); wave w gates heads w, w+4, ..., loading kBatch
// heads' output and gate rows before the first product.
template <int D>
__global__ __launch_bounds__(256) void attn_gate(AttnGateArgs a) {
    constexpr int E = D / 64;
    const int j = (int)(blockIdx.x % (unsigned)a.n_rows);
    const int s = (int)(blockIdx.x / (unsigned)a.n_rows);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    bool checked = false;
    for (int first = wave; first < a.H; first += 4 * kBatch) {
        float g[kBatch][E], o[kBatch][E];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int h = first + 4 * b;
            if (h >= a.H) break;
            load_row<E>(a.qg + (int64_t)h * a.g_nb1 + (int64_t)j * a.g_nb2 + (int64_t)s * a.g_nb3 + (int64_t)D * 4, lane,
                        g[b]);
            load_row<E>(a.out + (int64_t)h * a.o_nb1 + (int64_t)j * a.o_nb2 + (int64_t)s * a.o_nb3, lane, o[b]);
        }
        // the row's length is read once the first loads are in flight (every row is in bounds)
        if (!checked) {
            if (a.q_len && j >= a.q_len[s]) return;
            checked = true;
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            if (first + 4 * b >= a.H) break;
#pragma unroll
            for (int e = 0; e < E; ++e) o[b][e] = o[b][e] * (1.0f / (1.0f + expf(-g[b][e])));
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int h = first + 4 * b;
            if (h >= a.H) break;
            store_row<E>(a.out + (int64_t)h * a.o_nb1 + (int64_t)j * a.o_nb2 + (int64_t)s * a.o_nb3, lane, o[b]);
        }
    }
}

}  // namespace

hipError_t launch_qk_prologue(const QkPrologueArgs& a, hipStream_t stream) {
    const int64_t rows = (int64_t)a.S * a.n_rows;
    if (rows == 0 || a.H + 2 * a.Hkv == 0) return hipSuccess;
    const dim3 grid((unsigned)rows), block(256);
    if (a.D == 128) {
        if (a.cache_q8)
            hipLaunchKernelGGL((qk_prologue<128, true>), grid, block, 0, stream, a);
        else
            hipLaunchKernelGGL((qk_prologue<128, false>), grid, block, 0, stream, a);
    } else {
        if (a.cache_q8)
            hipLaunchKernelGGL((qk_prologue<256, true>), grid, block, 0, stream, a);
        else
            hipLaunchKernelGGL((qk_prologue<256, false>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

hipError_t launch_attn_gate(const AttnGateArgs& a, hipStream_t stream) {
    const int64_t rows = (int64_t)a.S * a.n_rows;
    if (rows == 0 || a.H == 0) return hipSuccess;
    const dim3 grid((unsigned)rows), block(256);
    if (a.D == 128)
        hipLaunchKernelGGL(attn_gate<128>, grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL(attn_gate<256>, grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace sixi
