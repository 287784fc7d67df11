// fa_q8_stage.hip -- q8_0 KV where no q8_0 kernel applies (256-dim heads: prefill chunks, and
// rows that are not 16-byte aligned): the operands are staged as f16 in the workspace and the
// f16 kernels run on them.
//
// The values are exactly the MFMA operands the q8_0 split-K kernels use (fa_decode.hip), so
// both paths compute ggml's q8_0 attention the same way:
//   K, V  f16(q * d) per element (one rounding; d is the block's f16 scale), written as dense
//         f16 rows [stream][cell][kv-head] of D elements;
//   Q     ggml's conversion of Q to K's dot type, q8_0 per 32-dim block (d = amax/127,
//         q = round-half-away(x * 127/amax) clamped to +-127, src/core/numeric.cpp:349-384),
//         entering the MFMA as f16(q * f16(d)); dense rows [stream][row][q-head].
// Only the cells a stream's rows can see are staged (kv_len + q_len, or every cell without
// lengths); the prefill kernel's range-checked loads never read past them.
//
// Both kernels move bytes (HBM-bound): one thread per 32-element block, a 34-byte q8_0 read
// (or a 128-byte f32 Q read) and a 64-byte f16 write.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "fa_internal.hpp"

namespace sixi {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// K (blocks 0 .. g-1) and V (blocks g .. 2g-1) in one launch
__global__ __launch_bounds__(256) void q8_kv_to_f16(Q8StageArgs a, unsigned g) {
    const int which = blockIdx.x >= g ? 1 : 0;
    const char* src = which ? a.v : a.k;
    const int64_t nb1 = which ? a.v_nb1 : a.k_nb1, nb2 = which ? a.v_nb2 : a.k_nb2, nb3 = which ? a.v_nb3 : a.k_nb3;
    char* dst = which ? a.v16 : a.k16;
    const int nb = a.D / 32;  // q8_0 blocks per head row
    const int64_t n = (int64_t)a.S * a.n_kv * a.Hkv * nb;
    const int64_t i = (int64_t)(blockIdx.x - (which ? g : 0u)) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int b = (int)(i % nb);
    int64_t r = i / nb;
    const int h = (int)(r % a.Hkv);
    r /= a.Hkv;
    const int64_t cell = r % a.n_kv;
    const int s = (int)(r / a.n_kv);
    int64_t nc = a.n_kv;
    if (a.kv_len) {
        const int64_t ql = a.q_len ? a.q_len[s] : a.n_q;
        int64_t kl = a.kv_len[s];
        kl = kl < 0 ? 0 : (kl > a.n_kv - ql ? a.n_kv - ql : kl);  // the attention's clamp
        nc = ql > 0 ? kl + ql : 0;
    }
    if (cell >= nc) return;
    // the cell's row: in its stream's range, or (paged) in its page
    int64_t row_off;
    if (a.pt) {
        const int page = min(max(a.pt[(int64_t)s * a.pt_stride + (cell >> 8)], 0), a.n_pages - 1);
        row_off = (int64_t)page * nb3 + (cell & (kPageCells - 1)) * nb1;
    } else {
        row_off = (int64_t)s * nb3 + cell * nb1;
    }
    // a q8_0 block is 34 bytes: the f16 scale, then 32 int8 quants (2-byte aligned)
    const uint16_t* blk = reinterpret_cast<const uint16_t*>(src + row_off + (int64_t)h * nb2 + b * 34);
    const float d = (float)__builtin_bit_cast(_Float16, blk[0]);
    u32x4* o = reinterpret_cast<u32x4*>(dst + ((((int64_t)s * a.n_kv + cell) * a.Hkv + h) * a.D + b * 32) * 2);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        f16x8 hv;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const uint16_t pair = blk[1 + (8 * u + e) / 2];
            hv[e] = (_Float16)((float)(int8_t)(pair & 0xff) * d);
            hv[e + 1] = (_Float16)((float)(int8_t)(pair >> 8) * d);
        }
        o[u] = __builtin_bit_cast(u32x4, hv);
    }
}

__global__ __launch_bounds__(256) void q8_q_to_f16(Q8StageArgs a) {
    const int nb = a.D / 32;
    const int64_t n = (int64_t)a.S * a.n_q * a.H * nb;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int b = (int)(i % nb);
    int64_t r = i / nb;
    const int h = (int)(r % a.H);
    r /= a.H;
    const int j = (int)(r % a.n_q);
    const int s = (int)(r / a.n_q);
    const char* p = a.q + (int64_t)j * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)s * a.q_nb3 + (int64_t)b * 32 * a.q_es;
    float x[32];
    if (a.q_f16) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f16x8 hv = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(p + 16 * u));
#pragma unroll
            for (int e = 0; e < 8; ++e) x[8 * u + e] = (float)hv[e];
        }
    } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(p + 16 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * u + e] = v[e];
        }
    }
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) am = fmaxf(am, fabsf(x[e]));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 127.0f / am : 0.0f;
    const float dh = (float)(_Float16)d;
    u32x4* o = reinterpret_cast<u32x4*>(a.q16 + ((((int64_t)s * a.n_q + j) * a.H + h) * a.D + b * 32) * 2);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        f16x8 hv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float qv = fminf(fmaxf(roundf(x[8 * u + e] * id), -127.0f), 127.0f);
            hv[e] = (_Float16)(qv * dh);
        }
        o[u] = __builtin_bit_cast(u32x4, hv);
    }
}

}  // namespace

hipError_t launch_q8_stage(const Q8StageArgs& a, hipStream_t stream) {
    const int64_t nkv = (int64_t)a.S * a.n_kv * a.Hkv * (a.D / 32);
    const int64_t nq = (int64_t)a.S * a.n_q * a.H * (a.D / 32);
    if (nkv > 0) {
        const unsigned g = (unsigned)((nkv + 255) / 256);
        hipLaunchKernelGGL(q8_kv_to_f16, dim3(2 * g), dim3(256), 0, stream, a, g);
    }
    if (nq > 0 && a.q16) hipLaunchKernelGGL(q8_q_to_f16, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace sixi
