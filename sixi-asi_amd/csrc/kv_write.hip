// kv_write.hip -- writes a block's K or V rows into the per-stream KV cache (f32/f16 -> f16
// or q8_0) and copies cell ranges between streams.
//
// The engine stores the K and V of every new token before it runs attention over them:
// llama.cpp's KV cache copies the step's K/V rows into the cache cells of their stream
// (upstream ggml_set_rows into the cache view, inside every llama_decode the reference
// makes at src/core/core_execution.cpp:2074, :3536 and :3811).  A stream's cells are one
// contiguous range, so row j of stream s goes to cell kv_len[s] + j.  Rollback
// (src/core/core_execution.cpp:4021-4062, llama_memory_seq_rm) only shortens kv_len and
// moves no data; copying one stream's cells to another (llama_memory_seq_cp at
// src/core/core_execution.cpp:3215-3216 and :3245-3246, a whole-stream copy when the cache
// keeps one stream per sequence) is kv_copy below.
//
// Conversions are the reference's codecs (src/core/numeric.cpp):
//   f16   round to nearest even, subnormals kept, overflow to inf (:28-106) -- the gfx950
//         v_cvt_f16_f32 conversion in the default rounding mode;
//   q8_0  per 32-element block: amax = max |x|, d = amax / 127 stored as f16,
//         id = 127 / amax (0 when d is 0), q = clamp(round(x * id), -127, 127) with
//         round half away from zero (:349-384); both divisions are IEEE-rounded here.
//
// Both kernels are HBM-bound byte work: one thread per 32-element block (a 128-byte f32
// read and a 64-byte f16 or 34-byte q8_0 write), one thread per 4-byte word of the copy.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kv_internal.hpp"

namespace sixi {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// 32 source elements of one block as f32 (f32 rows: eight 16-byte loads; f16: four)
__device__ __forceinline__ void load_block(const char* p, bool src_f16, float (&x)[32]) {
    if (src_f16) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f16x8 h = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(p + 16 * u));
#pragma unroll
            for (int e = 0; e < 8; ++e) x[8 * u + e] = (float)h[e];
        }
    } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(p + 16 * u);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * u + e] = v[e];
        }
    }
}

__global__ __launch_bounds__(256) void kv_write_kernel(KvWriteArgs a) {
    const int64_t blocks_row = a.D / 32;
    const int64_t n = (int64_t)a.S * a.n_rows * a.Hkv * blocks_row;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int b = (int)(i % blocks_row);
    int64_t r = i / blocks_row;
    const int h = (int)(r % a.Hkv);
    r /= a.Hkv;
    const int j = (int)(r % a.n_rows);
    const int s = (int)(r / a.n_rows);
    const int ql = a.q_len ? a.q_len[s] : a.n_rows;
    if (j >= ql) return;
    const int64_t cell = (int64_t)(a.kv_len ? a.kv_len[s] : 0) + j;
    if (cell < 0 || cell >= a.n_cells) return;  // outside the stream's cells: not written

    float x[32];
    load_block(a.src + (int64_t)j * a.s_nb1 + (int64_t)h * a.s_nb2 + (int64_t)s * a.s_nb3 + (int64_t)b * 32 * a.s_es,
               a.src_f16 != 0, x);
    int64_t row_off;
    if (a.pt) {
        const int page = min(max(a.pt[(int64_t)s * a.pt_stride + (cell >> 8)], 0), a.n_pages - 1);
        row_off = (int64_t)page * a.d_nb3 + (cell & 255) * a.d_nb1;
    } else {
        row_off = cell * a.d_nb1 + (int64_t)s * a.d_nb3;
    }
    char* row = a.dst + row_off + (int64_t)h * a.d_nb2;
    if (!a.dst_q8) {
        u32x4* o = reinterpret_cast<u32x4*>(row + (int64_t)b * 64);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            f16x8 hv;
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = (_Float16)x[8 * u + e];
            o[u] = __builtin_bit_cast(u32x4, hv);
        }
        return;
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(x[e]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 127.0f / amax : 0.0f;
    // a q8_0 block is 34 bytes, so only 2-byte alignment holds: d, then the 32 quants as
    // 16 pairs
    uint16_t* o = reinterpret_cast<uint16_t*>(row + (int64_t)b * 34);
    o[0] = __builtin_bit_cast(uint16_t, (_Float16)d);
#pragma unroll
    for (int e = 0; e < 32; e += 2) {
        const int q0 = (int)fminf(fmaxf(roundf(x[e] * id), -127.0f), 127.0f);
        const int q1 = (int)fminf(fmaxf(roundf(x[e + 1] * id), -127.0f), 127.0f);
        o[1 + e / 2] = (uint16_t)((uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8));
    }
}

// One thread per 4-byte word (or 2-byte half word) of every (cell, head) row.
template <typename W>
__global__ __launch_bounds__(256) void kv_copy_kernel(KvCopyArgs a) {
    const int64_t words = a.row_bytes / (int64_t)sizeof(W);
    const int64_t n = a.n_cells * a.Hkv * words;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t w = i % words;
    const int64_t r = i / words;
    const int64_t h = r % a.Hkv;
    const int64_t c = r / a.Hkv;
    const W* src = reinterpret_cast<const W*>(a.base + (a.src_cell + c) * a.nb1 + h * a.nb2 + a.src_stream * a.nb3);
    W* dst = reinterpret_cast<W*>(a.base + (a.dst_cell + c) * a.nb1 + h * a.nb2 + a.dst_stream * a.nb3);
    dst[w] = src[w];
}

// One chunk of a table store: the values travel in the kernel's arguments.
struct TableChunk {
    int32_t* dst;
    int32_t n;
    int32_t v[kTableChunk];
};
static_assert(sizeof(TableChunk) <= 4000, "kernel arguments stay below 4 KB");

__global__ __launch_bounds__(256) void table_store_kernel(TableChunk c) {
    for (int i = threadIdx.x; i < c.n; i += blockDim.x) c.dst[i] = c.v[i];
}

}  // namespace

hipError_t launch_table_store(int32_t* dst, const int32_t* src, int64_t n, hipStream_t stream) {
    for (int64_t i = 0; i < n; i += kTableChunk) {
        TableChunk c;
        c.dst = dst + i;
        c.n = (int32_t)(n - i < kTableChunk ? n - i : kTableChunk);
        for (int k = 0; k < c.n; ++k) c.v[k] = src[i + k];
        hipLaunchKernelGGL(table_store_kernel, dim3(1), dim3(256), 0, stream, c);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t stream) {
    const int64_t n = (int64_t)a.S * a.n_rows * a.Hkv * (a.D / 32);
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(kv_write_kernel, dim3(grid), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kv_copy(const KvCopyArgs& a, hipStream_t stream) {
    const bool words4 = (a.row_bytes % 4) == 0 && a.word4_aligned;
    const int64_t n = a.n_cells * a.Hkv * (a.row_bytes / (words4 ? 4 : 2));
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (words4)
        hipLaunchKernelGGL(kv_copy_kernel<uint32_t>, dim3(grid), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(kv_copy_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace sixi
