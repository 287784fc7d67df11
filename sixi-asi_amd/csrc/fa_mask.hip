// fa_mask.hip -- the pre-pass of explicit ggml masks (the FLASH_ATTN_EXT hook's path).
//
// llama.cpp hands the attention a KQ mask that it builds from the positions of the batch
// (src/core/core_execution.cpp:2047-2062): for a verify block or a prefill chunk, row j of
// stream s sees cells [0, N_s + j] (0) and nothing else (-inf).  Read per tile and head, such
// a mask costs more bytes than the K/V it masks.  This pass reads it once per call and gives
// each row a verdict: kl = v - 1 - j when the row's scanned cells [0, nc) are v >= 1 zeros (+0
// or -0) followed only by -inf and kl >= 0; kMaskNotPrefix otherwise (kMaskRowIdle for rows
// past the stream's q_len).  When every row of a stream has the same kl, and every stream
// passes, the attention runs the lengths-only block-causal body with those offsets, which
// computes exactly what the mask specifies (mask_rows_block_causal / mask_as_lengths in
// fa_device.hpp); otherwise the mask body runs.  The choice is made on the device, so the call
// stays asynchronous and capturable.
#include "fa_device.hpp"

namespace sixi {
namespace {

constexpr int kScanMaxThreads = 1024;
constexpr int kScanUnroll = 8;  // 16-byte loads per thread and round, all issued before any is used

// grid = (n_q rows, S streams), one work-group per row; blockDim.x = scan_threads(n_kv), so that
// one round of loads covers the longest row the view allows.  Thread t takes the eight-cell
// pieces 8t + 8T u (T threads, u < kScanUnroll) of the row through a range-checked resource
// over the stream's mask rows (16-byte aligned: the callers launch this only for masks the
// staged-mask kernels can read); pieces at or past the stream's nc cells are not loaded.
__global__ __launch_bounds__(kScanMaxThreads) void mask_prefix_rows(FaArgs a) {
    const int j = blockIdx.x, s = blockIdx.y;
    const int nt = (int)blockDim.x;
    const StreamDims sd = stream_dims(a, s);
    int32_t* dst = a.row_kl + (int64_t)s * a.n_q + j;
    if (j >= sd.ql) {
        if (threadIdx.x == 0) *dst = kMaskRowIdle;
        return;
    }
    const int nc = sd.nc;
    const buf_rsrc rs = make_rsrc(a.mask + (int64_t)(s % a.m_ne3) * a.m_nb3, (uint32_t)a.m_span);
    const uint32_t row = (uint32_t)((int64_t)j * a.m_nb1);
    int first_nz = nc;  // first cell holding neither +0 nor -0
    int last_fin = -1;  // last cell not holding -inf
    for (int r0 = 8 * (int)threadIdx.x; r0 < nc; r0 += kScanUnroll * 8 * nt) {
        u32x4 w[kScanUnroll];
#pragma unroll
        for (int u = 0; u < kScanUnroll; ++u) {
            const int c0 = r0 + u * 8 * nt;
            w[u] = c0 < nc ? buf_ld16(rs, row + 2u * (uint32_t)c0) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kScanUnroll; ++u)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int c = r0 + u * 8 * nt + e;
                const uint32_t bits = (e & 1) ? (w[u][e >> 1] >> 16) : (w[u][e >> 1] & 0xffffu);
                if (c < nc) {
                    if ((bits & 0x7fffu) != 0u) first_nz = min(first_nz, c);
                    if (bits != 0xfc00u) last_fin = max(last_fin, c);
                }
            }
    }
    // work-group min / max
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        first_nz = min(first_nz, __shfl_xor(first_nz, off, 64));
        last_fin = max(last_fin, __shfl_xor(last_fin, off, 64));
    }
    __shared__ int red[2][kScanMaxThreads / 64];
    const int w = (int)threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[0][w] = first_nz;
        red[1][w] = last_fin;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int v = red[0][0], lf = red[1][0];
        for (int k = 1; k < nt / 64; ++k) {
            v = min(v, red[0][k]);
            lf = max(lf, red[1][k]);
        }
        // a prefix: zeros on [0, v), -inf on [v, nc), v >= 1, and at least the j + 1 cells of
        // a block-causal row
        *dst = (v >= 1 && lf == v - 1 && v - 1 - j >= 0) ? v - 1 - j : kMaskNotPrefix;
    }
}

// Threads per row: one round of kScanUnroll loads covers n_kv cells (64 to 1024 threads).
int scan_threads(int n_kv) {
    const int per_thread = 8 * kScanUnroll;
    int t = (n_kv + per_thread - 1) / per_thread;
    t = (t + 63) / 64 * 64;
    return t < 64 ? 64 : (t > kScanMaxThreads ? kScanMaxThreads : t);
}

}  // namespace

hipError_t launch_mask_prefix(const FaArgs& a, hipStream_t stream) {
    if (a.S <= 0 || a.n_q <= 0) return hipSuccess;
    hipLaunchKernelGGL(mask_prefix_rows, dim3((unsigned)a.n_q, (unsigned)a.S), dim3((unsigned)scan_threads(a.n_kv)), 0,
                       stream, a);
    return hipGetLastError();
}

}  // namespace sixi
