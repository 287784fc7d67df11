// kv_internal.hpp -- kernel arguments shared by the KV-cache ABI (sixi_kv_abi.cpp) and its
// kernels (kv_write.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sixi {

// Row j < q_len[s] of stream s -> cell kv_len[s] + j of the cache (skipped outside
// [0, n_cells)).  Byte strides as in the ggml views; rows are contiguous (element stride
// s_es: 4 for f32, 2 for f16 sources).
struct KvWriteArgs {
    const char* src;
    int64_t s_es, s_nb1, s_nb2, s_nb3;
    int src_f16;
    char* dst;
    int64_t d_nb1, d_nb2, d_nb3;
    int dst_q8;
    int D, n_rows, Hkv, S;
    int64_t n_cells;
    const int32_t* kv_len;  // may be null: row j -> cell j
    const int32_t* q_len;   // may be null: every row
    const int32_t* pt;      // paged cache: cell c of stream s -> cell c % 256 of page
                            // pt[s*pt_stride + c/256] (d_nb3 the page stride); null: contiguous
    int64_t pt_stride;
    int n_pages;
};

// Cells [src_cell, src_cell + n_cells) of stream src_stream -> [dst_cell, ...) of
// dst_stream, every head, row_bytes bytes per (cell, head).
struct KvCopyArgs {
    char* base;
    int64_t nb1, nb2, nb3;
    int64_t row_bytes;
    int64_t Hkv;
    int64_t src_stream, dst_stream;
    int64_t src_cell, dst_cell, n_cells;
    int word4_aligned;  // base and strides are multiples of 4
};

hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t stream);
hipError_t launch_kv_copy(const KvCopyArgs& a, hipStream_t stream);

// dst[0, n) = src[0, n) by kernel launches that carry the values as by-value arguments
// (kTableChunk entries per launch): a captured graph keeps the values of the call, and the
// host memory may change as soon as the call returns.
constexpr int kTableChunk = 960;
hipError_t launch_table_store(int32_t* dst, const int32_t* src, int64_t n, hipStream_t stream);

}  // namespace sixi
