// gdn_internal.hpp -- kernel arguments shared by the GDN ABI (sixi_gdn_abi.cpp) and its kernel
// (gdn_verify.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sixi {

// Byte strides of the ggml views (q, k, v, y rows and state rows contiguous, 16-byte aligned).
struct GdnArgs {
    const char* q;
    int64_t q_nb1, q_nb2, q_nb3;     // group, row, stream
    const char* k;
    int64_t k_nb1, k_nb2, k_nb3;
    const char* v;
    int64_t v_nb1, v_nb2, v_nb3;
    const char* alpha;
    int64_t a_nb0, a_nb1, a_nb2;     // group, row, stream
    const char* beta;
    int64_t b_nb0, b_nb1, b_nb2;
    char* y;
    int64_t y_nb1, y_nb2, y_nb3;
    const char* s_in;
    int64_t si_nb1, si_nb2, si_nb3;  // state row, group, stream
    char* s_out;
    int64_t so_nb1, so_nb2, so_nb3;
    const int32_t* q_len;            // may be null: every row
    const int32_t* snap;             // may be null: the state after q_len rows
    int decay_first;
    int K, HD, G, n_rows, S;
};

hipError_t launch_gdn_verify(const GdnArgs& a, hipStream_t stream);

}  // namespace sixi
