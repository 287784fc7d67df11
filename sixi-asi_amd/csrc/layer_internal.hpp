// layer_internal.hpp -- kernel arguments shared by the layer ABI (sixi_layer_abi.cpp) and its
// kernels (layer_prologue.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sixi {

// Byte strides of the ggml views; rows are contiguous f32 (16-byte aligned).
struct QkPrologueArgs {
    const char* qg;
    int64_t qg_nb1, qg_nb2, qg_nb3;  // head, row, stream
    const char* k;
    int64_t k_nb1, k_nb2, k_nb3;     // head, row, stream
    const char* v;
    int64_t v_nb1, v_nb2, v_nb3;
    const float* q_norm;
    const float* k_norm;
    float eps;
    float theta_scale;               // rope_base^(-2/n_rot), rounded to f32 once on the host
    int n_rot;
    const int32_t* kv_len;           // may be null: positions from 0
    const int32_t* q_len;            // may be null: every row
    char* q_out;
    int64_t qo_nb1, qo_nb2, qo_nb3;  // row, head, stream
    int q_out_f16;                   // q_out rows in f16 (RNE) rather than f32
    char* kc;
    int64_t kc_nb1, kc_nb2, kc_nb3;  // cell, head, stream
    char* vc;
    int64_t vc_nb1, vc_nb2, vc_nb3;
    int cache_q8;
    int D, H, Hkv, n_rows, S;
    int64_t n_cells;
    const int32_t* pt;               // paged caches: cell c of stream s -> cell c % 256 of page
                                     // pt[s*pt_stride + c/256] (kc_nb3/vc_nb3 the page strides)
    int64_t pt_stride;
    int n_pages;
};

struct AttnGateArgs {
    char* out;
    int64_t o_nb1, o_nb2, o_nb3;     // head, row, stream
    const char* qg;
    int64_t g_nb1, g_nb2, g_nb3;     // head, row, stream (the gate starts D elements in)
    const int32_t* q_len;
    int D, H, n_rows, S;
};

hipError_t launch_qk_prologue(const QkPrologueArgs& a, hipStream_t stream);
hipError_t launch_attn_gate(const AttnGateArgs& a, hipStream_t stream);

}  // namespace sixi
