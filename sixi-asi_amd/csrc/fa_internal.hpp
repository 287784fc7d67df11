// fa_internal.hpp -- argument block shared by the host dispatcher (sixi_attn_abi.cpp) and
// the gfx950 kernels.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "sixi_attn.h"

namespace sixi {

// Everything a kernel needs, resolved from the ggml-style views on the host.
struct FaArgs {
    const char* q;         // Q base; element (d, j, h, s) at q + d*q_es + j*q_nb1 + h*q_nb2 + s*q_nb3
    int64_t q_nb1, q_nb2, q_nb3;
    int32_t q_es;          // 4 (f32) or 2 (f16) -- the element stride is the element size
    int32_t q_f16;

    const char* k;         // cell c of head g of stream s at k + c*k_nb1 + g*k_nb2 + s*k_nb3
    int64_t k_nb1, k_nb2, k_nb3;
    const char* v;
    int64_t v_nb1, v_nb2, v_nb3;

    char* out;             // row (d, h, j, s) at out + d*4 + h*o_nb1 + j*o_nb2 + s*o_nb3
    int64_t o_nb1, o_nb2, o_nb3;

    const int32_t* kv_len; // device, may be null
    const int32_t* q_len;  // device, may be null

    const char* mask;      // EXPLICIT: f16 at mask + c*2 + j*m_nb1 + (s % m_ne3)*m_nb3
    int64_t m_nb1, m_nb3;
    int32_t m_ne3;

    int32_t S, H, Hkv, G;  // streams, q heads, kv heads, H / Hkv
    int32_t n_q, n_kv;     // view extents (max rows per stream, cells per stream)
    float scale;           // softmax scale (already divided by the softcap when it is on)
    float scale_log2;      // scale * log2(e)
    float softcap;         // 0 = off
    float alibi_m0, alibi_m1;
    int32_t alibi_nlog2;   // 0 = ALiBi off

    // split-K bookkeeping (workspace)
    float* part;           // partial slots: [slot][rows_max*D] O, then [rows_max] m, [rows_max] l
    int32_t* meta;         // [S+1] tile prefix over streams, written by work-group 0
    int32_t P;             // work-groups of the split-K launch
    int32_t rows_max;      // G * n_q rounded up to 16
    int64_t slot_floats;   // floats per slot
};

// Host-side launchers (defined in the .hip files).
hipError_t launch_splitk(const FaArgs& a, int kv_type, int mask_mode, int head_dim,
                         hipStream_t stream);
hipError_t launch_prefill(const FaArgs& a, int kv_type, int mask_mode, int head_dim,
                          hipStream_t stream);

// Sizing rules shared by the dispatcher and the launchers.
constexpr int kSplitTile = 32;        // KV cells per wave step of the split-K kernel
constexpr int kSplitWaves = 4;        // waves per split-K work-group
constexpr int kMaxStreams = 1024;     // LDS prefix table bound
constexpr int kMaxSplitGroups = 1024; // work-groups of a split-K launch (workspace bound)
int splitk_num_groups(const FaArgs& a, int cu_count);

}  // namespace sixi
