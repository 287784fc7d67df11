// abi_util.hpp -- host-side view arithmetic shared by the C ABIs (sixi_attn_abi.cpp,
// sixi_kv_abi.cpp): overflow-checked spans of ggml-style views and element sizes.
#pragma once

#include <cstdint>

#include "sixi_attn.h"

namespace sixi_abi {

inline bool mul_ok(int64_t a, int64_t b, int64_t* out) { return !__builtin_mul_overflow(a, b, out); }
inline bool add_ok(int64_t a, int64_t b, int64_t* out) { return !__builtin_add_overflow(a, b, out); }

// Largest byte offset touched by a view (0 for empty), or -1 on overflow.
inline int64_t view_span(const sixi_view& v, int64_t row_bytes) {
    int64_t span = row_bytes, t = 0;
    for (int d = 1; d < 4; ++d) {
        if (v.ne[d] <= 0) return 0;
        if (!mul_ok(v.ne[d] - 1, v.nb[d], &t) || !add_ok(span, t, &span)) return -1;
    }
    return span;
}

inline int elem_bytes(int32_t type) {
    switch (type) {
        case SIXI_TYPE_F32: return 4;
        case SIXI_TYPE_F16: return 2;
        default: return 0;
    }
}

// Bytes of one head row of D elements.
inline int64_t row_bytes(int32_t type, int64_t D) {
    if (type == SIXI_TYPE_Q8_0) return D / 32 * 34;
    return D * elem_bytes(type);
}

// True when the (ne[1], ne[2], ne[3]) rows of row_bytes bytes each are pairwise disjoint:
// taken by increasing stride, every dimension's rows fit below the next dimension's stride.
// (A sufficient test; written views must pass it.)
inline bool rows_disjoint(const sixi_view& v, int64_t row_bytes) {
    int dims[3] = {1, 2, 3};
    for (int i = 0; i < 3; ++i)
        for (int k = i + 1; k < 3; ++k)
            if (v.nb[dims[k]] < v.nb[dims[i]]) {
                const int t = dims[i];
                dims[i] = dims[k];
                dims[k] = t;
            }
    int64_t span = row_bytes, t = 0;
    for (int i = 0; i < 3; ++i) {
        const int d = dims[i];
        if (v.ne[d] <= 1) continue;
        if (v.nb[d] < span) return false;
        if (!mul_ok(v.ne[d] - 1, v.nb[d], &t) || !add_ok(span, t, &span)) return false;
    }
    return true;
}

inline bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)a) == 0; }

// Whether the byte ranges [a, a + a_bytes) and [b, b + b_bytes) intersect (empty ranges never do).
inline bool ranges_overlap(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes) {
    if (a_bytes <= 0 || b_bytes <= 0) return false;
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + (uintptr_t)b_bytes && b0 < a0 + (uintptr_t)a_bytes;
}

// Whether two views' byte ranges intersect; each view's span (view_span with its row bytes)
// must have been checked for overflow.
inline bool views_overlap(const sixi_view& a, int64_t a_row, const sixi_view& b, int64_t b_row) {
    return ranges_overlap(a.data, view_span(a, a_row), b.data, view_span(b, b_row));
}

}  // namespace sixi_abi
