// sixi_kv_abi.cpp -- the C ABI of include/sixi_kv.h: view validation on the host, the
// kernels in kv_write.hip.
//
// As in sixi_attn_abi.cpp every error is a status (the reference's ErrorCode values of
// include/sixi_asi/common.hpp:40-67, negated) where ggml would GGML_ASSERT.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "abi_util.hpp"
#include "kv_internal.hpp"
#include "sixi_kv.h"

namespace {

using namespace sixi_abi;

bool cache_type(int32_t t) { return t == SIXI_TYPE_F16 || t == SIXI_TYPE_Q8_0; }

int resolve_write(const sixi_kv_write_params* p, sixi::KvWriteArgs* out) {
    if (!p || !p->src.data || !p->dst.data) return SIXI_E_INVALID_ARGUMENT;
    if (p->flags != 0) return SIXI_E_INVALID_ARGUMENT;
    const sixi_view& s = p->src;
    const sixi_view& d = p->dst;
    if (s.type != SIXI_TYPE_F32 && s.type != SIXI_TYPE_F16) return SIXI_E_INVALID_ARGUMENT;
    if (!cache_type(d.type)) return SIXI_E_INVALID_ARGUMENT;
    for (int i = 0; i < 4; ++i)
        if (s.ne[i] < 0 || d.ne[i] < 0 || s.nb[i] < 0 || d.nb[i] < 0) return SIXI_E_INVALID_ARGUMENT;
    const int64_t D = s.ne[0];
    if (D <= 0 || D % 32 != 0 || d.ne[0] != D) return SIXI_E_INVALID_ARGUMENT;
    const bool paged = p->page_table != nullptr;
    if (d.ne[2] != s.ne[2] || (!paged && d.ne[3] != s.ne[3])) return SIXI_E_INVALID_ARGUMENT;
    if (paged) {
        if (d.ne[1] != SIXI_KV_PAGE_CELLS || d.ne[3] <= 0 || d.ne[3] > INT32_MAX) return SIXI_E_INVALID_ARGUMENT;
        if (p->page_table_stride <= 0 || p->page_table_stride > ((int64_t)1 << 26) / SIXI_KV_PAGE_CELLS)
            return SIXI_E_INVALID_ARGUMENT;
        if (!aligned(p->page_table, 4)) return SIXI_E_ALIGNMENT;
    }
    if (s.ne[1] > INT32_MAX || s.ne[2] > INT32_MAX || s.ne[3] > INT32_MAX || D > INT32_MAX)
        return SIXI_E_INTEGER_OVERFLOW;
    // rows must be contiguous: the kernel reads 16-byte vectors of consecutive elements
    const int64_t es = elem_bytes(s.type);
    if (s.nb[0] != es) return SIXI_E_INVALID_ARGUMENT;
    if (d.type == SIXI_TYPE_F16 && d.nb[0] != 2) return SIXI_E_INVALID_ARGUMENT;
    if (d.type == SIXI_TYPE_Q8_0 && d.nb[0] != 34) return SIXI_E_INVALID_ARGUMENT;
    if (view_span(s, row_bytes(s.type, D)) < 0 || view_span(d, row_bytes(d.type, D)) < 0)
        return SIXI_E_INTEGER_OVERFLOW;
    // distinct (cell, head, stream) rows of the cache must not alias: each is written whole
    if (!rows_disjoint(d, row_bytes(d.type, D))) return SIXI_E_INVALID_ARGUMENT;
    if (!aligned(s.data, 16) || s.nb[1] % 16 || s.nb[2] % 16 || s.nb[3] % 16) return SIXI_E_ALIGNMENT;
    const int64_t da = d.type == SIXI_TYPE_F16 ? 16 : 2;
    if (!aligned(d.data, da) || d.nb[1] % da || d.nb[2] % da || d.nb[3] % da) return SIXI_E_ALIGNMENT;

    sixi::KvWriteArgs a{};
    a.src = static_cast<const char*>(s.data);
    a.s_es = es;
    a.s_nb1 = s.nb[1];
    a.s_nb2 = s.nb[2];
    a.s_nb3 = s.nb[3];
    a.src_f16 = s.type == SIXI_TYPE_F16;
    a.dst = static_cast<char*>(const_cast<void*>(d.data));
    a.d_nb1 = d.nb[1];
    a.d_nb2 = d.nb[2];
    a.d_nb3 = d.nb[3];
    a.dst_q8 = d.type == SIXI_TYPE_Q8_0;
    a.D = (int)D;
    a.n_rows = (int)s.ne[1];
    a.Hkv = (int)s.ne[2];
    a.S = (int)s.ne[3];
    a.n_cells = paged ? p->page_table_stride * SIXI_KV_PAGE_CELLS : d.ne[1];
    a.kv_len = p->kv_len;
    a.q_len = p->q_len;
    if (paged) {
        a.pt = p->page_table;
        a.pt_stride = p->page_table_stride;
        a.n_pages = (int)d.ne[3];
    }
    *out = a;
    return SIXI_OK;
}

}  // namespace

extern "C" {

int sixi_kv_write_validate(const sixi_kv_write_params* p) {
    sixi::KvWriteArgs a;
    return resolve_write(p, &a);
}

int sixi_kv_write(const sixi_kv_write_params* p) {
    sixi::KvWriteArgs a;
    const int rc = resolve_write(p, &a);
    if (rc != SIXI_OK) return rc;
    return sixi::launch_kv_write(a, static_cast<hipStream_t>(p->stream)) == hipSuccess ? SIXI_OK : SIXI_E_BACKEND;
}

int sixi_kv_copy(const sixi_kv_copy_params* p) {
    if (!p || !p->cache.data) return SIXI_E_INVALID_ARGUMENT;
    const sixi_view& v = p->cache;
    if (!cache_type(v.type)) return SIXI_E_INVALID_ARGUMENT;
    for (int i = 0; i < 4; ++i)
        if (v.ne[i] < 0 || v.nb[i] < 0) return SIXI_E_INVALID_ARGUMENT;
    const int64_t D = v.ne[0];
    if (D <= 0 || (v.type == SIXI_TYPE_Q8_0 && D % 32 != 0)) return SIXI_E_INVALID_ARGUMENT;
    if (v.nb[0] != (v.type == SIXI_TYPE_F16 ? 2 : 34)) return SIXI_E_INVALID_ARGUMENT;
    const int64_t rb = row_bytes(v.type, D);
    if (view_span(v, rb) < 0) return SIXI_E_INTEGER_OVERFLOW;
    if (!rows_disjoint(v, rb)) return SIXI_E_INVALID_ARGUMENT;
    if (p->n_cells < 0 || p->src_cell < 0 || p->dst_cell < 0) return SIXI_E_INVALID_ARGUMENT;
    if (p->src_stream < 0 || p->src_stream >= v.ne[3] || p->dst_stream < 0 || p->dst_stream >= v.ne[3])
        return SIXI_E_OUT_OF_BOUNDS;
    if (p->n_cells == 0) return SIXI_OK;
    int64_t se = 0, de = 0;
    if (!add_ok(p->src_cell, p->n_cells, &se) || !add_ok(p->dst_cell, p->n_cells, &de))
        return SIXI_E_INTEGER_OVERFLOW;
    if (se > v.ne[1] || de > v.ne[1]) return SIXI_E_OUT_OF_BOUNDS;
    // distinct rows never alias (checked above), so only the same cells of one stream can
    // overlap: rejected like memcpy's overlapping ranges
    if (p->src_stream == p->dst_stream && p->src_cell < de && p->dst_cell < se) return SIXI_E_INVALID_ARGUMENT;
    if (!aligned(v.data, 2) || v.nb[1] % 2 || v.nb[2] % 2 || v.nb[3] % 2) return SIXI_E_ALIGNMENT;

    sixi::KvCopyArgs a{};
    a.base = static_cast<char*>(const_cast<void*>(v.data));
    a.nb1 = v.nb[1];
    a.nb2 = v.nb[2];
    a.nb3 = v.nb[3];
    a.row_bytes = rb;
    a.Hkv = v.ne[2];
    a.src_stream = p->src_stream;
    a.dst_stream = p->dst_stream;
    a.src_cell = p->src_cell;
    a.dst_cell = p->dst_cell;
    a.n_cells = p->n_cells;
    a.word4_aligned = aligned(v.data, 4) && v.nb[1] % 4 == 0 && v.nb[2] % 4 == 0 && v.nb[3] % 4 == 0;
    return sixi::launch_kv_copy(a, static_cast<hipStream_t>(p->stream)) == hipSuccess ? SIXI_OK : SIXI_E_BACKEND;
}

}  // extern "C"
