// sixi_layer_abi.cpp -- the C ABI of include/sixi_layer.h: view validation on the host, the
// kernels in layer_prologue.hip.
//
// As in sixi_attn_abi.cpp every error is a status (the reference's ErrorCode values of
// include/sixi_asi/common.hpp:40-67, negated) where ggml would GGML_ASSERT.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "abi_util.hpp"
#include "layer_internal.hpp"
#include "sixi_layer.h"

namespace {

using namespace sixi_abi;

bool dims_are(const sixi_view& v, int64_t n0, int64_t n1, int64_t n2, int64_t n3) {
    return v.ne[0] == n0 && v.ne[1] == n1 && v.ne[2] == n2 && v.ne[3] == n3;
}

bool nonneg(const sixi_view& v) {
    for (int i = 0; i < 4; ++i)
        if (v.ne[i] < 0 || v.nb[i] < 0) return false;
    return true;
}

// f32 rows read or written as 16-byte vectors
bool f32_rows_ok(const sixi_view& v) {
    return v.type == SIXI_TYPE_F32 && v.nb[0] == 4 && v.data != nullptr;
}

bool rows16(const sixi_view& v) { return aligned(v.data, 16) && v.nb[1] % 16 == 0 && v.nb[2] % 16 == 0 && v.nb[3] % 16 == 0; }

int resolve_prologue(const sixi_qk_prologue_params* p, sixi::QkPrologueArgs* out) {
    if (!p || p->flags != 0 || !p->q_norm || !p->k_norm) return SIXI_E_INVALID_ARGUMENT;
    const sixi_view &qg = p->qg, &k = p->k, &v = p->v, &qo = p->q_out, &kc = p->k_cache, &vc = p->v_cache;
    for (const sixi_view* x : {&qg, &k, &v, &qo, &kc, &vc})
        if (!nonneg(*x)) return SIXI_E_INVALID_ARGUMENT;
    // q_out: f32, or f16 over an f16 cache (half the bytes written here and read by the attention,
    // which rounds Q to f16 for an f16 cache anyway)
    const bool qo_f16 = qo.type == SIXI_TYPE_F16 && qo.nb[0] == 2 && qo.data != nullptr;
    if (!f32_rows_ok(qg) || !f32_rows_ok(k) || !f32_rows_ok(v) || (!f32_rows_ok(qo) && !qo_f16))
        return SIXI_E_INVALID_ARGUMENT;
    const int64_t D = qo.ne[0];
    if (D != 128 && D != 256) return SIXI_E_UNSUPPORTED;
    const int64_t H = qg.ne[1], n_rows = qg.ne[2], S = qg.ne[3], Hkv = k.ne[1];
    const bool paged = p->page_table != nullptr;
    if (paged && (p->page_table_stride <= 0 || p->page_table_stride > ((int64_t)1 << 26) / SIXI_KV_PAGE_CELLS))
        return SIXI_E_INVALID_ARGUMENT;
    if (paged && !aligned(p->page_table, 4)) return SIXI_E_ALIGNMENT;
    const int64_t n_cells = paged ? p->page_table_stride * SIXI_KV_PAGE_CELLS : kc.ne[1];
    // the cache views: [D, n_cells, Hkv, S], or (paged) pools [D, 256, Hkv, n_pages]
    const int64_t c_ne1 = paged ? SIXI_KV_PAGE_CELLS : n_cells, c_ne3 = paged ? kc.ne[3] : S;
    if (paged && (c_ne3 <= 0 || c_ne3 > INT32_MAX)) return SIXI_E_INVALID_ARGUMENT;
    if (qg.ne[0] != 2 * D || !dims_are(qo, D, n_rows, H, S)) return SIXI_E_INVALID_ARGUMENT;
    if (!dims_are(k, D, Hkv, n_rows, S) || !dims_are(v, D, Hkv, n_rows, S)) return SIXI_E_INVALID_ARGUMENT;
    if (kc.type != vc.type || (kc.type != SIXI_TYPE_F16 && kc.type != SIXI_TYPE_Q8_0)) return SIXI_E_INVALID_ARGUMENT;
    // an f16 Q only for an f16 cache: over q8_0 the attention converts Q to the q8_0 dot type from
    // its f32 values (ggml's rule), which an f16 Q would change
    if (qo_f16 && kc.type != SIXI_TYPE_F16) return SIXI_E_INVALID_ARGUMENT;
    if (!kc.data || !vc.data) return SIXI_E_INVALID_ARGUMENT;
    if (!dims_are(kc, D, c_ne1, Hkv, c_ne3) || !dims_are(vc, D, c_ne1, Hkv, c_ne3)) return SIXI_E_INVALID_ARGUMENT;
    const int64_t cnb0 = kc.type == SIXI_TYPE_F16 ? 2 : 34;
    if (kc.nb[0] != cnb0 || vc.nb[0] != cnb0) return SIXI_E_INVALID_ARGUMENT;
    if (p->n_rot < 0 || p->n_rot > D || p->n_rot % (D / 32) != 0) return SIXI_E_INVALID_ARGUMENT;
    if (!std::isfinite(p->eps) || p->eps < 0.0f) return SIXI_E_INVALID_ARGUMENT;
    if (!std::isfinite(p->rope_base) || p->rope_base <= 0.0f) return SIXI_E_INVALID_ARGUMENT;
    if (H > INT32_MAX || Hkv > INT32_MAX || n_rows > INT32_MAX || S > INT32_MAX) return SIXI_E_INTEGER_OVERFLOW;
    int64_t rows = 0;  // one block per (stream, row)
    if (!mul_ok(S, n_rows, &rows) || rows >= (int64_t)UINT32_MAX) return SIXI_E_INTEGER_OVERFLOW;
    const int64_t crb = row_bytes(kc.type, D);
    if (view_span(qg, 2 * D * 4) < 0 || view_span(k, D * 4) < 0 || view_span(v, D * 4) < 0 ||
        view_span(qo, D * (qo_f16 ? 2 : 4)) < 0 || view_span(kc, crb) < 0 || view_span(vc, crb) < 0)
        return SIXI_E_INTEGER_OVERFLOW;
    // written rows must not alias one another
    if (!rows_disjoint(qo, D * (qo_f16 ? 2 : 4)) || !rows_disjoint(kc, crb) || !rows_disjoint(vc, crb))
        return SIXI_E_INVALID_ARGUMENT;
    if (!rows16(qg) || !rows16(k) || !rows16(v) || !rows16(qo)) return SIXI_E_ALIGNMENT;
    if (!aligned(p->q_norm, 16) || !aligned(p->k_norm, 16)) return SIXI_E_ALIGNMENT;
    if (kc.type == SIXI_TYPE_F16 ? (!rows16(kc) || !rows16(vc))
                                 : (!aligned(kc.data, 2) || !aligned(vc.data, 2) || kc.nb[1] % 2 || kc.nb[2] % 2 ||
                                    kc.nb[3] % 2 || vc.nb[1] % 2 || vc.nb[2] % 2 || vc.nb[3] % 2))
        return SIXI_E_ALIGNMENT;

    sixi::QkPrologueArgs a{};
    a.qg = static_cast<const char*>(qg.data);
    a.qg_nb1 = qg.nb[1];
    a.qg_nb2 = qg.nb[2];
    a.qg_nb3 = qg.nb[3];
    a.k = static_cast<const char*>(k.data);
    a.k_nb1 = k.nb[1];
    a.k_nb2 = k.nb[2];
    a.k_nb3 = k.nb[3];
    a.v = static_cast<const char*>(v.data);
    a.v_nb1 = v.nb[1];
    a.v_nb2 = v.nb[2];
    a.v_nb3 = v.nb[3];
    a.q_norm = p->q_norm;
    a.k_norm = p->k_norm;
    a.eps = p->eps;
    // ggml: theta_scale = powf(freq_base, -2.0f/n_dims), in f32 on the host
    a.theta_scale = p->n_rot > 0 ? powf(p->rope_base, -2.0f / (float)p->n_rot) : 1.0f;
    a.n_rot = p->n_rot;
    a.kv_len = p->kv_len;
    a.q_len = p->q_len;
    a.q_out = static_cast<char*>(const_cast<void*>(qo.data));
    a.qo_nb1 = qo.nb[1];
    a.qo_nb2 = qo.nb[2];
    a.qo_nb3 = qo.nb[3];
    a.q_out_f16 = qo_f16 ? 1 : 0;
    a.kc = static_cast<char*>(const_cast<void*>(kc.data));
    a.kc_nb1 = kc.nb[1];
    a.kc_nb2 = kc.nb[2];
    a.kc_nb3 = kc.nb[3];
    a.vc = static_cast<char*>(const_cast<void*>(vc.data));
    a.vc_nb1 = vc.nb[1];
    a.vc_nb2 = vc.nb[2];
    a.vc_nb3 = vc.nb[3];
    a.cache_q8 = kc.type == SIXI_TYPE_Q8_0;
    a.D = (int)D;
    a.H = (int)H;
    a.Hkv = (int)Hkv;
    a.n_rows = (int)n_rows;
    a.S = (int)S;
    a.n_cells = n_cells;
    if (paged) {
        a.pt = p->page_table;
        a.pt_stride = p->page_table_stride;
        a.n_pages = (int)c_ne3;
    }
    *out = a;
    return SIXI_OK;
}

int resolve_gate(const sixi_attn_gate_params* p, sixi::AttnGateArgs* out) {
    if (!p) return SIXI_E_INVALID_ARGUMENT;
    const sixi_view &o = p->out, &g = p->qg;
    if (!nonneg(o) || !nonneg(g) || !f32_rows_ok(o) || !f32_rows_ok(g)) return SIXI_E_INVALID_ARGUMENT;
    const int64_t D = o.ne[0], H = o.ne[1], n_rows = o.ne[2], S = o.ne[3];
    if (D != 128 && D != 256) return SIXI_E_UNSUPPORTED;
    if (!dims_are(g, 2 * D, H, n_rows, S)) return SIXI_E_INVALID_ARGUMENT;
    if (H > INT32_MAX || n_rows > INT32_MAX || S > INT32_MAX) return SIXI_E_INTEGER_OVERFLOW;
    int64_t rows = 0;  // one block per (stream, row)
    if (!mul_ok(S, n_rows, &rows) || rows >= (int64_t)UINT32_MAX) return SIXI_E_INTEGER_OVERFLOW;
    if (view_span(o, D * 4) < 0 || view_span(g, 2 * D * 4) < 0) return SIXI_E_INTEGER_OVERFLOW;
    if (!rows_disjoint(o, D * 4)) return SIXI_E_INVALID_ARGUMENT;
    if (!rows16(o) || !rows16(g)) return SIXI_E_ALIGNMENT;
    sixi::AttnGateArgs a{};
    a.out = static_cast<char*>(const_cast<void*>(o.data));
    a.o_nb1 = o.nb[1];
    a.o_nb2 = o.nb[2];
    a.o_nb3 = o.nb[3];
    a.qg = static_cast<const char*>(g.data);
    a.g_nb1 = g.nb[1];
    a.g_nb2 = g.nb[2];
    a.g_nb3 = g.nb[3];
    a.q_len = p->q_len;
    a.D = (int)D;
    a.H = (int)H;
    a.n_rows = (int)n_rows;
    a.S = (int)S;
    *out = a;
    return SIXI_OK;
}

}  // namespace

extern "C" {

int sixi_qk_prologue(const sixi_qk_prologue_params* p) {
    sixi::QkPrologueArgs a;
    const int rc = resolve_prologue(p, &a);
    if (rc != SIXI_OK) return rc;
    return sixi::launch_qk_prologue(a, static_cast<hipStream_t>(p->stream)) == hipSuccess ? SIXI_OK : SIXI_E_BACKEND;
}

int sixi_attn_gate(const sixi_attn_gate_params* p) {
    sixi::AttnGateArgs a;
    const int rc = resolve_gate(p, &a);
    if (rc != SIXI_OK) return rc;
    return sixi::launch_attn_gate(a, static_cast<hipStream_t>(p->stream)) == hipSuccess ? SIXI_OK : SIXI_E_BACKEND;
}

}  // extern "C"
