// sixi_gdn_abi.cpp -- the C ABI of include/sixi_gdn.h: view validation on the host, the kernel
// in gdn_verify.hip.
//
// As in sixi_attn_abi.cpp every error is a status (the reference's ErrorCode values of
// include/sixi_asi/common.hpp:40-67, negated); the reference's step returns InvalidArgument for
// null pointers and empty dimensions (src/core/core_execution.cpp:262-268).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "abi_util.hpp"
#include "gdn_internal.hpp"
#include "sixi_gdn.h"

namespace {

using namespace sixi_abi;

bool shape_is(const sixi_view& v, int64_t n0, int64_t n1, int64_t n2, int64_t n3) {
    return v.ne[0] == n0 && v.ne[1] == n1 && v.ne[2] == n2 && v.ne[3] == n3;
}

bool f32_view(const sixi_view& v) {
    if (!v.data || v.type != SIXI_TYPE_F32) return false;
    for (int i = 0; i < 4; ++i)
        if (v.ne[i] < 0 || v.nb[i] < 0) return false;
    return true;
}

bool rows16(const sixi_view& v) {
    return v.nb[0] == 4 && aligned(v.data, 16) && v.nb[1] % 16 == 0 && v.nb[2] % 16 == 0 && v.nb[3] % 16 == 0;
}

// byte range [lo, hi) a view of 4-byte elements touches (every dim at its own stride; the
// spans were checked for overflow before)
void byte_range(const sixi_view& v, uintptr_t* lo, uintptr_t* hi) {
    int64_t span = 4;
    for (int d = 0; d < 4; ++d)
        if (v.ne[d] > 0) span += (v.ne[d] - 1) * v.nb[d];
    *lo = reinterpret_cast<uintptr_t>(v.data);
    *hi = *lo + (uintptr_t)span;
}

bool overlap(const sixi_view& a, const sixi_view& b) {
    uintptr_t a0, a1, b0, b1;
    byte_range(a, &a0, &a1);
    byte_range(b, &b0, &b1);
    return a0 < b1 && b0 < a1;
}

int resolve(const sixi_gdn_params* p, sixi::GdnArgs* out) {
    if (!p || (p->flags & ~SIXI_GDN_DECAY_FIRST) != 0) return SIXI_E_INVALID_ARGUMENT;
    const sixi_view &q = p->q, &k = p->k, &v = p->v, &al = p->alpha, &be = p->beta, &y = p->y, &si = p->state_in,
                    &so = p->state_out;
    for (const sixi_view* x : {&q, &k, &v, &al, &be, &y, &si, &so})
        if (!f32_view(*x)) return SIXI_E_INVALID_ARGUMENT;
    const int64_t K = q.ne[0], G = q.ne[1], n_rows = q.ne[2], S = q.ne[3], HD = v.ne[0];
    if (!((K == 64 || K == 128) && (HD == 64 || HD == 128))) return SIXI_E_UNSUPPORTED;
    if (!shape_is(k, K, G, n_rows, S) || !shape_is(v, HD, G, n_rows, S) || !shape_is(y, HD, G, n_rows, S))
        return SIXI_E_INVALID_ARGUMENT;
    if (!shape_is(al, G, n_rows, S, 1) || !shape_is(be, G, n_rows, S, 1)) return SIXI_E_INVALID_ARGUMENT;
    if (!shape_is(si, K, HD, G, S) || !shape_is(so, K, HD, G, S)) return SIXI_E_INVALID_ARGUMENT;
    if (G > INT32_MAX || n_rows > INT32_MAX || S > INT32_MAX) return SIXI_E_INTEGER_OVERFLOW;
    int64_t blocks = 0;
    if (!mul_ok(S, G, &blocks) || blocks >= (int64_t)UINT32_MAX) return SIXI_E_INTEGER_OVERFLOW;
    if (view_span(q, K * 4) < 0 || view_span(k, K * 4) < 0 || view_span(v, HD * 4) < 0 || view_span(y, HD * 4) < 0 ||
        view_span(si, K * 4) < 0 || view_span(so, K * 4) < 0)
        return SIXI_E_INTEGER_OVERFLOW;
    for (const sixi_view* x : {&al, &be}) {  // single elements at arbitrary strides
        int64_t span = 4, t = 0;
        for (int d = 0; d < 3; ++d) {
            if (x->ne[d] == 0) break;
            if (!mul_ok(x->ne[d] - 1, x->nb[d], &t) || !add_ok(span, t, &span)) return SIXI_E_INTEGER_OVERFLOW;
        }
    }
    // written rows must not alias one another
    if (!rows_disjoint(y, HD * 4) || !rows_disjoint(so, K * 4)) return SIXI_E_INVALID_ARGUMENT;
    // Work-groups read and write in no fixed order across streams and groups, so what a call
    // writes (y, the output state) must not overlap what it reads or each other.  The one
    // exception is the state updated in place: the output state is the input view itself.
    const bool same = si.data == so.data && si.nb[1] == so.nb[1] && si.nb[2] == so.nb[2] && si.nb[3] == so.nb[3];
    if (blocks > 0 && n_rows > 0) {
        for (const sixi_view* x : {&q, &k, &v, &al, &be, &si, &so})
            if (overlap(y, *x)) return SIXI_E_INVALID_ARGUMENT;
        for (const sixi_view* x : {&q, &k, &v, &al, &be})
            if (overlap(so, *x)) return SIXI_E_INVALID_ARGUMENT;
    }
    if (!same && blocks > 0 && overlap(si, so)) return SIXI_E_INVALID_ARGUMENT;
    if (!rows16(q) || !rows16(k) || !rows16(v) || !rows16(y) || !rows16(si) || !rows16(so)) return SIXI_E_ALIGNMENT;
    // state rows are whole rows of K values apart
    if (si.nb[1] < K * 4) return SIXI_E_INVALID_ARGUMENT;
    if (!aligned(al.data, 4) || !aligned(be.data, 4)) return SIXI_E_ALIGNMENT;
    for (int d = 0; d < 3; ++d)
        if (al.nb[d] % 4 || be.nb[d] % 4) return SIXI_E_ALIGNMENT;

    sixi::GdnArgs a{};
    a.q = static_cast<const char*>(q.data);
    a.q_nb1 = q.nb[1];
    a.q_nb2 = q.nb[2];
    a.q_nb3 = q.nb[3];
    a.k = static_cast<const char*>(k.data);
    a.k_nb1 = k.nb[1];
    a.k_nb2 = k.nb[2];
    a.k_nb3 = k.nb[3];
    a.v = static_cast<const char*>(v.data);
    a.v_nb1 = v.nb[1];
    a.v_nb2 = v.nb[2];
    a.v_nb3 = v.nb[3];
    a.alpha = static_cast<const char*>(al.data);
    a.a_nb0 = al.nb[0];
    a.a_nb1 = al.nb[1];
    a.a_nb2 = al.nb[2];
    a.beta = static_cast<const char*>(be.data);
    a.b_nb0 = be.nb[0];
    a.b_nb1 = be.nb[1];
    a.b_nb2 = be.nb[2];
    a.y = static_cast<char*>(const_cast<void*>(y.data));
    a.y_nb1 = y.nb[1];
    a.y_nb2 = y.nb[2];
    a.y_nb3 = y.nb[3];
    a.s_in = static_cast<const char*>(si.data);
    a.si_nb1 = si.nb[1];
    a.si_nb2 = si.nb[2];
    a.si_nb3 = si.nb[3];
    a.s_out = static_cast<char*>(const_cast<void*>(so.data));
    a.so_nb1 = so.nb[1];
    a.so_nb2 = so.nb[2];
    a.so_nb3 = so.nb[3];
    a.q_len = p->q_len;
    a.snap = p->snap;
    a.decay_first = (p->flags & SIXI_GDN_DECAY_FIRST) != 0;
    a.K = (int)K;
    a.HD = (int)HD;
    a.G = (int)G;
    a.n_rows = (int)n_rows;
    a.S = (int)S;
    *out = a;
    return SIXI_OK;
}

}  // namespace

extern "C" int sixi_gdn_verify(const sixi_gdn_params* p) {
    sixi::GdnArgs a;
    const int rc = resolve(p, &a);
    if (rc != SIXI_OK) return rc;
    return sixi::launch_gdn_verify(a, static_cast<hipStream_t>(p->stream)) == hipSuccess ? SIXI_OK : SIXI_E_BACKEND;
}
