// sixi_attn_abi.cpp -- the C ABI of include/sixi_attn.h: validation, workspace sizing and
// kernel choice on the host; the kernels themselves live in fa_decode.hip and
// fa_prefill.hip.
//
// Errors follow the reference's convention of returning a status instead of aborting
// (include/sixi_asi/common.hpp:40-67, codes negated), where ggml_flash_attn_ext would
// GGML_ASSERT.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "abi_util.hpp"
#include "fa_internal.hpp"
#include "sixi_attn.h"

namespace {

using sixi::FaArgs;
using namespace sixi_abi;

constexpr size_t kWsAlign = 256;
// head dims built for gfx950: 128 everywhere; 256 for f16 KV
constexpr bool head_dim_built(int64_t D) { return D == 128 || D == 256; }
constexpr int kSplitMaxRows = 16 * sixi::kDecodeMaxRowTiles;  // G * n_q of the split-K kernel
constexpr int64_t kQ8MaxRows = 48;  // rows per kv-head group of one q8_0 split-K launch

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// The small device arrays a call reads besides its views: the lengths and the page table.
struct DevRange {
    const void* p;
    int64_t bytes;
};
std::array<DevRange, 3> device_arrays(const sixi_attn_params* p, int64_t S) {
    const int64_t pt = p->page_table ? S * p->page_table_stride * 4 : 0;
    return {DevRange{p->kv_len, p->kv_len ? S * 4 : 0}, DevRange{p->q_len, p->q_len ? S * 4 : 0},
            DevRange{p->page_table, pt}};
}

// Whether [ws, ws + bytes) meets anything the call reads or writes.  The views' spans were
// checked for overflow by resolve().
bool workspace_overlaps(const sixi_attn_params* p, const void* ws, size_t bytes) {
    const int64_t D = p->q.ne[0];
    const int64_t n = (int64_t)bytes;
    const int64_t kvrow = row_bytes(p->k.type, D);
    if (ranges_overlap(ws, n, p->q.data, view_span(p->q, D * elem_bytes(p->q.type))) ||
        ranges_overlap(ws, n, p->k.data, view_span(p->k, kvrow)) ||
        ranges_overlap(ws, n, p->v.data, view_span(p->v, kvrow)) ||
        ranges_overlap(ws, n, p->out.data, view_span(p->out, D * 4)))
        return true;
    if (p->mask_mode == SIXI_MASK_EXPLICIT && ranges_overlap(ws, n, p->mask.data, view_span(p->mask, p->mask.ne[0] * 2)))
        return true;
    if ((p->flags & SIXI_ATTN_FLAG_GATE) && ranges_overlap(ws, n, p->gate_qg.data, view_span(p->gate_qg, 2 * D * 4)))
        return true;
    for (const DevRange& x : device_arrays(p, p->q.ne[3]))
        if (ranges_overlap(ws, n, x.p, x.bytes)) return true;
    return false;
}

struct Plan {
    FaArgs a{};
    int kv_type = 0;
    int mask_mode = 0;
    int D = 0;
    bool splitk = true;
    bool generic = false;      // explicit mask or softcap: the decode kernels' per-cell mode
    size_t seg_offset = 0;  // split-K: byte offset of the per-segment piece table
    int row_tiles = 0;
    bool q8_stage = false;     // q8_0 KV staged as f16 rows in the workspace, then the f16 kernels
    size_t stage_k = 0, stage_v = 0, stage_q = 0;  // byte offsets of the staged K, V and Q
    size_t stage_bytes = 0;    // the split-K workspace follows the staging area
    bool mask_prepass = false; // explicit mask reduced to per-row offsets first (fa_mask.hip)
    size_t prepass_offset = 0; // byte offset of its table (S * n_q int32), after the rest
    size_t ws_bytes = 0;
};

// Appends the pre-pass table to the workspace layout (after everything else, so that the
// staging and split-K offsets do not move).
void prepass_layout(Plan& pl) {
    if (!pl.mask_prepass) return;
    pl.prepass_offset = align_up(pl.ws_bytes, kWsAlign);
    pl.ws_bytes = pl.prepass_offset + align_up((size_t)pl.a.S * pl.a.n_q * sizeof(int32_t), kWsAlign);
}

int cu_count_cached() {
    static int cached = -1;
    if (cached < 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cached = n;
        else
            cached = 256;
    }
    return cached;
}

// Split-K workspace after the staging area: `slots` partial slots, then the (first, last)
// piece of every segment.
void splitk_layout(Plan& pl, int64_t slots) {
    const int64_t segs = (int64_t)pl.a.S * pl.a.Hkv;
    pl.seg_offset = align_up((size_t)(slots * pl.a.slot_floats) * sizeof(float), kWsAlign);
    pl.ws_bytes = pl.stage_bytes + align_up(pl.seg_offset + (size_t)segs * 2 * sizeof(int32_t), kWsAlign);
}

// Resolves and validates a description.  Touches no device memory.  A q8_0 cache is staged
// as f16 only where the staging takes at most `stage_cap` bytes (or where it cannot be
// avoided: 256-dim rows that are not 16-byte aligned).
int resolve(const sixi_attn_params* p, Plan* out, size_t stage_cap = SIXI_ATTN_STAGE_CAP_BYTES) {
    if (!p || !out) return SIXI_E_INVALID_ARGUMENT;
    if ((p->flags & ~(SIXI_ATTN_FLAG_BOUNDED_WORKSPACE | SIXI_ATTN_FLAG_GATE)) != 0) return SIXI_E_INVALID_ARGUMENT;
    if (p->flags & SIXI_ATTN_FLAG_BOUNDED_WORKSPACE) stage_cap = 0;
    const sixi_view &q = p->q, &k = p->k, &v = p->v, &o = p->out;
    if (!q.data || !k.data || !v.data || !o.data) return SIXI_E_INVALID_ARGUMENT;

    // types
    if (q.type != SIXI_TYPE_F32 && q.type != SIXI_TYPE_F16) return SIXI_E_UNSUPPORTED;
    if (k.type != SIXI_TYPE_F16 && k.type != SIXI_TYPE_Q8_0) return SIXI_E_UNSUPPORTED;
    if (v.type != k.type) return SIXI_E_UNSUPPORTED;
    if (o.type != SIXI_TYPE_F32) return SIXI_E_UNSUPPORTED;

    // extents
    for (int d = 0; d < 4; ++d)
        if (q.ne[d] <= 0 || k.ne[d] <= 0 || v.ne[d] <= 0 || o.ne[d] <= 0) return SIXI_E_INVALID_ARGUMENT;
    const int64_t D = q.ne[0], n_q = q.ne[1], H = q.ne[2], S = q.ne[3];
    const int64_t Hkv = k.ne[2];
    // paged: k and v are pools of 256-cell pages, a stream spans page_table_stride pages
    const bool paged = p->page_table != nullptr;
    int64_t n_kv = k.ne[1];
    if (k.ne[0] != D || v.ne[0] != D) return SIXI_E_INVALID_ARGUMENT;
    if (paged) {
        if (k.ne[1] != SIXI_KV_PAGE_CELLS || v.ne[1] != SIXI_KV_PAGE_CELLS || v.ne[2] != Hkv || v.ne[3] != k.ne[3])
            return SIXI_E_INVALID_ARGUMENT;
        if (p->page_table_stride <= 0 || p->page_table_stride > ((int64_t)1 << 26) / SIXI_KV_PAGE_CELLS)
            return SIXI_E_INVALID_ARGUMENT;
        if (k.ne[3] > INT32_MAX) return SIXI_E_UNSUPPORTED;
        if (!aligned(p->page_table, 4)) return SIXI_E_ALIGNMENT;
        n_kv = p->page_table_stride * SIXI_KV_PAGE_CELLS;
    } else if (v.ne[1] != n_kv || v.ne[2] != Hkv || k.ne[3] != S || v.ne[3] != S) {
        return SIXI_E_INVALID_ARGUMENT;
    }
    if (H % Hkv != 0) return SIXI_E_INVALID_ARGUMENT;
    if (o.ne[0] != D || o.ne[1] != H || o.ne[2] != n_q || o.ne[3] != S) return SIXI_E_INVALID_ARGUMENT;
    if (S > sixi::kMaxStreams || H > 4096 || n_q > (1 << 20) || n_kv > (1 << 26)) return SIXI_E_UNSUPPORTED;
    if (!head_dim_built(D)) return SIXI_E_UNSUPPORTED;

    // element strides and alignment
    const int qes = elem_bytes(q.type);
    if (q.nb[0] != qes || o.nb[0] != 4) return SIXI_E_INVALID_ARGUMENT;
    if (k.nb[0] != (k.type == SIXI_TYPE_Q8_0 ? 34 : 2) || v.nb[0] != k.nb[0]) return SIXI_E_INVALID_ARGUMENT;
    // f16 rows are moved in 16-byte pieces, q8_0 rows (136 B) in dwords
    const int kv_align = (k.type == SIXI_TYPE_Q8_0) ? 4 : 16;
    for (int d = 1; d < 4; ++d) {
        if (q.nb[d] <= 0 || k.nb[d] <= 0 || v.nb[d] <= 0 || o.nb[d] <= 0) return SIXI_E_INVALID_ARGUMENT;
        if (q.nb[d] % qes) return SIXI_E_ALIGNMENT;
        if (k.nb[d] % kv_align || v.nb[d] % kv_align || o.nb[d] % 16) return SIXI_E_ALIGNMENT;
    }
    if (!aligned(q.data, qes) || !aligned(k.data, kv_align) || !aligned(v.data, kv_align) || !aligned(o.data, 16))
        return SIXI_E_ALIGNMENT;
    const int64_t kvrow = row_bytes(k.type, D);
    if (k.nb[1] < kvrow || v.nb[1] < kvrow) return SIXI_E_INVALID_ARGUMENT;  // rows must not overlap
    if (o.nb[1] < D * 4 || q.nb[1] < D * qes) return SIXI_E_INVALID_ARGUMENT;
    // the cells a buffer resource covers -- the rest of a stream (plus one tile of read-ahead),
    // or of a page -- are addressed with 32-bit offsets
    const int64_t span_cells = (paged ? SIXI_KV_PAGE_CELLS : n_kv) + sixi::kDecodeTileWide;
    int64_t kspan = 0, vspan = 0;
    if (!mul_ok(span_cells, k.nb[1], &kspan) || !mul_ok(span_cells, v.nb[1], &vspan) ||
        kspan >= (int64_t)UINT32_MAX || vspan >= (int64_t)UINT32_MAX)
        return SIXI_E_UNSUPPORTED;
    if (view_span(q, D * qes) < 0 || view_span(k, kvrow) < 0 || view_span(v, kvrow) < 0 ||
        view_span(o, D * 4) < 0)
        return SIXI_E_INTEGER_OVERFLOW;
    // Work-groups write output rows in no fixed order: every row must be its own, and no
    // written byte may be one that a work-group reads (Q, K, V; the mask below).
    if (!rows_disjoint(o, D * 4)) return SIXI_E_INVALID_ARGUMENT;
    if (views_overlap(o, D * 4, q, D * qes) || views_overlap(o, D * 4, k, kvrow) || views_overlap(o, D * 4, v, kvrow))
        return SIXI_E_INVALID_ARGUMENT;
    for (const DevRange& x : device_arrays(p, S))
        if (ranges_overlap(o.data, view_span(o, D * 4), x.p, x.bytes)) return SIXI_E_INVALID_ARGUMENT;

    // mask
    const int mode = p->mask_mode;
    if (mode < SIXI_MASK_NONE || mode > SIXI_MASK_EXPLICIT) return SIXI_E_INVALID_ARGUMENT;
    if (mode == SIXI_MASK_BLOCK_CAUSAL && (!p->kv_len || n_q > n_kv)) return SIXI_E_INVALID_ARGUMENT;
    if (p->kv_len && n_q > n_kv) return SIXI_E_INVALID_ARGUMENT;
    const sixi_view& m = p->mask;
    if (mode == SIXI_MASK_EXPLICIT) {
        if (!m.data || m.type != SIXI_TYPE_F16 || m.nb[0] != 2) return SIXI_E_INVALID_ARGUMENT;
        if (m.ne[0] < n_kv || m.ne[1] < n_q || m.ne[2] != 1 || (m.ne[3] != 1 && m.ne[3] != S))
            return SIXI_E_INVALID_ARGUMENT;
        if (m.nb[1] % 2 || m.nb[3] % 2 || !aligned(m.data, 2)) return SIXI_E_ALIGNMENT;
        if (view_span(m, m.ne[0] * 2) < 0) return SIXI_E_INTEGER_OVERFLOW;
        if (views_overlap(o, D * 4, m, m.ne[0] * 2)) return SIXI_E_INVALID_ARGUMENT;
    }

    // the fused output gate: qg [2D, H, >= n_q, S] f32, read while `out` is written
    const sixi_view& gq = p->gate_qg;
    const bool gate = (p->flags & SIXI_ATTN_FLAG_GATE) != 0;
    if (gate) {
        if (!gq.data || gq.type != SIXI_TYPE_F32 || gq.nb[0] != 4) return SIXI_E_INVALID_ARGUMENT;
        if (gq.ne[0] != 2 * D || gq.ne[1] != H || gq.ne[2] < n_q || gq.ne[3] != S) return SIXI_E_INVALID_ARGUMENT;
        for (int d = 1; d < 4; ++d) {
            if (gq.nb[d] <= 0) return SIXI_E_INVALID_ARGUMENT;
            if (gq.nb[d] % 16) return SIXI_E_ALIGNMENT;
        }
        if (!aligned(gq.data, 16)) return SIXI_E_ALIGNMENT;
        if (view_span(gq, 2 * D * 4) < 0) return SIXI_E_INTEGER_OVERFLOW;
        if (views_overlap(o, D * 4, gq, 2 * D * 4)) return SIXI_E_INVALID_ARGUMENT;
    }

    // scalars (ggml: ALiBi slopes multiply the mask, so they need one)
    if (!std::isfinite(p->scale) || !std::isfinite(p->max_bias) || !std::isfinite(p->logit_softcap))
        return SIXI_E_INVALID_ARGUMENT;
    if (p->max_bias < 0.0f || p->logit_softcap < 0.0f) return SIXI_E_INVALID_ARGUMENT;
    if (p->max_bias > 0.0f && mode != SIXI_MASK_EXPLICIT) return SIXI_E_INVALID_ARGUMENT;

    Plan pl;
    FaArgs& a = pl.a;
    a.q = static_cast<const char*>(q.data);
    a.q_nb1 = q.nb[1]; a.q_nb2 = q.nb[2]; a.q_nb3 = q.nb[3];
    a.q_es = qes;
    a.q_f16 = (q.type == SIXI_TYPE_F16);
    a.k = static_cast<const char*>(k.data);
    a.k_nb1 = k.nb[1]; a.k_nb2 = k.nb[2]; a.k_nb3 = k.nb[3];
    a.v = static_cast<const char*>(v.data);
    a.v_nb1 = v.nb[1]; a.v_nb2 = v.nb[2]; a.v_nb3 = v.nb[3];
    if (paged) {
        a.pt = p->page_table;
        a.pt_stride = p->page_table_stride;
        a.n_pages = (int32_t)k.ne[3];
    }
    a.out = static_cast<char*>(const_cast<void*>(o.data));
    a.o_nb1 = o.nb[1]; a.o_nb2 = o.nb[2]; a.o_nb3 = o.nb[3];
    a.kv_len = p->kv_len;
    a.kv_len_stride = 1;
    a.q_len = p->q_len;
    if (mode == SIXI_MASK_EXPLICIT) {
        a.mask = static_cast<const char*>(m.data);
        a.m_nb1 = m.nb[1]; a.m_nb3 = m.nb[3];
        a.m_ne3 = (int32_t)m.ne[3];
        // the 32-cell kernel stages rows j < 32 of every step through LDS with 16-byte DMA
        // loads: whole rows of 16-byte alignment, reachable with 32-bit offsets
        const int64_t rows = std::min<int64_t>(n_q, 32);
        const int64_t span = (rows - 1) * m.nb[1] + m.ne[0] * 2;
        a.mask_stage = (n_q <= 32 && m.nb[1] % 16 == 0 && (m.ne[3] == 1 || m.nb[3] % 16 == 0) &&
                        aligned(m.data, 16) && span < (int64_t)UINT32_MAX)
                           ? 1 : 0;
        a.m_bytes = a.mask_stage ? (uint32_t)span : 0u;
        // the prefill kernel stages every row j < n_q: the exact bytes of one stream's rows
        // (its tail tile reads cells past ne[0], which this bound turns into zeros on the last
        // row; the other rows read into their successor and mask those cells by length)
        a.m_span = (n_q - 1) * m.nb[1] + m.ne[0] * 2;
    } else {
        a.m_ne3 = 1;
    }
    if (gate) {
        a.gate = static_cast<const char*>(gq.data) + D * 4;  // the gate half of each head's row
        a.g_nb1 = gq.nb[1]; a.g_nb2 = gq.nb[2]; a.g_nb3 = gq.nb[3];
    }
    a.S = (int32_t)S; a.H = (int32_t)H; a.Hkv = (int32_t)Hkv; a.G = (int32_t)(H / Hkv);
    a.Gr = a.G; a.hoff = 0;
    a.n_q = (int32_t)n_q; a.n_kv = (int32_t)n_kv;
    const float softcap = p->logit_softcap;
    a.scale = softcap != 0.0f ? p->scale / softcap : p->scale;
    a.scale_log2 = a.scale * 1.4426950408889634f;
    a.softcap = softcap;
    if (p->max_bias > 0.0f) {
        int nlog2 = 1;
        while (nlog2 * 2 <= H) nlog2 *= 2;
        a.alibi_nlog2 = nlog2;
        a.alibi_m0 = std::pow(2.0f, -p->max_bias / (float)nlog2);
        a.alibi_m1 = std::pow(2.0f, -(p->max_bias / 2.0f) / (float)nlog2);
    }

    pl.kv_type = k.type;
    pl.mask_mode = mode;
    pl.generic = mode == SIXI_MASK_EXPLICIT || softcap != 0.0f;
    pl.D = (int)D;
    const int64_t rows = (int64_t)a.G * n_q;
    pl.splitk = rows <= kSplitMaxRows;
    // q8_0 KV runs the split-K kernels in one launch that reads the KV once: at 128-dim heads
    // the 16-cell kernel up to 48 rows (with a mask or softcap: up to 16), the 32-cell q8_0
    // kernel beyond; at 256-dim heads (16-byte aligned rows) the 32-cell q8_0 kernel.  Prefill
    // blocks are staged as f16 up to stage_cap bytes (one pass over the cache, then the f16
    // kernel: faster than converting every tile in each work-group that reads it), beyond it the
    // prefill kernel reads the q8_0 tiles and converts them in LDS.
    if (k.type == SIXI_TYPE_Q8_0 && (rows > kQ8MaxRows || D != 128)) {
        // 256-dim q8_0 rows (272 B) are read by 16-byte LDS-DMA loads: every row must start
        // 16-byte aligned
        auto rows16 = [](const sixi_view& t) {
            return aligned(t.data, 16) && t.nb[1] % 16 == 0 && t.nb[2] % 16 == 0 && t.nb[3] % 16 == 0;
        };
        const bool dma16 = D == 128 || (D == 256 && rows16(k) && rows16(v));
        // the f16 staging (fa_q8_stage.hip) in the workspace: K and V, and for a split-K call Q
        // (the prefill kernel converts Q itself)
        int64_t kv_bytes = 0, q_bytes = 0, cells = 0, span = 0;
        if (!mul_ok(S * Hkv, n_kv, &cells) || !mul_ok(cells, D * 2, &kv_bytes) ||
            !mul_ok(S * H, n_q, &q_bytes) || !mul_ok(q_bytes, D * 2, &q_bytes) ||
            !mul_ok(n_kv + sixi::kDecodeTileWide, Hkv * D * 2, &span))
            return SIXI_E_INTEGER_OVERFLOW;
        const size_t stage_v = align_up((size_t)kv_bytes, kWsAlign);
        const size_t stage_q = stage_v + align_up((size_t)kv_bytes, kWsAlign);
        const size_t stage_bytes = stage_q + (pl.splitk ? align_up((size_t)q_bytes, kWsAlign) : 0);
        if (pl.splitk && dma16) {
            // one launch of the 32-cell q8_0 kernel
        } else if (!pl.splitk && dma16 && stage_bytes > stage_cap) {
            // the prefill kernel converts each tile's q8_0 rows to f16 in LDS
        } else {
            // staged as f16 operands in the workspace, then the f16 kernels: a prefill-sized
            // block while the copy is small (one pass over the cache instead of a conversion per
            // work-group that reads a tile), or 256-dim rows that are not 16-byte aligned
            if (span >= (int64_t)UINT32_MAX) return SIXI_E_UNSUPPORTED;
            pl.q8_stage = true;
            pl.kv_type = SIXI_TYPE_F16;
            pl.stage_k = 0;
            pl.stage_v = stage_v;
            pl.stage_q = stage_q;
            pl.stage_bytes = stage_bytes;
        }
    }
    // An explicit mask alone (no softcap, no ALiBi) with 16-byte aligned rows within one 32-bit
    // range is first reduced to the kv offset each row implies (fa_mask.hip); where every row is
    // the block-causal prefix of its stream's offset, the dual kernels then run the lengths-only
    // body on those offsets, and otherwise the mask.  A split-K call is then planned as the
    // lengths-only call of its shape (mask_prepass_decode), a prefill call keeps its plan.
    const bool mask_alone = mode == SIXI_MASK_EXPLICIT && softcap == 0.0f && a.alibi_nlog2 == 0 &&
                            S * n_q <= sixi::kMaskPrepassMaxRows && aligned(m.data, 16) && m.nb[1] % 16 == 0 &&
                            (m.ne[3] == 1 || m.nb[3] % 16 == 0) && a.m_span < (int64_t)UINT32_MAX;
    if (mask_alone && !pl.splitk) pl.mask_prepass = true;
    if (mask_alone && pl.splitk &&
        sixi::mask_prepass_decode(pl.kv_type, sixi::decode_row_tiles(rows, pl.D, pl.kv_type, false), pl.D,
                                  a.mask_stage != 0)) {
        pl.generic = false;
        // single-stream decode: the kernels read the one mask row themselves (no pre-pass launch)
        if (S == 1 && n_q == 1 && n_kv <= sixi::kMaskInlineMaxCells)
            a.mask_inline = 1;
        else
            pl.mask_prepass = true;
    }
    if (pl.splitk) {
        pl.row_tiles = sixi::decode_row_tiles(rows, pl.D, pl.kv_type, pl.generic);
        a.slot_floats = sixi::decode_slot_floats(pl.row_tiles, pl.D);
        a.tile_cells = sixi::decode_tile_cells(pl.kv_type, pl.row_tiles, pl.D, pl.generic);
        a.seg_cost = sixi::decode_seg_cost(pl.kv_type, pl.row_tiles, pl.D, pl.generic);
        // the kernels sum the streams' costs (tiles + seg_cost each) in 32-bit integers: a paged
        // call may describe up to 2^26 cells per stream, which 512 full streams would overflow
        const int64_t stream_cost = (n_kv + a.tile_cells - 1) / a.tile_cells + a.seg_cost;
        if (stream_cost * S > (int64_t)INT32_MAX) return SIXI_E_UNSUPPORTED;
        // slot indices run up to S*Hkv + P - 2 for a launch of P <= kMaxSplitGroups work-groups
        splitk_layout(pl, S * Hkv + sixi::kMaxSplitGroups);
    } else {
        // the prefill kernel keeps everything on chip; a token workspace keeps the contract uniform
        if (S * H * ((n_q + 127) / 128) > (int64_t)INT32_MAX) return SIXI_E_UNSUPPORTED;
        pl.ws_bytes = pl.stage_bytes > 0 ? pl.stage_bytes : kWsAlign;
    }
    prepass_layout(pl);
    *out = pl;
    return SIXI_OK;
}

// ---- scratch of the no-allocation entry point ----
// One copy per GPU the library runs on, held until the process ends.  On the host `scratch`
// names a stand-in, not device memory: host code only ever uses the device address that
// scratch_base() looks up (once per device, with that device current).
constexpr size_t kScratchBytes = SIXI_ATTN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

// Device address of the current device's `scratch`, or null if the lookup fails.
char* scratch_base() {
    static std::mutex mu;
    static char* base[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!base[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        base[dev] = static_cast<char*>(ptr);
    }
    return base[dev];
}

// Work-groups of the launch: the split-K grid, or (prefill) the CU count its order needs.
int launch_groups(const Plan& pl) {
    return pl.splitk ? sixi::decode_num_groups(pl.a, cu_count_cached(),
                                               sixi::decode_groups_per_cu(pl.kv_type, pl.row_tiles, pl.D, pl.generic))
                     : cu_count_cached();
}

// Launches a resolved call on `ws` (laid out as pl says).
int run(Plan& pl, char* ws, hipStream_t stream) {
    FaArgs& a = pl.a;
    hipError_t e;
    if (pl.q8_stage) {
        sixi::Q8StageArgs st{};
        st.q = a.q; st.q_nb1 = a.q_nb1; st.q_nb2 = a.q_nb2; st.q_nb3 = a.q_nb3;
        st.q_es = a.q_es; st.q_f16 = a.q_f16;
        st.k = a.k; st.k_nb1 = a.k_nb1; st.k_nb2 = a.k_nb2; st.k_nb3 = a.k_nb3;
        st.v = a.v; st.v_nb1 = a.v_nb1; st.v_nb2 = a.v_nb2; st.v_nb3 = a.v_nb3;
        st.pt = a.pt; st.pt_stride = a.pt_stride; st.n_pages = a.n_pages;
        st.kv_len = a.kv_len; st.q_len = a.q_len;
        st.S = a.S; st.H = a.H; st.Hkv = a.Hkv; st.n_q = a.n_q; st.n_kv = a.n_kv; st.D = pl.D;
        st.k16 = ws + pl.stage_k; st.v16 = ws + pl.stage_v; st.q16 = pl.splitk ? ws + pl.stage_q : nullptr;
        e = sixi::launch_q8_stage(st, stream);
        if (e != hipSuccess) return SIXI_E_BACKEND;
        const int64_t row = (int64_t)pl.D * 2;
        if (pl.splitk) {
            a.q = st.q16; a.q_nb2 = row; a.q_nb1 = (int64_t)a.H * row; a.q_nb3 = (int64_t)a.n_q * a.H * row;
            a.q_es = 2; a.q_f16 = 1;
        } else {
            a.q_q8 = 1;  // the prefill kernel converts Q to the q8_0 dot type itself
        }
        a.k = st.k16; a.k_nb2 = row; a.k_nb1 = (int64_t)a.Hkv * row; a.k_nb3 = (int64_t)a.n_kv * a.Hkv * row;
        a.v = st.v16; a.v_nb2 = row; a.v_nb1 = a.k_nb1; a.v_nb3 = a.k_nb3;
        a.pt = nullptr;  // the staged rows are one range per stream
    }
    if (pl.mask_prepass) {
        a.row_kl = reinterpret_cast<int32_t*>(ws + pl.prepass_offset);
        if (sixi::launch_mask_prefix(a, stream) != hipSuccess) return SIXI_E_BACKEND;
    }
    if (pl.q8_stage) ws += pl.stage_bytes;
    a.part = reinterpret_cast<float*>(ws);
    a.seg_pieces = pl.splitk ? reinterpret_cast<int32_t*>(ws + pl.seg_offset) : nullptr;
    a.P = launch_groups(pl);

    if (pl.splitk) {
        a.xcd_remap = 0;
        a.head_split = 0;
        a.piece_stride = 1;
        // every head of a GQA group in one launch (the split kernel and its merge), so each
        // K/V byte is read once for all of the group's rows
        e = sixi::launch_decode(a, pl.kv_type, pl.mask_mode, pl.D, pl.row_tiles, stream);
    } else {
        e = sixi::launch_prefill(a, pl.kv_type, pl.mask_mode, pl.D, stream);
    }
    if (e == hipErrorNotSupported) return SIXI_E_UNSUPPORTED;
    return e == hipSuccess ? SIXI_OK : SIXI_E_BACKEND;
}

}  // namespace

extern "C" {

int sixi_attn_validate(const sixi_attn_params* p) {
    Plan pl;
    return resolve(p, &pl);
}

int sixi_attn_workspace_bytes(const sixi_attn_params* p, size_t* bytes) {
    if (!bytes) return SIXI_E_INVALID_ARGUMENT;
    Plan pl;
    const int rc = resolve(p, &pl);
    if (rc != SIXI_OK) return rc;
    *bytes = pl.ws_bytes;
    return SIXI_OK;
}

int sixi_attn_forward(const sixi_attn_params* p) {
    Plan pl;
    int rc = resolve(p, &pl);
    if (rc != SIXI_OK) return rc;
    if (!p->workspace || p->workspace_bytes < pl.ws_bytes) return SIXI_E_OUT_OF_BOUNDS;
    if (!aligned(p->workspace, kWsAlign)) return SIXI_E_ALIGNMENT;
    // the kernels write the workspace while they read the views
    if (workspace_overlaps(p, p->workspace, pl.ws_bytes)) return SIXI_E_INVALID_ARGUMENT;
    return run(pl, static_cast<char*>(p->workspace), static_cast<hipStream_t>(p->stream));
}

int sixi_attn_forward_noalloc(const sixi_attn_params* p) {
    Plan pl;
    // stage a q8_0 cache only while the staging leaves room in the scratch for the rest
    int rc = resolve(p, &pl, kScratchBytes / 2);
    if (rc != SIXI_OK) return rc;
    // exact slots for this launch's work-groups, not the workspace bound of any launch
    if (pl.splitk) {
        splitk_layout(pl, (int64_t)pl.a.S * pl.a.Hkv + launch_groups(pl));
        prepass_layout(pl);
    }
    if (pl.ws_bytes > kScratchBytes) return SIXI_E_OUT_OF_BOUNDS;
    char* base = scratch_base();
    if (!base) return SIXI_E_BACKEND;
    return run(pl, base, static_cast<hipStream_t>(p->stream));
}

const char* sixi_attn_strerror(int code) {
    switch (code) {
        case SIXI_OK: return "ok";
        case SIXI_E_INVALID_ARGUMENT: return "invalid argument";
        case SIXI_E_OUT_OF_BOUNDS:
            return "out of bounds (workspace too small, or beyond the no-allocation entry point's fixed scratch)";
        case SIXI_E_INTEGER_OVERFLOW: return "integer overflow in view extents";
        case SIXI_E_ALIGNMENT: return "misaligned pointer or stride";
        case SIXI_E_BACKEND: return "HIP launch failed";
        case SIXI_E_UNSUPPORTED: return "shape or type not supported by the gfx950 kernels";
        default: return "unknown status";
    }
}

int sixi_attn_abi_version(void) { return SIXI_ATTN_ABI_VERSION; }

}  // extern "C"
