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
    int64_t k_nb1, k_nb2, k_nb3;  // (paged: k_nb3 is the page stride, see pt)
    const char* v;
    int64_t v_nb1, v_nb2, v_nb3;
    const int32_t* pt;     // paged KV: cell c of stream s in cell c % 256 of page
                           // pt[s*pt_stride + c/256] (clamped to [0, n_pages)); null: contiguous
    int64_t pt_stride;
    int32_t n_pages;

    char* out;             // row (d, h, j, s) at out + d*4 + h*o_nb1 + j*o_nb2 + s*o_nb3
    int64_t o_nb1, o_nb2, o_nb3;

    const int32_t* kv_len; // device, may be null; stream s's entry at kv_len[s * kv_len_stride]
    const int32_t* q_len;  // device, may be null
    int32_t kv_len_stride;

    // explicit masks (the ggml hook): the pre-pass's result per (stream s, row j) at
    // row_kl[s * n_q + j] -- the kv offset kl the row's mask implies when it is a block-causal
    // prefix (zeros on cells [0, kl + j + 1), -inf on the rest of the scanned cells),
    // kMaskNotPrefix when it is not, kMaskRowIdle for rows past the stream's q_len
    int32_t* row_kl;
    int32_t mask_inline;   // explicit mask, no table: one stream of one row whose mask row every
                           // work-group of the dual kernels reads itself (mask_rows_block_causal)

    const char* mask;      // EXPLICIT: f16 at mask + c*2 + j*m_nb1 + (s % m_ne3)*m_nb3
    int64_t m_nb1, m_nb3;
    int32_t m_ne3;
    int32_t mask_stage;    // EXPLICIT, rows j < 32 of a step staged through LDS (16-byte aligned
                           // rows); 0: read per cell from global memory
    uint32_t m_bytes;      // staged: bytes of a stream's mask rows the kernel may read
    int64_t m_span;        // EXPLICIT: bytes of a stream's n_q mask rows, (n_q-1)*nb1 + 2*ne[0]

    int32_t S, H, Hkv, G;  // streams, q heads, kv heads, H / Hkv
    int32_t Gr, hoff;      // heads of each GQA group this launch covers: hoff .. hoff+Gr-1
                           // (rows of a group = Gr * q_len, row r -> head g*G + hoff + r % Gr)
    int32_t n_q, n_kv;     // view extents (max rows per stream, cells per stream)
    float scale;           // softmax scale (already divided by the softcap when it is on)
    float scale_log2;      // scale * log2(e)
    float softcap;         // 0 = off
    float alibi_m0, alibi_m1;
    int32_t alibi_nlog2;   // 0 = ALiBi off

    // split-K bookkeeping (workspace)
    float* part;           // partial slots of slot_floats floats: O/l rows [rows][128] f16, then m, l
    int32_t P;             // work-groups of the split-K launch (prefill: CUs of the device)
    int32_t xcd_remap;     // 1: consecutive tile ranges go to work-groups of one XCD
    int32_t head_split;    // 1: the cost line runs over streams, and each range is taken by Hkv
                           // work-groups at once, one per kv-head (same cells, same start)
    int32_t piece_stride;  // slot of piece p of segment k: k + p * piece_stride
    int32_t tile_cells;    // KV cells per split tile (decode_tile_cells)
    int32_t seg_cost;      // tiles' worth of work charged to each segment in the split
    int64_t slot_floats;   // floats per partial slot
    int32_t* seg_pieces;   // per segment: logical work-groups of its first and last piece
    int32_t q_q8;          // prefill over an f16-staged q8_0 cache: convert Q to the q8_0 dot type
                           // in the kernel (ggml's rule), as the q8_0 kernels do

    const char* gate;      // fused output gate (SIXI_ATTN_FLAG_GATE), or null: element (d, h, j, s)
    int64_t g_nb1, g_nb2, g_nb3;  // at gate + d*4 + h*g_nb1 + j*g_nb2 + s*g_nb3 (qg's gate half)
};

// q8_0 KV in blocks beyond the decode kernels (prefill chunks, 128- and 256-dim heads), while the
// copy takes at most the staging cap and SIXI_ATTN_FLAG_BOUNDED_WORKSPACE is not set
// (fa_q8_stage.hip): K and V staged as dense f16 rows in the workspace (Q too where q16 is set),
// then the f16 prefill kernel.  k16/v16: [S][n_kv][Hkv][D], q16: [S][n_q][H][D].
struct Q8StageArgs {
    const char* q;
    int64_t q_nb1, q_nb2, q_nb3;
    int32_t q_es, q_f16;
    const char* k;
    int64_t k_nb1, k_nb2, k_nb3;
    const char* v;
    int64_t v_nb1, v_nb2, v_nb3;
    const int32_t* pt;     // paged source cache (as FaArgs::pt), or null
    int64_t pt_stride;
    int32_t n_pages;
    const int32_t* kv_len;
    const int32_t* q_len;
    int32_t S, H, Hkv, n_q, D;
    int64_t n_kv;
    char *k16, *v16, *q16;  // q16 null: Q is not staged (the prefill kernel converts it)
};

constexpr int32_t kMaskNotPrefix = INT32_MIN;
constexpr int32_t kMaskRowIdle = INT32_MIN + 1;

// Host-side launchers (defined in the .hip files).  hipErrorNotSupported = not built.
hipError_t launch_q8_stage(const Q8StageArgs& a, hipStream_t stream);
// The explicit-mask pre-pass (fa_mask.hip): fills a.row_kl from a.mask.
hipError_t launch_mask_prefix(const FaArgs& a, hipStream_t stream);
hipError_t launch_decode(const FaArgs& a, int kv_type, int mask_mode, int head_dim, int row_tiles,
                         hipStream_t stream);
hipError_t launch_prefill(const FaArgs& a, int kv_type, int mask_mode, int head_dim,
                          hipStream_t stream);

// Sizing rules shared by the dispatcher and the launchers.
constexpr int kDecodeTile = 16;        // KV cells per wave step of the 16-cell kernel (<= 48 rows)
constexpr int kDecodeTileWide = 32;    // KV cells per step of the f16 kernel for 49..96 rows
constexpr int kDecodeMaxRowTiles = 6;  // 16-row MFMA tiles per (stream, kv-head): G*q_len <= 96
constexpr int kMaxStreams = 512;       // LDS prefix table bound
constexpr int kPageCells = SIXI_KV_PAGE_CELLS;  // paged KV: cells per page (a multiple of every tile)
static_assert(kPageCells == 256, "page arithmetic below uses c >> 8 and c & 255");
constexpr int kMaxSplitGroups = 2048;  // work-groups of a split-K launch (workspace bound)
constexpr int kXcds = 8;               // MI355X: work-groups are dealt round-robin over 8 XCDs
int decode_num_groups(const FaArgs& a, int cu_count, int groups_per_cu);
// Whether the 32-cell kernel runs this launch: f16 KV with more than 48 rows or 256-dim heads,
// f16 KV under an explicit mask or a softcap (`generic`: the per-cell work needs the 512
// registers per wave of that kernel), and q8_0 KV with more than 48 rows, or under a mask or
// softcap with more than 16 (128-dim heads) or any rows (256-dim heads).  Everything else --
// f16 and q8_0 up to 48 rows at 128-dim heads, q8_0 up to 48 rows at 256-dim heads -- runs the
// 16-cell kernel, which dequantises q8_0 in registers.
inline bool decode_wide_kernel(int kv_type, int row_tiles, int head_dim, bool generic) {
    if (kv_type == SIXI_TYPE_Q8_0)
        return row_tiles > 3 || (generic && (head_dim == 256 || row_tiles > 1));
    return kv_type == SIXI_TYPE_F16 && (row_tiles > 3 || head_dim == 256 || generic);
}
// Work-groups per CU of the 16-cell kernel: two at 128-dim heads (256 registers per wave; one
// group per CU removes the few spills of q8_0 at 48 rows and of q8_0 under a mask, but halves
// the waves that hide the loads: the 8 x 64k q8_0 verify took 286 against 171 us), one at
// 256-dim heads (its rings and Q operands fill the LDS, and 48 rows of 256-dim accumulators
// need the 512 registers of one wave per SIMD).
constexpr int t16_groups_per_cu(int head_dim) { return head_dim == 256 ? 1 : 2; }
// Work-groups per CU of a decode launch (the 32-cell kernel runs one).
inline int decode_groups_per_cu(int kv_type, int row_tiles, int head_dim, bool generic) {
    return decode_wide_kernel(kv_type, row_tiles, head_dim, generic) ? 1 : t16_groups_per_cu(head_dim);
}
// Cells per split tile of the decode launch.
inline int decode_tile_cells(int kv_type, int row_tiles, int head_dim, bool generic) {
    return decode_wide_kernel(kv_type, row_tiles, head_dim, generic) ? kDecodeTileWide : kDecodeTile;
}
// Fixed cost of starting a piece (loading Q, filling the ring, merging and writing the
// rows), in tiles of the split: each segment weighs tiles + seg_cost, so a work-group whose
// range enters a segment gets that many tiles less.
// (f16 at 128-dim heads, the pipelined kernel: 16; interleaved sweep on the 32 x 16 verify, 8 / 12
// / 16 / 24 / 32 tiles: 149.2 / 145.4 / 144.0 / 145.2 / 147.4 us.  q8_0 at 128-dim heads, 32 x 16
// verify, 8 / 12 / 16 / 20: 167.0 / 163.4 / 163.0 / 164.6 us.  256-dim heads, whose tiles are twice
// the bytes, 32 x 16 verify at 2 / 4 / 6 / 8 / 12 tiles: f16 278.7 / 274.7 / 272.1 / 271.5 / 274.0 us,
// q8_0 387.6 / 383.3 / 382.4 / 384.6 / 389.0 us.)
constexpr int kWideSegCost = 12;
constexpr int kWideSegCostF16D128 = 16;
constexpr int kWideSegCostD256 = 6;
inline int decode_seg_cost(int kv_type, int row_tiles, int head_dim, bool generic) {
    if (!decode_wide_kernel(kv_type, row_tiles, head_dim, generic)) return 0;
    if (head_dim == 256) return kWideSegCostD256;
    return kv_type == SIXI_TYPE_F16 ? kWideSegCostF16D128 : kWideSegCost;
}
// Row tiles the decode kernel runs for `rows` = G * n_q rows, i.e. exactly the rows of the
// launched kernel's partial slots (16 per tile): up to 3 per wave on the 16-cell kernel, beyond
// that two row groups of equal size (so 5 tiles run as 6); the 32-cell kernel holds at most
// two per wave at 256-dim heads, so there 3 tiles run as two row groups of two.
inline int decode_row_tiles(int64_t rows, int head_dim, int kv_type, bool generic) {
    const int rt = (int)((rows + 15) / 16);
    if (rt <= 2 || (rt == 3 && !decode_wide_kernel(kv_type, rt, head_dim, generic))) return rt;
    if (rt == 3 && head_dim != 256) return rt;
    return 2 * ((rt + 1) / 2);
}
// Explicit-mask split-K calls that take the mask pre-pass (fa_mask.hip) and its dual kernels,
// planned as the lengths-only call of the same shape (`row_tiles` without the per-cell
// mode): every shape of the 16-cell kernel (its fallback is the per-cell mode), and the
// 32-cell kernels' shapes where their staged-mask mode can read the mask (mask_stage).
inline bool mask_prepass_decode(int kv_type, int row_tiles, int head_dim, bool mask_stage) {
    return mask_stage || !decode_wide_kernel(kv_type, row_tiles, head_dim, false);
}
// Rows (streams x rows per stream) of a call that takes the pre-pass: every work-group of the
// dual kernels reads the table once.
constexpr int64_t kMaskPrepassMaxRows = 16384;
// Cells of a single-stream, single-row call's mask row that every work-group of the dual
// kernels reads itself instead of a pre-pass launch (single-stream decode).
constexpr int64_t kMaskInlineMaxCells = 16384;

inline int64_t decode_slot_floats(int row_tiles, int head_dim) {
    // O/l rows [16*row_tiles][head_dim] f16 (head_dim/2 floats' worth), then m and l per row
    return (int64_t)row_tiles * 16 * (head_dim / 2 + 2);
}

}  // namespace sixi
