// fa_decode.hip -- split-K flash-decoding for single-token decode and speculative verify
// on gfx950 (head_dim 128 and 256, f16 or q8_0 KV, up to 96 rows per GQA group).
//
// Work decomposition.  A segment is one (stream s, kv-head g): nt_s tiles of KV cells, and
// all R = G*q_len_s query rows of the GQA group ride along with every tile, so each K/V
// byte leaves HBM once for the whole group.  Segments are laid end to end (stream-major,
// then kv-head) on a cost line where each weighs seg_cost + nt_s units, and the P
// work-groups take equal shares [p*T/P, (p+1)*T/P) of it ("stream-K"), so any mix of
// lengths balances over the CUs and a work-group that has to start an extra segment gets
// correspondingly fewer tiles.  The share of work-group p inside a segment is a piece.  A
// work-group that owns a whole segment writes the rows directly; every other piece leaves
// (m, l, O) in a workspace slot, and a second launch combines the pieces of each split
// segment in a fixed order (decode_merge_rows; decode_merge_pieces for segments of many pieces).  The kernel boundary orders the two launches, so
// neither needs device-scope fences or atomics.
//
// Three kernels share this split:
//   decode_t16 (<= 48 rows: f16 and q8_0 at 128-dim heads, q8_0 at 256): tiles of 16 cells;
//     four waves per work-group (two work-groups per CU at 128-dim heads, one at 256), the
//     waves independent tile lanes with private LDS rings (no barrier in the tile loop).
//     Described next.
//   decode_wide (f16 KV: 49..96 rows of 128-dim heads, any rows of 256-dim heads, and f16
//     calls under a mask or softcap): steps of 32 cells; described further down.
//   decode_wide_q8 (q8_0 KV beyond the 16-cell kernel): the 32-cell kernel over q8_0 rows
//     converted to f16 in LDS.
// Calls with an explicit ggml mask first run the mask pre-pass (fa_mask.hip); their kernels
// (the *_dual forms) then choose on the device between the lengths-only body over the offsets
// the mask implies and the mask body.
// K/V reach LDS by direct global->LDS loads (buffer_load_dword{,x4} ... lds), so bytes in
// flight cost no VGPRs.  f16 rows go in with the non-temporal policy (nt): each is read by one
// work-group once and fills whole cache lines, so it should leave L2 before the lines that are
// reused (Q, partial slots, page tables, q8_0 lines shared by neighbouring heads); measured
// 138.2 -> 128.8 us on the 32 x 16 verify over head-major pages, 237.9 -> 208.5 us on the
// 256-dim 32 x 4 verify.  q8_0 rows keep the default policy (nt measured 23% slower on the
// long q8_0 decode: a 136-byte head row shares lines with the next head's).
//
// decode_t16, per 16-cell tile and wave (128-dim heads; 256-dim heads run twice the k-steps
// and output tiles):
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16, A = 16 cells x 32 dims straight from the ring
//                 (lane (r, c) holds cell r, dims 32ks+8c..+7), B = Q^T from LDS;
//                 lane (r, c) receives cells 4c..4c+3 of row r;
//   softmax       row max over the four lane groups with v_permlane{32,16}_swap; the
//                 exponent reference moves lazily (only when the tile max exceeds it by
//                 more than 2^8), so the O rescale is rare; p = 2^(s*c - m*c) in one FMA;
//   O^T += V^T P^T  v_mfma_f32_16x16x16_f16: B = P^T is exactly the lane's own four
//                 probabilities, A = V^T from an in-register 4x8 16-bit transpose
//                 (v_perm_b32) of the four 16-byte V rows the lane staged (cells 4c..4c+3,
//                 dims 8r..8r+7), so output tile tt holds dims 8r + tt.
// Only the tiles that reach past the first causal boundary (or the stream's end) apply a
// mask; the rest run the unmasked body.
//
// q8_0 KV (ggml blocks {f16 d; int8 q[32]}, 136 B per 128-dim head row, only 4-byte aligned)
// uses the same core: the raw rows of a tile are copied to LDS with dword LDS-DMA
// (buffer_load_dword ... lds), each lane pulls the eight int8 values of its operand with
// aligned dword reads and v_alignbyte_b32, and dequantises them in registers
// (dequant_q8x8: one f16 rounding of q*d).  Q is quantised to q8_0 exactly as ggml's
// flash_attn_ext does before the dot (per 32-dim block, d = amax/127) and enters the MFMA as
// its dequantised f16 values.
#include <type_traits>

#include "fa_device.hpp"

namespace sixi {
namespace {

constexpr int kTile = kDecodeTile;  // 16 cells
constexpr int kQ8Row = 136;         // bytes of one q8_0 head row (4 blocks of 34)
constexpr int kQ8Dma = 9;           // dword LDS-DMA loads covering 16 q8_0 rows (2304 >= 2176 B)
constexpr float kLazyLog2 = 8.0f;   // headroom (log2 units) before the exponent reference moves
constexpr int kMaxPieces = 64;      // target bound on the pieces of one full-length segment

// FAST: no mask beyond the lengths; MASK: an explicit ggml mask staged through LDS, no softcap
// and no ALiBi (the drop-in's case); GENERIC: everything else (softcap, ALiBi, masks read from
// global memory).  FAST and MASK keep scores as raw dot products and exponent references in
// those units; GENERIC works with log2-domain logits.
enum { MODE_FAST = 0, MODE_GENERIC = 1, MODE_MASK = 2 };
template <int MODE> constexpr bool raw_units() { return MODE != MODE_GENERIC; }

// Per-stream (rows, cached cells), kept in LDS so that a piece reads its extents there.
struct StreamTable {
    int ps[kMaxStreams + 1];  // inclusive tile prefix over streams
    int2 dims[kMaxStreams];   // (ql, kl) of every stream
};
// (every lane reads the same entry; readfirstlane tells the compiler the values are uniform)
__device__ __forceinline__ StreamDims table_dims(const StreamTable& t, int s) {
    StreamDims d;
    d.ql = __builtin_amdgcn_readfirstlane(t.dims[s].x);
    d.kl = __builtin_amdgcn_readfirstlane(t.dims[s].y);
    d.nc = d.ql > 0 ? d.kl + d.ql : 0;
    return d;
}

// Per head dim of the 16-cell kernel: k-steps of 32 dims (KS), output tiles of 16 dims (DT),
// dims of a V row that one lane stages (VD), bytes of a q8_0 head row (Q8ROW).
template <int D> struct T16Dim;
template <> struct T16Dim<128> { static constexpr int KS = 4, DT = 8, VD = 8, Q8ROW = kQ8Row; };
template <> struct T16Dim<256> { static constexpr int KS = 8, DT = 16, VD = 16, Q8ROW = 2 * kQ8Row; };

// Per KV type and head dim: bytes of one ring slot (one 16-cell tile of K and V), LDS-DMA loads
// a tile takes per wave, and the byte offset of V in the slot.  256-dim q8_0 rows (272 B,
// 16-byte aligned) come in as five 1 KB loads each for K and V (4352 B of rows, then spare).
template <int KV, int D> struct KvTile;
template <> struct KvTile<SIXI_TYPE_F16, 128> { static constexpr int slot_bytes = 8192, dma = 8, v_off = 4096; };
template <> struct KvTile<SIXI_TYPE_Q8_0, 128> {
    static constexpr int slot_bytes = 2 * kQ8Dma * 256, dma = 2 * kQ8Dma, v_off = kQ8Dma * 256;
};
template <> struct KvTile<SIXI_TYPE_Q8_0, 256> { static constexpr int slot_bytes = 2 * 5 * 1024, dma = 10, v_off = 5 * 1024; };

// Four independent tile lanes (one wave each) per work-group: two work-groups per CU at
// 128-dim heads, one at 256 (t16_groups_per_cu).
template <int KV> struct Shape;
template <> struct Shape<SIXI_TYPE_F16> { static constexpr int waves = 4, lanes = 4, slots = 2; };
template <> struct Shape<SIXI_TYPE_Q8_0> { static constexpr int waves = 4, lanes = 4, slots = 3; };

template <int NT, int NS, int DT = 8>
struct MergeBuf {
    f32x4 o[NS][NT * DT * 64];  // [slot][n*DT + tt][lane]
    float m[NS][NT * 64];
    float l[NS][NT * 64];
};

// NTW = row tiles per wave.
template <int NTW, int KV, int D = 128>
struct DecodeLds {
    using Sh = Shape<KV>;
    union {
        struct {
            u32x4 ring[Sh::lanes * Sh::slots * KvTile<KV, D>::slot_bytes / 16];
            u32x4 q[NTW * T16Dim<D>::KS * 64];  // Q^T B operands: [row tile][ks][lane], 8 f16 each
        } t;
        MergeBuf<NTW, Sh::lanes / 2, T16Dim<D>::DT> mg;  // reused after the tile loop
    };
    int ps[kMaxStreams + 1];  // (no extents table: it would not leave room for two groups per CU)
};

template <int NT, int DT = 8>
struct Acc {
    f32x4 o[DT][NT];  // O^T tiles of 16 dims (the kernels state which dims each lane holds)
    float m[NT];     // exponent reference: raw score (FAST) or log2 units (GENERIC, merged)
    float l[NT];     // this lane's share of the row sum until the end of the tile loop
};

template <int NT, int DT>
__device__ __forceinline__ void acc_clear(Acc<NT, DT>& acc) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        acc.m[n] = neg_inf();
        acc.l[n] = 0.0f;
#pragma unroll
        for (int t = 0; t < DT; ++t) acc.o[t][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
}

// (m, l, O) <- merge of (m, l, O) and (m2, l2, O2), log2-domain references.
template <int K>
__device__ __forceinline__ void merge_row(float& m, float& l, f32x4* o, float m2, float l2,
                                          const f32x4* o2) {
    const float mn = fmaxf(m, m2);
    const float ms = (mn == neg_inf()) ? 0.0f : mn;
    const float a1 = fast_exp2(m - ms);
    const float a2 = fast_exp2(m2 - ms);
    l = l * a1 + l2 * a2;
    m = mn;
#pragma unroll
    for (int t = 0; t < K; ++t) o[t] = o[t] * a1 + o2[t] * a2;
}

template <int NT, int NS, int DT>
__device__ __forceinline__ void acc_to_lds(MergeBuf<NT, NS, DT>& mg, int slot, const Acc<NT, DT>& acc, int lane) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int t = 0; t < DT; ++t) mg.o[slot][(n * DT + t) * 64 + lane] = acc.o[t][n];
        mg.m[slot][n * 64 + lane] = acc.m[n];
        mg.l[slot][n * 64 + lane] = acc.l[n];
    }
}

template <int NT, int NS, int DT>
__device__ __forceinline__ void acc_merge_lds(const MergeBuf<NT, NS, DT>& mg, int slot, Acc<NT, DT>& acc, int lane) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        f32x4 o[DT], o2[DT];
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            o[t] = acc.o[t][n];
            o2[t] = mg.o[slot][(n * DT + t) * 64 + lane];
        }
        merge_row<DT>(acc.m[n], acc.l[n], o, mg.m[slot][n * 64 + lane], mg.l[slot][n * 64 + lane], o2);
#pragma unroll
        for (int t = 0; t < DT; ++t) acc.o[t][n] = o[t];
    }
}

// Merges the tile lanes of each row group into tile lane 0: with four lanes (2,3) -> (0,1)
// then 1 -> 0, with two lanes 1 -> 0, with one lane nothing.  Every wave must call it.
// Returns whether this wave owns its rows afterwards.
template <int NTW, int TL, int NS, int DT>
__device__ __forceinline__ bool merge_lanes(MergeBuf<NTW, NS, DT>& mg, Acc<NTW, DT>& acc, int rg, int tl, int lane) {
    constexpr int H = TL / 2;  // merge slots per row group
    static_assert(TL == 1 || TL == 2 || TL == 4, "tile lanes");
    if (TL == 1) return true;
    if (TL == 4) {
        if (tl >= 2) acc_to_lds(mg, H * rg + tl - 2, acc, lane);
        __syncthreads();
        if (tl < 2) acc_merge_lds(mg, H * rg + tl, acc, lane);
        __syncthreads();
    }
    if (tl == 1) acc_to_lds(mg, H * rg, acc, lane);
    __syncthreads();
    if (tl == 0) acc_merge_lds(mg, H * rg, acc, lane);
    return tl == 0;
}

// Inclusive prefix of segment costs over streams into ps[0..S] (a stream with rows weighs
// tiles + seg_cost per kv-head) and, if given, the stream extents (run by one wave).
__device__ __forceinline__ void build_tile_prefix(const FaArgs& a, int* ps, int2* dims = nullptr) {
    const int lane = threadIdx.x & 63;
    if (lane == 0) ps[0] = 0;
    int carry = 0;
    for (int base = 0; base < a.S; base += 64) {
        const int s = base + lane;
        int x = 0;
        if (s < a.S) {
            const StreamDims d = stream_dims(a, s < a.S ? s : 0);
            x = d.nc > 0 ? (d.nc + a.tile_cells - 1) / a.tile_cells + a.seg_cost : 0;
            if (dims) dims[s] = int2{d.ql, d.kl};
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (s < a.S) ps[s + 1] = carry + x;
        carry += __shfl(x, 63, 64);
    }
}

// Per-piece constants of one lane.
template <int NT>
struct RowInfo {
    int vis[NT];     // cells visible to the lane's row of tile n (non-explicit masks)
    int j[NT];       // block row of the lane's row of tile n
    float slope[NT]; // ALiBi slope (explicit masks)
};

// One 16-cell tile from a staged ring slot.  MASKED applies the visibility of each row;
// `after_reads` runs once the slot's LDS reads are consumed.  The phases run over all row
// tiles at once (every QK^T, then every row max, one rare rescale branch, then every
// exponential and PV), so each phase offers the scheduler NT independent chains.
template <int NT, int KV, int MODE, bool MASKED, int D, typename F>
__device__ __forceinline__ void tile_step(const FaArgs& a, Acc<NT, T16Dim<D>::DT>& acc, const u32x4* slot,
                                          const u32x4* qs, int c0, const RowInfo<NT>& ri,
                                          const char* mrow, int nc, int lane, F&& after_reads) {
    using TD = T16Dim<D>;
    constexpr int KS = TD::KS, DT = TD::DT, VH = TD::VD / 8;
    static_assert(D == 128 || KV == SIXI_TYPE_Q8_0, "256-dim heads: q8_0 only");
    const int c = lane >> 4;
    const int r = lane & 15;

    // K operands (cell r, dims 32ks + 8c .. +7) and V rows (cells 4c + e, dims VD*r .. +VD-1,
    // as VH groups of eight f16)
    f16x8 kop[KS];
    u32x4 vr[4][VH];
    if constexpr (KV == SIXI_TYPE_F16) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kop[ks] = as_f16x8(slot[ks * 64 + lane]);
#pragma unroll
        for (int e = 0; e < 4; ++e) vr[e][0] = slot[(4 + e) * 64 + lane];
    } else {
        // raw q8_0 rows packed at Q8ROW bytes: block b of row x holds d at x*Q8ROW + 34b and the
        // int8 values at x*Q8ROW + 34b + 2 (2 bytes past a dword boundary for even b)
        constexpr int RB = TD::Q8ROW;
        const uint32_t* kraw = reinterpret_cast<const uint32_t*>(slot);
        const uint32_t* vraw = kraw + KvTile<KV, D>::v_off / 4;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint32_t w0, w1;
            ld8_at(kraw, r * RB + 34 * ks + 2 + 8 * c, (ks & 1) == 0, w0, w1);
            kop[ks] = as_f16x8(dequant_q8x8(w0, w1, ld_half_at(kraw, r * RB + 34 * ks)));
        }
        // the lane's VD dims lie in block b at byte VD * (r % (32 / VD)) of its quants
        const int b = (TD::VD * r) >> 5;
        const int qo = 2 + TD::VD * (r & (32 / TD::VD - 1));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int x = 4 * c + e;
            const uint16_t dv = ld_half_at(vraw, x * RB + 34 * b);
            if constexpr (VH == 1) {
                uint32_t w0, w1;
                ld8_at(vraw, x * RB + 34 * b + qo, (b & 1) == 0, w0, w1);
                vr[e][0] = dequant_q8x8(w0, w1, dv);
            } else {
                uint32_t w[4];
                ld16_at_any(vraw, x * RB + 34 * b + qo, w);
                vr[e][0] = dequant_q8x8(w[0], w[1], dv);
                vr[e][1] = dequant_q8x8(w[2], w[3], dv);
            }
        }
    }

    // ---- S^T = K Q^T for every row tile ----
    f32x4 st[NT];
    // Raised wave priority while a wave issues its MFMAs (here and around O^T += V^T P^T below):
    // at 128-dim heads two work-groups share a CU, so two waves share each SIMD, and the one with
    // matrix work goes first while the other dequantises (the 8 x 64k q8_0 verify, 48 rows:
    // 161.9 -> 157.9 us; the other calls unchanged, outputs bitwise equal).  At 256-dim heads a
    // wave has its SIMD to itself.
    if constexpr (D == 128) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        st[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) st[n] = mfma16x16x32(kop[ks], as_f16x8(qs[(n * KS + ks) * 64 + lane]), st[n]);
    }
    if constexpr (D == 128) __builtin_amdgcn_s_setprio(0);
    after_reads();

    // V^T operands: tile tt holds dim VD*r + tt of cells 4c..4c+3
    u32x2 vt[DT];
#pragma unroll
    for (int tt = 0; tt < DT; ++tt) {
        const int h = tt >> 3, d2 = (tt & 7) >> 1;
        const uint32_t sel = (tt & 1) ? 0x07060302u : 0x05040100u;
        vt[tt][0] = __builtin_amdgcn_perm(vr[1][h][d2], vr[0][h][d2], sel);
        vt[tt][1] = __builtin_amdgcn_perm(vr[3][h][d2], vr[2][h][d2], sel);
    }

    // ---- scores (FAST: raw dot products; GENERIC: log2-domain logits) and row maxima ----
    const float c2 = a.scale_log2;
    float sv[NT][4];
    float mx[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int cell = c0 + 4 * c + e;
            float x = st[n][e];
            if (MODE == MODE_GENERIC) {
                x *= a.scale;
                if (a.softcap != 0.0f) x = a.softcap * tanhf(x);
                if (a.mask) {
                    float mv = neg_inf();
                    if (cell < nc) {
                        const uint16_t bits = *reinterpret_cast<const uint16_t*>(
                            mrow + (int64_t)ri.j[n] * a.m_nb1 + (int64_t)cell * 2);
                        mv = ri.slope[n] * half_bits_to_float(bits);
                    }
                    x = (mv == neg_inf()) ? neg_inf() : x + mv;
                } else if (cell >= ri.vis[n]) {
                    x = neg_inf();
                }
                x *= kLog2e;
            } else if (MASKED) {
                if (cell >= ri.vis[n]) x = neg_inf();
            }
            sv[n][e] = x;
        }
        mx[n] = max4_rowgroups(max3f(sv[n][0], sv[n][1], fmaxf(sv[n][2], sv[n][3])));
    }

    // ---- lazy exponent reference: move it only when the tile max exceeds it by 2^8 ----
    // (the first tile of a piece always moves it; O and l are zero then)
    const float thr = (MODE == MODE_FAST) ? kLazyLog2 / c2 : kLazyLog2;
    bool need[NT];
    bool need_any = false;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        need[n] = mx[n] > acc.m[n] + thr;
        need_any |= need[n];
    }
    if (__builtin_amdgcn_ballot_w64(need_any) != 0) {
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            float alpha = 1.0f;
            if (need[n]) {
                alpha = fast_exp2((MODE == MODE_FAST) ? (acc.m[n] - mx[n]) * c2 : acc.m[n] - mx[n]);
                acc.m[n] = mx[n];
            }
            acc.l[n] *= alpha;
#pragma unroll
            for (int t = 0; t < DT; ++t) acc.o[t][n] *= alpha;
        }
    }

    // ---- probabilities (f32 row sums, f16 MFMA operand) and O^T += V^T P^T ----
    if constexpr (D == 128) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const float ref = acc.m[n];
        const float mc = (ref == neg_inf()) ? 0.0f : ((MODE == MODE_FAST) ? ref * c2 : ref);
        f16x4 pf;
        float ps[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            ps[e] = fast_exp2((MODE == MODE_FAST) ? fmaf(sv[n][e], c2, -mc) : sv[n][e] - mc);
            pf[e] = (_Float16)ps[e];
        }
        acc.l[n] += (ps[0] + ps[1]) + (ps[2] + ps[3]);

        if (MODE == MODE_GENERIC && a.mask) {
            // explicit masks: a cell that none of these 16 rows sees may hold NaN bits, so
            // its V^T column is zeroed for them (0 * NaN must not reach the accumulator)
            uint32_t keep[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint64_t b0 = __builtin_amdgcn_ballot_w64((float)pf[2 * h] != 0.0f);
                const uint64_t b1 = __builtin_amdgcn_ballot_w64((float)pf[2 * h + 1] != 0.0f);
                keep[h] = ((((b0 >> (16 * c)) & 0xffffull) != 0) ? 0x0000ffffu : 0u) |
                          ((((b1 >> (16 * c)) & 0xffffull) != 0) ? 0xffff0000u : 0u);
            }
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                const u32x2 vm = {vt[tt][0] & keep[0], vt[tt][1] & keep[1]};
                acc.o[tt][n] = mfma16x16x16(__builtin_bit_cast(f16x4, vm), pf, acc.o[tt][n]);
            }
        } else {
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
                acc.o[tt][n] = mfma16x16x16(__builtin_bit_cast(f16x4, vt[tt]), pf, acc.o[tt][n]);
        }
    }
    if constexpr (D == 128) __builtin_amdgcn_s_setprio(0);
}

// Writes the normalised rows of row tiles n0 .. n0+NT-1 held by this lane: dims
// (D/4)c + DT*i + tt of row 16n + r at o[tt][n][i].  (With the fused output gate the merge
// kernel gates these rows afterwards.)
template <int NT, int DT>
__device__ __forceinline__ void write_rows(const FaArgs& a, const Acc<NT, DT>& acc, int n0, int s, int g,
                                           int R, int lane) {
    // (the row addresses are computed here: hoisted out of the piece loop they would be held,
    // as 64-bit values, across every piece's steps, and spilled)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r = ln & 15, c = ln >> 4;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const int row = 16 * (n0 + n) + r;
        if (row >= R) continue;
        const int j = row / a.Gr;
        const int h = g * a.G + a.hoff + row % a.Gr;
        const float inv = acc.l[n] == 0.0f ? 0.0f : 1.0f / acc.l[n];
        char* dst = a.out + (int64_t)j * a.o_nb2 + (int64_t)h * a.o_nb1 + (int64_t)s * a.o_nb3 + c * 4 * DT * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int t = 0; t < DT; t += 4)
                st16(dst + (i * DT + t) * 4,
                     f32x4{acc.o[t][n][i], acc.o[t + 1][n][i], acc.o[t + 2][n][i], acc.o[t + 3][n][i]} * inv);
    }
}

// Partial slot of `rows_slot` rows: normalised O rows [row][128] f16 (O/l, a convex
// combination of f16 V rows, so it fits f16 and rounds by at most 2^-11 relative), then
// m[row] and l[row] in f32 (log2-domain references).
template <int NT, int DT>
__device__ __forceinline__ void write_partial(float* slot, int rows_slot, int n0, int R, const Acc<NT, DT>& acc,
                                              int lane) {
    constexpr int D = 16 * DT;
    // (row offsets computed here, not held across the piece loop; see write_rows)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r = ln & 15, c = ln >> 4;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const int row = 16 * (n0 + n) + r;
        if (row >= R) continue;
        const float inv = acc.l[n] == 0.0f ? 0.0f : 1.0f / acc.l[n];
        char* dst = reinterpret_cast<char*>(slot) + (int64_t)row * (2 * D) + c * (D / 2);  // dims (D/4)c ..
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int t0 = 0; t0 < DT; t0 += 8) {
                f16x8 h;
#pragma unroll
                for (int t = 0; t < 8; ++t) h[t] = (_Float16)(acc.o[t0 + t][n][i] * inv);
                *reinterpret_cast<u32x4*>(dst + (i * DT + t0) * 2) = as_u32x4(h);
            }
        if (c == 0) {
            slot[(int64_t)rows_slot * (D / 2) + row] = acc.m[n];
            slot[(int64_t)rows_slot * (D / 2 + 1) + row] = acc.l[n];
        }
    }
}

// Work-group-uniform description of one piece.
struct Piece {
    int s, g, tb, te, nt_seg;
    int64_t slot;  // partial slot (segment + logical work-group)
};

// One piece: tiles [tb, te) of segment (s, g), for row tiles n0 .. n0 + NTW - 1 of the NTOT
// that the launch's partial slots hold (all of them, n0 = 0, except in the per-row-tile
// fallback of the dual kernel).
template <int NTW, int KV, int MODE, int D, int NTOT = NTW>
__device__ __forceinline__ void decode_piece(const FaArgs& a, DecodeLds<NTOT, KV, D>& sh, int causal, const Piece& pc,
                                             int n0 = 0) {
    using TD = T16Dim<D>;
    constexpr int KS = TD::KS, DCH = D / 8;  // k-steps; 8-dim chunks of a Q row
    constexpr int TL = Shape<KV>::lanes;   // tile lanes (one wave each)
    constexpr int NSLOT = Shape<KV>::slots;
    constexpr int NTHREADS = Shape<KV>::waves * 64;
    constexpr int SLOT16 = KvTile<KV, D>::slot_bytes / 16;
    constexpr int DMA = KvTile<KV, D>::dma;  // LDS-DMA loads per tile per wave
    static_assert(Shape<KV>::waves == TL, "one row group");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int rg = 0;
    const int tl = w;
    const int r = lane & 15;
    const int c = lane >> 4;
    const int s = pc.s, g = pc.g, tb = pc.tb, te = pc.te;
    const StreamDims sd = stream_dims(a, s);
    const int G = a.Gr;                 // rows of one block row (heads of this launch)
    const int hb = g * a.G + a.hoff;    // first of those heads
    const int R = G * sd.ql;
    (void)rg;

    // ---- Q rows of the group -> f16 B operands in LDS (row 16n+r, dims 32ks+8c..+7) ----
    // Item idx = tid + k*NTHREADS is row 16 n0 + idx/DCH, 8-dim chunk idx%DCH.  Every load is
    // issued before any is used (padding rows read row 0, which every piece has), so the
    // staging costs one memory latency.
    constexpr int QIT = NTW * 16 * DCH / NTHREADS;
    static_assert(QIT * NTHREADS == NTW * 16 * DCH, "Q items per thread");
    const char* qsrc[QIT];
    bool qok[QIT];
#pragma unroll
    for (int k = 0; k < QIT; ++k) {
        const int idx = tid + k * NTHREADS;
        const int row = 16 * n0 + idx / DCH;
        qok[k] = row < R;
        const int rr = qok[k] ? row : 0;
        qsrc[k] = a.q + (int64_t)(rr / G) * a.q_nb1 + (int64_t)(hb + rr % G) * a.q_nb2 + (int64_t)s * a.q_nb3 +
                  (int64_t)(idx % DCH) * 8 * a.q_es;
    }
    float xv[QIT][8];
    if (a.q_f16) {
        u32x4 raw[QIT];
#pragma unroll
        for (int k = 0; k < QIT; ++k) raw[k] = ld16(qsrc[k]);
#pragma unroll
        for (int k = 0; k < QIT; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[k][e] = (float)as_f16x8(raw[k])[e];
    } else {
        f32x4 lo[QIT], hi[QIT];
#pragma unroll
        for (int k = 0; k < QIT; ++k) {
            lo[k] = *reinterpret_cast<const f32x4*>(qsrc[k]);
            hi[k] = *reinterpret_cast<const f32x4*>(qsrc[k] + 16);
        }
#pragma unroll
        for (int k = 0; k < QIT; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xv[k][e] = lo[k][e];
                xv[k][4 + e] = hi[k][e];
            }
    }
#pragma unroll
    for (int k = 0; k < QIT; ++k) {
        f16x8 hv;
        if constexpr (KV == SIXI_TYPE_Q8_0) {
            // ggml converts Q to the K dot type: q8_0 per 32-dim block, d = amax/127,
            // q = round-half-away(x * 127/amax) clamped to +-127; the MFMA takes q*d
            float am = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(xv[k][e]));
            am = fmaxf(am, __shfl_xor(am, 1, 64));
            am = fmaxf(am, __shfl_xor(am, 2, 64));
            const float d = am / 127.0f;
            const float id = d != 0.0f ? 127.0f / am : 0.0f;
            const _Float16 dh = (_Float16)d;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float qv = fminf(fmaxf(roundf(xv[k][e] * id), -127.0f), 127.0f);
                hv[e] = (_Float16)(qv * (float)dh);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = (_Float16)xv[k][e];
        }
        const int idx = tid + k * NTHREADS;
        const int row = 16 * n0 + idx / DCH;
        const int chunk = idx % DCH;  // ks = chunk/4, c = chunk%4
        const int n = row >> 4, rr = row & 15, ks = chunk >> 2, cc = chunk & 3;
        sh.t.q[(n * KS + ks) * 64 + cc * 16 + rr] = qok[k] ? as_u32x4(hv) : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();

    RowInfo<NTW> ri;
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        const int row = 16 * (n0 + n) + r;
        const bool valid = row < R;
        const int j = valid ? row / G : 0;
        ri.j[n] = j;
        ri.vis[n] = (valid && causal) ? sd.kl + j + 1 : sd.nc;
        ri.slope[n] = (MODE == MODE_GENERIC) ? alibi_slope(a, hb + (valid ? row % G : 0)) : 1.0f;
    }
    // tiles below t_full see no masked cell for any row
    const int t_full = (MODE == MODE_GENERIC) ? 0 : (causal ? (sd.kl + 1) / kTile : sd.nc / kTile);
    const char* mrow = nullptr;
    if (MODE == MODE_GENERIC && a.mask) mrow = a.mask + (int64_t)(s % a.m_ne3) * a.m_nb3;
    const u32x4* qs = sh.t.q + n0 * KS * 64;

    Acc<NTW, TD::DT> acc;
    acc_clear(acc);

    // K/V of this (stream, kv-head), per tile through range-checked buffer resources based at
    // the tile's first cell (in its page, for paged caches): cells >= nc read as zeros (and are
    // masked), so the tail tile needs no clamping and cannot fault.
    const int64_t rowb = (KV == SIXI_TYPE_F16) ? D * 2 : TD::Q8ROW;
    const uint32_t knb = (uint32_t)a.k_nb1, vnb = (uint32_t)a.v_nb1;

    // tiles of this lane: tb + tl + TL*i, i < n_my
    const int t0 = tb + tl;
    const int n_my = t0 < te ? (te - t0 + TL - 1) / TL : 0;
    u32x4* ring = sh.t.ring + (size_t)tl * NSLOT * SLOT16;
    const uint32_t ring_base = lds_addr(ring);

    // q8_0: unit t = 64u + lane of the packed 16-row tile (a dword at 128-dim heads, 16 bytes
    // at 256) is unit t % UPR of row t / UPR; lanes past the 16 rows repeat the last unit into
    // the slot's spare tail
    constexpr int Q8U = (D == 128) ? 4 : 16;          // bytes per lane and load
    constexpr int UPR = TD::Q8ROW / Q8U;              // units per row: 34 dwords or 17 x 16 B
    constexpr int Q8L = (D == 128) ? kQ8Dma : 5;      // loads per K (or V) of a tile
    uint32_t q8_cell[Q8L], q8_dw[Q8L];
    if constexpr (KV == SIXI_TYPE_Q8_0) {
#pragma unroll
        for (int u = 0; u < Q8L; ++u) {
            const int t = 64 * u + lane;
            const bool in = t < 16 * UPR;
            q8_cell[u] = in ? t / UPR : 15;
            q8_dw[u] = in ? t % UPR : UPR - 1;
        }
    }

    // Stage tile i of this lane into slot i % NSLOT.
    PageIds pages = page_ids_load(a, s, (t0 * kTile) >> 8);
    auto issue = [&](int i) {
        // uniform over the wave (the compiler cannot tell): scalar page and span arithmetic
        const int c0 = __builtin_amdgcn_readfirstlane((t0 + i * TL) * kTile);
        const uint32_t base = ring_base + (uint32_t)(i % NSLOT) * KvTile<KV, D>::slot_bytes;
        const int page = c0 < sd.nc ? page_id(pages, a, s, c0 >> 8) : 0;
        const KvSpan ksp = kv_span(a, a.k, a.k_nb1, a.k_nb2, a.k_nb3, s, g, c0, sd.nc, rowb, page);
        const KvSpan vsp = kv_span(a, a.v, a.v_nb1, a.v_nb2, a.v_nb3, s, g, c0, sd.nc, rowb, page);
        const buf_rsrc krs = make_rsrc_uniform(ksp.p, ksp.bytes);
        const buf_rsrc vrs = make_rsrc_uniform(vsp.p, vsp.bytes);
        if constexpr (KV == SIXI_TYPE_F16) {
            const uint32_t off = r * knb + c * 16;
            const uint32_t vo = (4 * c) * vnb + r * 16;
            uint32_t ko4[4], vo4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ko4[e] = off + e * 64;
                vo4[e] = vo + e * vnb;
            }
            dma16x4_to_lds<true>(krs, ko4, base);  // (f16 rows: streamed once, non-temporal)
            dma16x4_to_lds<true>(vrs, vo4, base + 4 * 1024);
        } else {
            static_assert(kQ8Dma == 9, "dword LDS-DMA batch of nine loads");
            uint32_t ko[Q8L], vo[Q8L];
#pragma unroll
            for (int u = 0; u < Q8L; ++u) {
                ko[u] = q8_cell[u] * knb + q8_dw[u] * Q8U;
                vo[u] = q8_cell[u] * vnb + q8_dw[u] * Q8U;
            }
            if constexpr (D == 128) {
                dma4x9_to_lds(krs, ko, base);
                dma4x9_to_lds(vrs, vo, base + KvTile<KV, D>::v_off);
            } else {
                dma16x5_to_lds(krs, ko, base);
                dma16x5_to_lds(vrs, vo, base + KvTile<KV, D>::v_off);
            }
        }
    };
    auto step = [&](int i, auto&& after_reads) {
        const u32x4* slot = ring + (i % NSLOT) * SLOT16;
        const int t = t0 + i * TL;
        if (t < t_full)
            tile_step<NTW, KV, MODE, false, D>(a, acc, slot, qs, t * kTile, ri, mrow, sd.nc, lane, after_reads);
        else
            tile_step<NTW, KV, MODE, true, D>(a, acc, slot, qs, t * kTile, ri, mrow, sd.nc, lane, after_reads);
    };

    // private ring: the slot just read is refilled with tile i+NSLOT
    static_assert(NSLOT == 2 || NSLOT == 3, "ring depth");
#pragma unroll
    for (int i = 0; i < NSLOT; ++i)
        if (i < n_my) issue(i);
#pragma unroll 1
    for (int i = 0; i < n_my; ++i) {
        const int ahead = n_my - 1 - i;  // own tiles issued after tile i
        wait_batches<DMA, NSLOT - 1>(ahead);
        step(i, [&] {
            wait_lgkmcnt0();
            if (i + NSLOT < n_my) issue(i + NSLOT);
        });
    }

    // row sums over the lane groups; FAST references to log2 units for merging
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        acc.l[n] = sum4_rowgroups(acc.l[n]);
        if (raw_units<MODE>() && acc.m[n] != neg_inf()) acc.m[n] *= a.scale_log2;
    }

    __syncthreads();  // every wave is past its ring (each drained its own loads)
    auto& mg = reinterpret_cast<MergeBuf<NTW, TL / 2, TD::DT>&>(sh.mg);  // (NTW <= NTOT tiles)
    if (merge_lanes<NTW, TL>(mg, acc, rg, tl, lane)) {
        if (tb == 0 && te == pc.nt_seg)
            write_rows(a, acc, n0, s, g, R, lane);
        else
            write_partial(a.part + pc.slot * a.slot_floats, NTOT * 16, n0, R, acc, lane);
    }
    __syncthreads();  // LDS (q, merge buffers, rings) is reused by the next piece
}

// ---------------------------------------------------------------------------------------
// f16 KV, 49..96 rows per GQA group (128-dim heads), and every row count of 256-dim heads
// (up to 64 rows per launch): 32-cell steps.
//
// Same split as the kernel above.  A work-group holds wide_lanes() piece lanes of RS
// waves each: the waves of a lane are its row groups (NTW row tiles each) and read the same
// staged steps; with two row groups each stages half of every step (row group 0 the K rows,
// row group 1 the V rows), with one it stages both.  The lanes take the piece's steps round
// robin, and the whole group meets at one barrier per step.  The lanes' (m, l, O) are merged
// in LDS at the end of the piece.  One work-group per CU, so each wave has a SIMD and up to
// 512 registers to itself.  For 128-dim heads a three-slot ring per lane keeps two steps in
// flight while one is computed, and a step reads all its K and V^T operands from LDS before
// its first MFMA needs them; 256-dim heads (32 KB steps) use two-slot rings and read the
// operands as the MFMAs go.
// A step covers 32 cells:
//   * O^T += V^T P^T runs on v_mfma_f32_16x16x32_f16 (the 16x16x16 form issues at half
//     that rate on gfx950), and each row maximum and Q^T operand covers twice the cells;
//   * P^T needs no shuffle: the two S^T halves (cells 0-15, 16-31) give lane (r, c) row r
//     at cells 4c+i and 16+4c+i, and the PV reduction index k = 8c + e is taken to mean
//     cell 16(e/4) + 4c + e%4; V^T uses the same order;
//   * V^T comes from LDS with ds_read_b64_tr_b16: the V rows of a step sit in LDS as
//     [cell][dim] with the 32-byte dim chunks XOR-swizzled by cell%8 (bank-conflict-free
//     transposed reads); lane (g, j) of a read addresses cell 16h + 4g + j/4 at dims
//     16db + 4(j%4), so lane (g, i) receives dim 16db + i of cells 16h + 4g .. +3;
//   * Q^T stays in registers for the whole piece.
// O layout: lane (r, c) holds row 16n + r, dims 16t + 4c + i at o[t][n][i].
constexpr int kWide = kDecodeTileWide;  // 32 cells
// Per head dim D: a step's K then V, 32 cell rows of ROW = 2D bytes each (chunk-swizzled);
// KS k-steps of 32 dims, DT output tiles of 16 dims; CPL cells per 1 KB LDS-DMA load.
template <int D>
struct WideDim {
    static constexpr int ROW = 2 * D, KS = D / 32, DT = D / 16, CPL = 1024 / ROW, CPR = ROW / 16;
    static constexpr int HALF = 16 * ROW;     // bytes of 16 cells (one S^T half)
    static constexpr int SLOT = 2 * 32 * ROW;  // K + V of one step
    static constexpr int LOADS = 32 * ROW / 1024;  // LDS-DMA loads per wave per step (K or V)
};
struct WideShape { static constexpr int groups_per_cu = 1; };
// Piece lanes per work-group: two, except 96 rows of 256-dim heads (three row groups of 32
// rows), which run one lane so that each wave keeps a SIMD and 512 registers.
template <int RS, int D> constexpr int wide_lanes() { return (D == 256 && RS == 3) ? 1 : 2; }
// Ring depth per lane (LDS: lanes x slots x SLOT): two steps in flight where it fits.
template <int D, int TL> constexpr int wide_slots() { return (D == 128 || TL == 1) ? 3 : 2; }
// The fast mode of 128-dim heads with two lanes runs the software-pipelined step loop.  It
// reads K of the next step and V of the current one, so K and V have rings of their own
// (8 KB slots; row group 0 stages K, row group 1 V), each as deep as LDS allows: while a
// lane computes, 4 K and 3 V batches can be in flight (56 KB per lane).
constexpr int kPipeK = 5, kPipeV = 4;
template <int MODE, int D, int TL> constexpr bool wide_pipelined() { return MODE == MODE_FAST && D == 128 && TL == 2; }
// Ring bytes of one lane.
template <int D, int TL, bool GEN> constexpr int wide_lane_ring_bytes() {
    return (!GEN && D == 128 && TL == 2) ? (kPipeK + kPipeV) * 32 * WideDim<D>::ROW
                                         : wide_slots<D, TL>() * WideDim<D>::SLOT;
}
struct WideSplit { int ntw, rs; };            // row tiles per wave x waves per lane
constexpr WideSplit kWide64 = {2, 2};         // 64 rows
constexpr WideSplit kWide96 = {3, 2};         // 96 rows

// Explicit masks: the mask rows j < 32 of a step's 32 cells (64 B per row, 2 KB) are staged
// with the step's K and V, in a ring of their own.
constexpr int kMaskTile = 32 * 64;
// RS row groups (waves per lane) of NTW row tiles each; GEN: with the mask ring.
template <int NTW, int RS, int D, bool GEN>
struct alignas(256) WideLds {
    union {
        u32x4 ring[wide_lanes<RS, D>() * wide_lane_ring_bytes<D, wide_lanes<RS, D>(), GEN>() / 16];
        MergeBuf<NTW, (RS * wide_lanes<RS, D>() + 1) / 2, WideDim<D>::DT> mg;  // reused after the step loop
    };
    u32x4 mring[GEN ? wide_lanes<RS, D>() * wide_slots<D, wide_lanes<RS, D>()>() * kMaskTile / 16 : 1];
    StreamTable st;
};

// Q^T B operands of row tiles n0 .. n0+NT-1 in registers: lane (r, c) gets row 16(n0+n) + r
// at dims 32ks + 8c .. +7 as f16 (rows >= R are zero).  All loads are issued before any is
// used -- padding rows read row 0, which every piece has -- so the piece start pays one
// memory latency, not one per operand.  Q8: Q goes through ggml's conversion to the q8_0 dot
// type first (per 32-dim block d = amax/127, q = round-half-away(x * 127/amax) clamped to
// +-127, the MFMA taking f16(q * f16(d))); the block's four lanes (c = 0..3) are lanes r + 16c.
template <int NT, int KS, bool Q8 = false>
__device__ __forceinline__ void load_q_operands(const FaArgs& a, int s, int g, int R, int n0, int lane,
                                                f16x8 (&qv)[NT][KS]) {
    const int r = lane & 15, c = lane >> 4;
    const char* src[NT];
    bool valid[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const int row = 16 * (n0 + n) + r;
        valid[n] = row < R;
        const int rr = valid[n] ? row : 0;
        src[n] = a.q + (int64_t)(rr / a.Gr) * a.q_nb1 + (int64_t)(g * a.G + a.hoff + rr % a.Gr) * a.q_nb2 +
                 (int64_t)s * a.q_nb3 + (int64_t)(8 * c) * a.q_es;
    }
    auto store = [&](int n, int ks, const float (&x)[8]) {
        f16x8 hv;
        if constexpr (Q8) {
            float am = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(x[e]));
            am = fmaxf(am, __shfl_xor(am, 16, 64));
            am = fmaxf(am, __shfl_xor(am, 32, 64));
            const float d = am / 127.0f;
            const float id = d != 0.0f ? 127.0f / am : 0.0f;
            const float dh = (float)(_Float16)d;
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = (_Float16)(fminf(fmaxf(roundf(x[e] * id), -127.0f), 127.0f) * dh);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = (_Float16)x[e];
        }
        qv[n][ks] = valid[n] ? hv : f16x8{};
    };
    if (a.q_f16) {
        u32x4 raw[NT][KS];
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) raw[n][ks] = ld16(src[n] + 64 * ks);
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if constexpr (Q8) {
                    float x[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = (float)as_f16x8(raw[n][ks])[e];
                    store(n, ks, x);
                } else {
                    qv[n][ks] = valid[n] ? as_f16x8(raw[n][ks]) : f16x8{};
                }
            }
    } else {
        f32x4 raw[NT][KS][2];
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                raw[n][ks][0] = *reinterpret_cast<const f32x4*>(src[n] + 128 * ks);
                raw[n][ks][1] = *reinterpret_cast<const f32x4*>(src[n] + 128 * ks + 16);
            }
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                float x[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[e] = raw[n][ks][0][e];
                    x[4 + e] = raw[n][ks][1][e];
                }
                store(n, ks, x);
            }
    }
}

// V^T operand t of a step (vlane ^ 32t: chunk t of the lane's row; the next 16 cells one half
// on).
template <int D>
__device__ __forceinline__ u32x4 wide_vread(uint32_t vlane, int t) {
    const lds_char* vp = lds_ptr(vlane ^ (32u * t));
    const u32x2 lo = ld_tr16(vp);
    const u32x2 hi = ld_tr16(vp + WideDim<D>::HALF);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Softmax state of one step between its score phase and its PV phase.
template <int NT, int D>
struct WideStep {
    float sv[NT][8];              // scores (FAST: raw dot products; GENERIC: log2-domain logits)
    float mx[NT];                 // row maxima of the step
    bool need[NT];                // the row's exponent reference moves
    bool mask_any;                // MASK: some mask value of the step is not 0 (wave-uniform)
    u32x4 vt[WideDim<D>::DT];     // V^T operands, when read ahead with the K operands
};

// Score phase of a step: S^T = K Q^T, the mask, the row maxima and whether a row's lazy
// exponent reference has to move; returns that for any row of the wave (uniform).
template <int NT, int MODE, bool MASKED, int D, bool PF = (D == 128)>
__device__ __forceinline__ bool wide_scores(const FaArgs& a, const Acc<NT, WideDim<D>::DT>& acc, WideStep<NT, D>& ws,
                                            const u32x4* kslot, uint32_t vlane,
                                            const uint32_t (&kofs)[WideDim<D>::KS],
                                            const f16x8 (&qv)[NT][WideDim<D>::KS], int c0, const RowInfo<NT>& ri,
                                            const char* mrow, uint32_t mslot, int nc, int lane) {
    const int c = lane >> 4;

    // ---- S^T halves: lane (r, c) receives cells 16h + 4c + i of row r ----
    using W = WideDim<D>;
    // PF: read all K and V^T operands of the step before the first MFMA, so that their
    // latency hides under the scores and the softmax (128-dim heads in the plain step loop;
    // the pipelined loop hides it under the other step's work instead)
    auto kread = [&](int h, int ks) {
        return as_f16x8(*reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kslot) + kofs[ks] + W::HALF * h));
    };
    f16x8 kop[2][W::KS];
    if constexpr (PF) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int ks = 0; ks < W::KS; ++ks) kop[h][ks] = kread(h, ks);
#pragma unroll
        for (int t = 0; t < W::DT; ++t) ws.vt[t] = wide_vread<D>(vlane, t);
    }
    f32x4 st[2][NT];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < W::KS; ++ks) {
            const f16x8 kk = PF ? kop[h][ks] : kread(h, ks);
#pragma unroll
            for (int n = 0; n < NT; ++n)
                st[h][n] = mfma16x16x32(kk, qv[n][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[h][n]);
        }

    // explicit mask values of the lane's cells 16h + 4c .. +3 for each row tile (staged: from
    // the step's LDS tile, row j at 64 j)
    u32x2 mstage[NT][2];
    if ((MODE == MODE_GENERIC && a.mask && a.mask_stage) || MODE == MODE_MASK) {
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                mstage[n][h] = lds_ld8(mslot + 64u * (uint32_t)ri.j[n] + 2u * (uint32_t)(16 * h + 4 * c));
    }

    // MASK: a step whose mask values are all 0 (+-0) for every row of the wave adds nothing;
    // only the other steps (for a causal mask: those on the diagonal) add them per cell
    ws.mask_any = false;
    if constexpr (MODE == MODE_MASK) {
        uint32_t bits = 0;
#pragma unroll
        for (int n = 0; n < NT; ++n) bits |= mstage[n][0][0] | mstage[n][0][1] | mstage[n][1][0] | mstage[n][1][1];
        ws.mask_any = __builtin_amdgcn_ballot_w64((bits & 0x7fff7fffu) != 0) != 0;
    }
    const float inv_scale = 1.0f / a.scale;

    // ---- scores and row maxima ----
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int cell = c0 + 16 * (e >> 2) + 4 * c + (e & 3);
            float x = st[e >> 2][n][e & 3];
            if (MODE == MODE_MASK) {
                // raw units: s = dot + mask/scale; -inf (or a cell past the stream) skips the
                // cell whatever its K holds
                if (ws.mask_any) {
                    const uint32_t w = mstage[n][e >> 2][(e & 3) >> 1];
                    const float mv = half_bits_to_float((uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu)));
                    x = (mv == neg_inf() || (MASKED && cell >= nc)) ? neg_inf() : fmaf(mv, inv_scale, x);
                } else if (MASKED && cell >= nc) {
                    x = neg_inf();
                }
            } else if (MODE == MODE_GENERIC) {
                x *= a.scale;
                if (a.softcap != 0.0f) x = a.softcap * tanhf(x);
                if (a.mask && a.mask_stage) {
                    const uint32_t w = mstage[n][e >> 2][(e & 3) >> 1];
                    const uint16_t bits = (uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu));
                    const float mv = cell < nc ? ri.slope[n] * half_bits_to_float(bits) : neg_inf();
                    x = (mv == neg_inf()) ? neg_inf() : x + mv;
                } else if (a.mask) {
                    float mv = neg_inf();
                    if (cell < nc) {
                        const uint16_t bits = *reinterpret_cast<const uint16_t*>(
                            mrow + (int64_t)ri.j[n] * a.m_nb1 + (int64_t)cell * 2);
                        mv = ri.slope[n] * half_bits_to_float(bits);
                    }
                    x = (mv == neg_inf()) ? neg_inf() : x + mv;
                } else if (cell >= ri.vis[n]) {
                    x = neg_inf();
                }
                x *= kLog2e;
            } else if (MASKED) {
                if (cell >= ri.vis[n]) x = neg_inf();
            }
            ws.sv[n][e] = x;
        }
        ws.mx[n] = max4_rowgroups(max3f(max3f(ws.sv[n][0], ws.sv[n][1], ws.sv[n][2]),
                                        max3f(ws.sv[n][3], ws.sv[n][4], ws.sv[n][5]), max2f(ws.sv[n][6], ws.sv[n][7])));
    }

    // ---- lazy exponent reference: it moves only when the step's max exceeds it by 2^8 ----
    const float thr = raw_units<MODE>() ? kLazyLog2 / a.scale_log2 : kLazyLog2;
    bool need_any = false;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        ws.need[n] = ws.mx[n] > acc.m[n] + thr;
        need_any |= ws.need[n];
    }
    return __builtin_amdgcn_ballot_w64(need_any) != 0;
}

// Moves the exponent reference of the rows that need it and rescales their l and O.
template <int NT, int MODE, int D>
__device__ __forceinline__ void wide_rescale(const FaArgs& a, Acc<NT, WideDim<D>::DT>& acc, const WideStep<NT, D>& ws) {
    const float c2 = a.scale_log2;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        float alpha = 1.0f;
        if (ws.need[n]) {
            alpha = fast_exp2(raw_units<MODE>() ? (acc.m[n] - ws.mx[n]) * c2 : acc.m[n] - ws.mx[n]);
            acc.m[n] = ws.mx[n];
        }
        acc.l[n] *= alpha;
#pragma unroll
        for (int t0 = 0; t0 < WideDim<D>::DT; t0 += 8) acc_settle8(acc.o, n, t0);
#pragma unroll
        for (int t = 0; t < WideDim<D>::DT; ++t) acc.o[t][n] *= alpha;
    }
}

// PV phase of a step: probabilities against the (settled) exponent reference, their f32 row
// sums, and O^T += V^T P^T.
template <int NT, int MODE, int D, bool PF = (D == 128)>
__device__ __forceinline__ void wide_pv(const FaArgs& a, Acc<NT, WideDim<D>::DT>& acc, const WideStep<NT, D>& ws,
                                        uint32_t vlane, int lane) {
    using W = WideDim<D>;
    const int c = lane >> 4;
    const float c2 = a.scale_log2;
    f16x8 pt[NT];
    const bool use_keep = (MODE == MODE_GENERIC && a.mask) || (MODE == MODE_MASK && ws.mask_any);
    u32x4 keep[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        keep[n] = u32x4{~0u, ~0u, ~0u, ~0u};
        const float ref = acc.m[n];
        const float mc = (ref == neg_inf()) ? 0.0f : (raw_units<MODE>() ? ref * c2 : ref);
        float ps[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            ps[e] = fast_exp2(raw_units<MODE>() ? fmaf(ws.sv[n][e], c2, -mc) : ws.sv[n][e] - mc);
            pt[n][e] = (_Float16)ps[e];
        }
        acc.l[n] += ((ps[0] + ps[1]) + (ps[2] + ps[3])) + ((ps[4] + ps[5]) + (ps[6] + ps[7]));
        if (use_keep) {
            // explicit masks: a cell that none of these 16 rows sees may hold NaN bits, so
            // its V^T column is zeroed for them (0 * NaN must not reach the accumulator)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint64_t b0 = __builtin_amdgcn_ballot_w64((float)pt[n][2 * w] != 0.0f);
                const uint64_t b1 = __builtin_amdgcn_ballot_w64((float)pt[n][2 * w + 1] != 0.0f);
                keep[n][w] = ((((b0 >> (16 * c)) & 0xffffull) != 0) ? 0x0000ffffu : 0u) |
                             ((((b1 >> (16 * c)) & 0xffffull) != 0) ? 0xffff0000u : 0u);
            }
        }
    }

    // ---- O^T += V^T P^T (asm MFMAs, the accumulators pinned in place), eight V^T operands
    // at a time.  Only the operands depend on the mask (all-ones keep masks otherwise): two
    // asm paths joining would make the compiler copy the accumulators right behind the
    // MFMAs, unaware of the asm's results still being in flight. ----
#pragma unroll
    for (int t0 = 0; t0 < W::DT; t0 += 8) {
        u32x4 vv[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) vv[t] = PF ? ws.vt[t0 + t] : wide_vread<D>(vlane, t0 + t);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            if (MODE != MODE_FAST) {
                u32x4 vm[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) vm[t] = vv[t] & keep[n];
                acc_mfma8(acc.o, n, t0, vm, pt[n]);
            } else {
                acc_mfma8(acc.o, n, t0, vv, pt[n]);
            }
        }
    }
}

// ---- Software-pipelined fast step loop (128-dim heads, lengths only) ----
// With one wave per SIMD nothing else hides a wave's VALU work behind its MFMAs.  Iteration
// i of this loop therefore computes the scores of step i+1 and the PV product of step i in
// one scheduling region: the score MFMAs issue between the exponentials of step i, the PV
// MFMAs between the row maxima of step i+1 (MFMAs are builtins here, so that the compiler
// interleaves them and inserts the wait states their results need).
template <int NT>
struct PipeState {
    float sv[NT][8];  // raw scores of the step, masked cells -inf
    float mx[NT];     // their row maxima
};

// S^T of a step: lane (r, c) receives cells 16h + 4c + i of row r.
template <int NT>
__device__ __forceinline__ void pipe_scores(const u32x4* kslot, const uint32_t (&kofs)[4], const f16x8 (&qv)[NT][4],
                                            f32x4 (&st)[2][NT]) {
    using W = WideDim<128>;
    f16x8 kop[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            kop[h][ks] = as_f16x8(*reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kslot) + kofs[ks] +
                                                                  W::HALF * h));
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int n = 0; n < NT; ++n)
                st[h][n] = mfma16x16x32(kop[h][ks], qv[n][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[h][n]);
}

// Row maxima of a step's scores (cells at or past a row's visibility bound -inf when MASKED);
// returns whether one of the lane's rows moves its exponent reference.
template <int NT, bool MASKED>
__device__ __forceinline__ bool pipe_max(const Acc<NT, 8>& acc, const f32x4 (&st)[2][NT], PipeState<NT>& ps, int c0,
                                         const RowInfo<NT>& ri, float thr, int lane) {
    const int c = lane >> 4;
    bool need = false;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float x = st[e >> 2][n][e & 3];
            if (MASKED && c0 + 16 * (e >> 2) + 4 * c + (e & 3) >= ri.vis[n]) x = neg_inf();
            ps.sv[n][e] = x;
        }
        ps.mx[n] = max4_rowgroups(max3f(max3f(ps.sv[n][0], ps.sv[n][1], ps.sv[n][2]),
                                        max3f(ps.sv[n][3], ps.sv[n][4], ps.sv[n][5]), max2f(ps.sv[n][6], ps.sv[n][7])));
        need |= ps.mx[n] > acc.m[n] + thr;
    }
    return need;
}

// Moves the exponent reference of the rows whose step maximum exceeds it by thr, rescaling
// their l and O (rare: only when the running maximum grows by 2^8 in exponent units).
template <int NT>
__device__ __forceinline__ void pipe_rescale(Acc<NT, 8>& acc, const PipeState<NT>& ps, float thr, float c2) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const bool move = ps.mx[n] > acc.m[n] + thr;
        const float alpha = move ? fast_exp2((acc.m[n] - ps.mx[n]) * c2) : 1.0f;
        acc.m[n] = move ? ps.mx[n] : acc.m[n];
        acc.l[n] *= alpha;
#pragma unroll
        for (int t = 0; t < 8; ++t) acc.o[t][n] *= alpha;
    }
}

// Probabilities of a step against the (settled) reference, in f16, and their f32 row sums.
template <int NT>
__device__ __forceinline__ void pipe_probs(Acc<NT, 8>& acc, const PipeState<NT>& ps, float c2, f16x8 (&pt)[NT]) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const float ref = acc.m[n];
        const float mc = (ref == neg_inf()) ? 0.0f : ref * c2;
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            p[e] = fast_exp2(fmaf(ps.sv[n][e], c2, -mc));
            pt[n][e] = (_Float16)p[e];
        }
        acc.l[n] += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
}

// O^T += V^T P^T, row tile by row tile.
template <int NT>
__device__ __forceinline__ void pipe_pv(Acc<NT, 8>& acc, const u32x4 (&vt)[8], const f16x8 (&pt)[NT]) {
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int t = 0; t < 8; ++t) acc.o[t][n] = mfma16x16x32(as_f16x8(vt[t]), pt[n], acc.o[t][n]);
}

// One pipelined iteration: scores of the next step (K at kslot) and the PV product of this one
// (V^T at vlane).  The issue order is fixed by scheduling fences, slot by slot: first the LDS
// reads, then 8*NT slots of one score MFMA and the exponential of one probability of this
// step, then 8*NT slots of one PV MFMA and a piece of the next step's row maxima.  Returns
// whether a row of the lane moves its exponent reference at the next step.
template <int NT, bool MASKED>
__device__ __forceinline__ bool pipe_iteration(Acc<NT, 8>& acc, PipeState<NT>& ps, const u32x4* kslot, uint32_t vlane,
                                               const uint32_t (&kofs)[4], const f16x8 (&qv)[NT][4], int c0n,
                                               const RowInfo<NT>& ri, float thr, float c2, int lane) {
    using W = WideDim<128>;
    const int c = lane >> 4;
    f16x8 kop[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            kop[h][ks] = as_f16x8(*reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kslot) + kofs[ks] +
                                                                  W::HALF * h));
    u32x4 vt[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) vt[t] = wide_vread<128>(vlane, t);
    __builtin_amdgcn_sched_barrier(0);

    f32x4 st[2][NT];
    f16x8 pt[NT];
    float pr[NT][8], mc[NT];
#pragma unroll
    for (int k = 0; k < 8 * NT; ++k) {
        const int ks = k / (2 * NT), h = (k / NT) % 2, n = k % NT;
        st[h][n] = mfma16x16x32(kop[h][ks], qv[n][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[h][n]);
        const int np = k / 8, e = k % 8;
        if (e == 0) mc[np] = (acc.m[np] == neg_inf()) ? 0.0f : acc.m[np] * c2;
        pr[np][e] = fast_exp2(fmaf(ps.sv[np][e], c2, -mc[np]));
        if (e & 1) {
            pt[np][e - 1] = (_Float16)pr[np][e - 1];
            pt[np][e] = (_Float16)pr[np][e];
        }
        if (e == 7)
            acc.l[np] += ((pr[np][0] + pr[np][1]) + (pr[np][2] + pr[np][3])) +
                         ((pr[np][4] + pr[np][5]) + (pr[np][6] + pr[np][7]));
        __builtin_amdgcn_sched_barrier(0);
    }

    bool need = false;
    float m01[NT], m2[NT], mx[NT];
#pragma unroll
    for (int k = 0; k < 8 * NT; ++k) {
        const int n = k / 8, t = k % 8;
        acc.o[t][n] = mfma16x16x32(as_f16x8(vt[t]), pt[n], acc.o[t][n]);
        if (t < 3) {
            // cells e = 3t .. 3t+2 (t = 2: e = 6, 7) of row tile n
#pragma unroll
            for (int e = 3 * t; e < 3 * t + 3 && e < 8; ++e) {
                float x = st[e >> 2][n][e & 3];
                if (MASKED && c0n + 16 * (e >> 2) + 4 * c + (e & 3) >= ri.vis[n]) x = neg_inf();
                ps.sv[n][e] = x;
            }
            if (t == 0) m01[n] = max3f(ps.sv[n][0], ps.sv[n][1], ps.sv[n][2]);
            if (t == 1) m2[n] = max3f(ps.sv[n][3], ps.sv[n][4], ps.sv[n][5]);
            if (t == 2) mx[n] = max3f(m01[n], m2[n], max2f(ps.sv[n][6], ps.sv[n][7]));
        } else if (t == 3) {
            auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx[n]), __float_as_uint(mx[n]), false, false);
            mx[n] = max2f(__uint_as_float(a[0]), __uint_as_float(a[1]));
        } else if (t == 4) {
            auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx[n]), __float_as_uint(mx[n]), false, false);
            ps.mx[n] = max2f(__uint_as_float(b[0]), __uint_as_float(b[1]));
        } else if (t == 5) {
            need |= ps.mx[n] > acc.m[n] + thr;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    return need;
}

// Normalised rows (O layout of the 32-cell kernel).  (With the fused output gate the merge
// kernel gates these rows afterwards.)
template <int NT, int DT>
__device__ __forceinline__ void write_rows_wide(const FaArgs& a, const Acc<NT, DT>& acc, int n0, int s, int g, int R,
                                                int lane) {
    const int r = lane & 15, c = lane >> 4;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const int row = 16 * (n0 + n) + r;
        if (row >= R) continue;
        const int j = row / a.Gr;
        const int h = g * a.G + a.hoff + row % a.Gr;
        const float inv = acc.l[n] == 0.0f ? 0.0f : 1.0f / acc.l[n];
        char* dst = a.out + (int64_t)j * a.o_nb2 + (int64_t)h * a.o_nb1 + (int64_t)s * a.o_nb3 + c * 16;
#pragma unroll
        for (int t = 0; t < DT; ++t) st16(dst + t * 64, acc.o[t][n] * inv);
    }
}

// Partial slot (same format as write_partial) from the 32-cell kernel's O layout.
template <int NT, int DT>
__device__ __forceinline__ void write_partial_wide(float* slot, int rows_slot, int n0, int R, const Acc<NT, DT>& acc,
                                                   int lane) {
    constexpr int D = 16 * DT;
    const int r = lane & 15, c = lane >> 4;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const int row = 16 * (n0 + n) + r;
        if (row >= R) continue;
        const float inv = acc.l[n] == 0.0f ? 0.0f : 1.0f / acc.l[n];
        char* dst = reinterpret_cast<char*>(slot) + (int64_t)row * (2 * D) + c * 8;  // dims 16t + 4c .. +3
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const f16x4 h = {(_Float16)(acc.o[t][n][0] * inv), (_Float16)(acc.o[t][n][1] * inv),
                             (_Float16)(acc.o[t][n][2] * inv), (_Float16)(acc.o[t][n][3] * inv)};
            *reinterpret_cast<u32x2*>(dst + t * 32) = __builtin_bit_cast(u32x2, h);
        }
        if (c == 0) {
            slot[(int64_t)rows_slot * (D / 2) + row] = acc.m[n];
            slot[(int64_t)rows_slot * (D / 2 + 1) + row] = acc.l[n];
        }
    }
}

// One piece of the 32-cell kernel: steps [tb, te) of segment (s, g).
template <int NTW, int RS, int MODE, int D>
__device__ __forceinline__ void decode_piece_wide(const FaArgs& a, WideLds<NTW, RS, D, MODE != MODE_FAST>& sh,
                                                  int causal, const Piece& pc) {
    using W = WideDim<D>;
    constexpr int TL = wide_lanes<RS, D>();
    constexpr int SLOT16 = W::SLOT / 16;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: row group and lane in SGPRs
    const int rg = w / TL;
    const int tl = w % TL;
    const int r = lane & 15;
    const int c = lane >> 4;
    const int s = pc.s, g = pc.g, tb = pc.tb, te = pc.te;
    const StreamDims sd = table_dims(sh.st, s);
    const int G = a.Gr;                 // rows of one block row (heads of this launch)
    const int hb = g * a.G + a.hoff;    // first of those heads
    const int R = G * sd.ql;
    const int n0 = rg * NTW;

    // ---- Q^T operands in registers: row 16(n0+n) + r, dims 32ks + 8c .. +7 ----
    f16x8 qv[NTW][W::KS];
    load_q_operands<NTW, W::KS>(a, s, g, R, n0, lane, qv);

    RowInfo<NTW> ri;
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        const int row = 16 * (n0 + n) + r;
        const bool valid = row < R;
        const int j = valid ? row / G : 0;
        ri.j[n] = j;
        ri.vis[n] = (valid && causal) ? sd.kl + j + 1 : sd.nc;
        ri.slope[n] = (MODE == MODE_GENERIC) ? alibi_slope(a, hb + (valid ? row % G : 0)) : 1.0f;
    }
    // steps below t_full need no per-row visibility test (MASK: no test for the stream's end;
    // its explicit mask is applied on every step)
    const int t_full = (MODE == MODE_GENERIC) ? 0 : ((causal && MODE == MODE_FAST) ? (sd.kl + 1) / kWide : sd.nc / kWide);
    const char* mrow = nullptr;
    if (MODE != MODE_FAST && a.mask) mrow = a.mask + (int64_t)(s % a.m_ne3) * a.m_nb3;

    Acc<NTW, W::DT> acc;
    acc_clear(acc);

    // K/V per step through range-checked resources based at the step's first cell (in its page,
    // for paged caches): cells >= nc read as zeros (and are masked)
    const uint32_t knb = (uint32_t)a.k_nb1, vnb = (uint32_t)a.v_nb1;
    // LDS-DMA source offsets from a step's first cell; every load copies the ROW-byte rows of
    // CPL cells (1 KB, whole cache lines).  K (row group 0), load u: lane t fills LDS row
    // CPL*u + t/CPR at 16-byte position t%CPR, which holds 16-byte chunk (t%CPR) ^ (row % 16)
    // (dims 8 * chunk); the A operand (h, ks) of lane (r, c) -- cell 16h + r, dims
    // 32ks + 8c .. +7 -- then sits at HALF*h + ROW*r + 16((4ks + c) ^ r), and the 16 lanes of
    // a read hit 16 different chunk positions (conflict-free).  V (row group 1), load u: lane
    // t fills LDS row CPL*u + t/CPR at 16-byte position t%CPR, i.e. 32-byte chunk (t%CPR)/2
    // of that row, which holds dims 16 * (chunk ^ (row % 8)).
    uint32_t kofs[W::KS];
#pragma unroll
    for (int ks = 0; ks < W::KS; ++ks) kofs[ks] = (uint32_t)W::ROW * r + 16u * (uint32_t)((4 * ks + c) ^ r);
    // transposed reads of a slot's V rows: lane (c, r) reads cell 4c + r/4 (+16h), dims
    // 16t + 4(r%4) .. +3, found in 32-byte chunk t ^ (cell % 8) of the row.  The row offset
    // has bits 5..8 clear, so chunk t lies at (row + 32*(cell % 8) + 8(r%4)) ^ 32t.
    const uint32_t vrow = (uint32_t)(4 * c + (r >> 2)) * (uint32_t)W::ROW + 32u * (4 * (c & 1) + (r >> 2)) + 8u * (r & 3);

    // steps of this lane: tb + tl + TL*i, i < n_my; n_iter is the same for the whole group
    const int t0 = tb + tl;
    const int n_my = t0 < te ? (te - t0 + TL - 1) / TL : 0;
    const int n_iter = (te - tb + TL - 1) / TL;
    constexpr bool GEN = MODE != MODE_FAST;
    constexpr bool PIPE = wide_pipelined<MODE, D, TL>();
    constexpr int NS = wide_slots<D, TL>();  // slots of the plain ring
    u32x4* ring = sh.ring + (size_t)tl * (wide_lane_ring_bytes<D, TL, GEN>() / 16);
    const uint32_t ring_base = lds_addr(ring);

    // explicit masks: rows j < 32 of a stream's mask; an empty resource (every load returns 0)
    // when the mask is read from global memory instead, so that every issue has the same loads
    const buf_rsrc mrs = make_rsrc_uniform(mrow, GEN && a.mask_stage ? a.m_bytes : 0u);
    const uint32_t mring_base = lds_addr(sh.mring) + (uint32_t)tl * NS * kMaskTile;
    PageIds pages = page_ids_load(a, s, (t0 * kWide) >> 8);
    auto issue = [&](int i, int slot) {
        // uniform over the wave (the compiler cannot tell): scalar page and span arithmetic
        const uint32_t c0 = (uint32_t)(t0 + i * TL) * kWide;
        const uint32_t base = ring_base + (uint32_t)slot * W::SLOT;
        const int page = (int)c0 < sd.nc ? page_id(pages, a, s, (int)(c0 >> 8)) : 0;
        const KvSpan ksp = kv_span(a, a.k, a.k_nb1, a.k_nb2, a.k_nb3, s, g, (int)c0, sd.nc, W::ROW, page);
        const KvSpan vsp = kv_span(a, a.v, a.v_nb1, a.v_nb2, a.v_nb3, s, g, (int)c0, sd.nc, W::ROW, page);
        const buf_rsrc krs = make_rsrc_uniform(ksp.p, ksp.bytes);
        const buf_rsrc vrs = make_rsrc_uniform(vsp.p, vsp.bytes);
        const uint32_t pos = (uint32_t)lane % W::CPR;  // 16-byte position in the row
        if constexpr (GEN) {
            // mask rows 16*half + lane/4, cells c0 + 8*(lane%4) .. +7: 1 KB per load, laid out
            // [row][32 cells] (64 B per row) in the slot's tile
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                if (RS == 1 || rg == half) {
                    const uint32_t j = 16u * half + (uint32_t)lane / 4;
                    dma16x1_to_lds(mrs, j * (uint32_t)a.m_nb1 + (c0 + 8u * (lane & 3)) * 2u,
                                   mring_base + (uint32_t)slot * kMaskTile + 1024u * half);
                }
            }
        }
#pragma unroll
        for (int b8 = 0; b8 < W::LOADS / 8; ++b8) {
            uint32_t o8[8];
            if (rg == 0) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t cell = W::CPL * (8 * b8 + u) + (uint32_t)lane / W::CPR;
                    o8[u] = cell * knb + 16u * (pos ^ (cell & 15u));
                }
                dma16x8_to_lds<true>(krs, o8, base + 8192u * b8);
            }
            if (rg == (RS == 1 ? 0 : 1)) {  // one row group stages both halves
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t cell = W::CPL * (8 * b8 + u) + (uint32_t)lane / W::CPR;
                    o8[u] = cell * vnb + 32u * ((pos >> 1) ^ (cell & 7u)) + 16u * (pos & 1u);
                }
                dma16x8_to_lds<true>(vrs, o8, base + 32 * W::ROW + 8192u * b8);
            }
        }
    };
    // loads one issue puts in flight for each wave (the wave of a single row group stages K and
    // V, and both halves of an explicit mask's tile)
    constexpr int LPW = (RS == 1 ? 2 : 1) * (W::LOADS + (GEN ? 1 : 0));
    // V^T read address of slot sl for this lane (the V area is 256-byte aligned, so ^ 32t
    // only moves bits 5..7 of vrow)
    auto vlane_at = [&](int slot) { return ring_base + (uint32_t)slot * W::SLOT + 32 * W::ROW + vrow; };
    // Steps that every lane has and that lie below t_full for every lane run the unmasked
    // score phase, the rest the masked one.  (One loop choosing the body per step makes the
    // compiler merge two accumulator sets every step: register copies and spills.)
    const int n_plain = min(max((t_full - tb) / TL, 0), (te - tb) / TL);
    {
        // Step i reads slot i % NS.  After the barrier of step i every wave has left step i-1,
        // so step i+NS-1 goes into that step's slot while steps i+1 .. i+NS-2 are still in
        // flight.  Each issue is one batch of LPW loads per wave, and the ring loads are the
        // only loads a wave has in flight in the step loop, so vmcnt counts the batches issued
        // after step i.
        // (the pipelined loop's ring and its pre-loop loads are set up below)
        constexpr int KB = 32 * W::ROW;  // bytes of one step's K (or V) rows
        const uint32_t vring_base = ring_base + kPipeK * KB;
        auto issue_k = [&](int j) {  // row group 0: K of step j into K slot j % kPipeK
            const uint32_t c0 = (uint32_t)(t0 + j * TL) * kWide;
            const int page = (int)c0 < sd.nc ? page_id(pages, a, s, (int)(c0 >> 8)) : 0;
            const KvSpan ksp = kv_span(a, a.k, a.k_nb1, a.k_nb2, a.k_nb3, s, g, (int)c0, sd.nc, W::ROW, page);
            const buf_rsrc krs = make_rsrc_uniform(ksp.p, ksp.bytes);
            const uint32_t pos = (uint32_t)lane % W::CPR;
            uint32_t o8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t cell = W::CPL * u + (uint32_t)lane / W::CPR;
                o8[u] = cell * knb + 16u * (pos ^ (cell & 15u));
            }
            dma16x8_to_lds<true>(krs, o8, ring_base + (uint32_t)(j % kPipeK) * KB);
        };
        auto issue_v = [&](int j) {  // row group 1: V of step j into V slot j % kPipeV
            const uint32_t c0 = (uint32_t)(t0 + j * TL) * kWide;
            const int page = (int)c0 < sd.nc ? page_id(pages, a, s, (int)(c0 >> 8)) : 0;
            const KvSpan vsp = kv_span(a, a.v, a.v_nb1, a.v_nb2, a.v_nb3, s, g, (int)c0, sd.nc, W::ROW, page);
            const buf_rsrc vrs = make_rsrc_uniform(vsp.p, vsp.bytes);
            const uint32_t pos = (uint32_t)lane % W::CPR;
            uint32_t o8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t cell = W::CPL * u + (uint32_t)lane / W::CPR;
                o8[u] = cell * vnb + 32u * ((pos >> 1) ^ (cell & 7u)) + 16u * (pos & 1u);
            }
            dma16x8_to_lds<true>(vrs, o8, vring_base + (uint32_t)(j % kPipeV) * KB);
        };
        if constexpr (PIPE) {
            static_assert(RS == 2 && W::LOADS == 8, "the pipelined ring: one K and one V loader wave per lane");
            if (rg == 0) {
#pragma unroll
                for (int q = 0; q < kPipeK; ++q)
                    if (q < n_my) issue_k(q);
            } else {
#pragma unroll
                for (int q = 0; q < kPipeV - 1; ++q)
                    if (q < n_my) issue_v(q);
            }
        } else {
#pragma unroll
            for (int q = 0; q < NS - 1; ++q)
                if (q < n_my) issue(q, q);
        }
        // The Q^T operands' loads end here, once per piece: left for the loop, the compiler's
        // wait for them lands in the step body (before an LDS read that reuses a register),
        // where it would drain the ring's DMA loads every step.
#pragma unroll
        for (int n = 0; n < NTW; ++n)
#pragma unroll
            for (int ks = 0; ks < W::KS; ++ks) asm volatile("" ::"v"(qv[n][ks]));
        if constexpr (PIPE) {
            // Iteration i reads K of step i+1 and V of step i.  Row group 0 keeps K of steps
            // up to i+kPipeK-1 issued and waits for K of step i+1 before the iteration's barrier,
            // then issues step i+kPipeK into the slot of step i (read in iteration i-1); row
            // group 1 keeps V up to step i+kPipeV-2 issued, waits for V of step i, then issues
            // step i+kPipeV-1 into the slot of step i-1.  Each wave counts only its own loads.
            auto wait_later = [&](int later) { wait_batches<LPW, kPipeK - 1>(later); };  // own batches in flight
            auto wait_k = [&](int j) { wait_later(max(min(j + kPipeK - 2, n_my - 1) - j, 0)); };  // K of step j
            auto wait_v = [&](int j) { wait_later(max(min(j + kPipeV - 2, n_my - 1) - j, 0)); };  // V of step j
            auto kslot = [&](int j) { return ring + (size_t)(j % kPipeK) * (KB / 16); };
            auto vlane = [&](int j) { return vring_base + (uint32_t)(j % kPipeV) * KB + vrow; };
            const float c2 = a.scale_log2;
            const float thr = kLazyLog2 / a.scale_log2;
            PipeState<NTW> ps;
            bool need = false;
            if (n_iter > 0) {
                if (rg == 0 && n_my > 0) wait_later(max(min(kPipeK - 1, n_my - 1), 0));
                __syncthreads();
                if (n_my > 0) {
                    f32x4 st[2][NTW];
                    pipe_scores(kslot(0), kofs, qv, st);
                    need = n_plain > 0 ? pipe_max<NTW, false>(acc, st, ps, t0 * kWide, ri, thr, lane)
                                       : pipe_max<NTW, true>(acc, st, ps, t0 * kWide, ri, thr, lane);
                }
            }
            auto head = [&](int i) {
                if (rg == 0) {
                    if (i + 1 < n_my) wait_k(i + 1);
                } else if (i < n_my) {
                    wait_v(i);
                }
                __syncthreads();
                if (rg == 0) {
                    if (i + kPipeK < n_my) issue_k(i + kPipeK);
                } else if (i + kPipeV - 1 < n_my) {
                    issue_v(i + kPipeV - 1);
                }
                if (i < n_my && __builtin_amdgcn_ballot_w64(need) != 0) pipe_rescale(acc, ps, thr, c2);
            };
            auto body = [&](int i, auto masked) {
                need = pipe_iteration<NTW, decltype(masked)::value>(acc, ps, kslot(i + 1), vlane(i), kofs, qv,
                                                                     (t0 + (i + 1) * TL) * kWide, ri, thr, c2, lane);
            };
            auto last = [&](int i) {  // PV of a step without a next one
                u32x4 vt[8];
                f16x8 pt[NTW];
#pragma unroll
                for (int t = 0; t < 8; ++t) vt[t] = wide_vread<128>(vlane(i), t);
                pipe_probs(acc, ps, c2, pt);
                pipe_pv(acc, vt, pt);
            };
            int i = 0;
            // next step unmasked (every lane has it)
#pragma unroll 1
            for (; i < n_plain - 1; ++i) {
                head(i);
                body(i, std::false_type{});
            }
#pragma unroll 1
            for (; i < n_iter - 1; ++i) {
                head(i);
                if (i + 1 < n_my) body(i, std::true_type{});
                else if (i < n_my) last(i);
            }
            if (n_iter > 0) {
                // V of the last step (nothing is issued any more)
                const int il = n_iter - 1;
                if (rg == 1 && il < n_my) wait_v(il);
                __syncthreads();
                if (il < n_my) {
                    if (__builtin_amdgcn_ballot_w64(need) != 0) pipe_rescale(acc, ps, thr, c2);
                    last(il);
                }
            }
        } else {
        // Score phase of step i after its data has landed; returns whether a row's exponent
        // reference moves (uniform over the wave).  Every wave passes the barrier of every step.
        auto scores = [&](int i, auto masked, WideStep<NTW, D>& ws) -> bool {
            wait_batches<LPW, NS - 2>(n_my - 1 - i);  // own batches of the steps issued after step i
            __syncthreads();
            if (i + NS - 1 < n_my) issue(i + NS - 1, (i + NS - 1) % NS);
            if (!decltype(masked)::value || i < n_my) {
                const int t = t0 + i * TL;
                const u32x4* kslot = ring + (i % NS) * SLOT16;
                return wide_scores<NTW, MODE, decltype(masked)::value, D>(
                    a, acc, ws, kslot, vlane_at((i) % NS), kofs, qv, t * kWide, ri, mrow,
                    mring_base + (uint32_t)(i % NS) * kMaskTile, sd.nc, lane);
            }
            return false;
        };
        auto finish = [&](int i, auto masked, const WideStep<NTW, D>& ws) {
            if (!decltype(masked)::value || i < n_my) wide_pv<NTW, MODE, D>(a, acc, ws, vlane_at((i) % NS), lane);
        };
        int i = 0;
        auto run = [&](int end, auto masked) {
#pragma unroll 1
            for (; i < end; ++i) {
                WideStep<NTW, D> ws;
                if (scores(i, masked, ws)) wide_rescale<NTW, MODE, D>(a, acc, ws);
                finish(i, masked, ws);
            }
        };
        run(n_plain, std::false_type{});
        run(n_iter, std::true_type{});
        }
    }
    acc_settle(acc.o);  // the asm MFMAs' results before the merge reads them

#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        acc.l[n] = sum4_rowgroups(acc.l[n]);
        if (raw_units<MODE>() && acc.m[n] != neg_inf()) acc.m[n] *= a.scale_log2;
    }

    __syncthreads();  // every wave is past its ring (each drained its own loads)
    if (merge_lanes<NTW, TL>(sh.mg, acc, rg, tl, lane)) {
        if (tb == 0 && te == pc.nt_seg)
            write_rows_wide(a, acc, n0, s, g, R, lane);
        else
            write_partial_wide(a.part + pc.slot * a.slot_floats, NTW * RS * 16, n0, R, acc, lane);
    }
    __syncthreads();  // LDS (merge buffers, rings) is reused by the next piece
}

// ---------------------------------------------------------------------------------------
// q8_0 KV, 49..96 rows per GQA group (128-dim heads): the 32-cell kernel over q8_0 steps.
//
// A step's q8_0 rows (32 cells x 136 B of K, the same of V) come in by dword LDS-DMA into a
// ring of q8_0 slots.  During step i the lane's waves convert step i+1 into f16 rows laid out
// exactly as the f16 kernel stages them (K 16-byte chunks swizzled by cell % 16, V 32-byte
// chunks by cell % 8), in one of two f16 buffers, so the score and PV code of the f16 kernel
// runs unchanged on them.  The conversion is f16(q * d), one rounding -- the operands the
// q8_0 16-cell kernel and the f16 staging path use -- and Q goes through ggml's conversion to
// the q8_0 dot type.  With two row groups, row group 0 stages and converts K, row group 1 V;
// one row group does both.  K and V are read once for all 96 rows (the 16-cell q8_0 kernel
// holds 48 rows, so such a block would take two launches, each reading the KV).
// Per head dim: ROW bytes of a q8_0 head row; a step's rows come in as LOADS LDS-DMA loads of
// LB bytes per lane (128-dim rows are only 4-byte aligned: dword loads, 17 x 256 B = 4352 B
// exactly; 256-dim rows are 16-byte aligned: 9 x 1 KB, the last half past the step's 8704 B);
// TL lanes per work-group (256 dims: one, for LDS).
template <int D> struct Q8Dim;
template <> struct Q8Dim<128> { static constexpr int ROW = 136, LB = 4, LOADS = 17, TL = 2; };
template <> struct Q8Dim<256> { static constexpr int ROW = 272, LB = 16, LOADS = 9, TL = 1; };
template <int D> constexpr int q8_step_lds() { return Q8Dim<D>::LOADS * 64 * Q8Dim<D>::LB; }  // K (or V) of a step
template <int D> constexpr int q8_slot_bytes() { return 2 * q8_step_lds<D>(); }              // K + V
static_assert(q8_step_lds<128>() == 32 * 136 && q8_step_lds<256>() >= 32 * 272, "a step's rows fit its loads");
template <int RS> constexpr int q8_slots() { return RS == 1 ? 3 : 4; }  // vmcnt holds 2 x 2 x 18 at most
template <int NTW, int RS, bool GEN, int D>
struct alignas(256) WideQ8Lds {
    static constexpr int TL = Q8Dim<D>::TL;
    union {
        struct {
            u32x4 f16buf[TL * 2 * WideDim<D>::SLOT / 16];   // two converted steps per lane
            u32x4 q8ring[TL * q8_slots<RS>() * q8_slot_bytes<D>() / 16];
        } t;
        MergeBuf<NTW, (RS * TL + 1) / 2, WideDim<D>::DT> mg;
    };
    u32x4 mring[GEN ? TL * q8_slots<RS>() * kMaskTile / 16 : 1];
    StreamTable st;
};

// Converts the q8_0 rows of one step (K or V, 32 cells) to f16 at `dst` in the f16 kernel's
// LDS layout: lane (h, x) = (lane / 32, lane % 32) takes block b = (D/64)h + m of cell x in
// pass m < D/64.  Block b starts 34b bytes into the row (whose length is a multiple of 4), so
// all lanes of a pass have the scale in the same half of a dword (no divergent unpacking);
// at 128 dims the 64 lanes' dword reads (row stride 34 dwords, h offset 17) hit 64 banks.
template <bool IS_V, int M, int D>
__device__ __forceinline__ void q8_block_to_f16(const uint32_t* src, char* dst, int x, int h) {
    const int b = (D / 64) * h + M;
    uint16_t d;
    uint32_t w[8];
    ld_q8_block<(M & 1) == 1>(src, x * Q8Dim<D>::ROW + 34 * b, d, w);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const u32x4 f = dequant_q8x8(w[2 * k], w[2 * k + 1], d);
        const int j = 4 * b + k;  // 16-byte chunk: dims 8j .. 8j+7
        const int pos = IS_V ? 32 * ((j >> 1) ^ (x & 7)) + 16 * (j & 1) : 16 * (j ^ (x & 15));
        *reinterpret_cast<u32x4*>(dst + x * WideDim<D>::ROW + pos) = f;
    }
}

template <bool IS_V, int D>
__device__ __forceinline__ void q8_step_to_f16(const uint32_t* src, char* dst, int lane) {
    q8_block_to_f16<IS_V, 0, D>(src, dst, lane & 31, lane >> 5);
    q8_block_to_f16<IS_V, 1, D>(src, dst, lane & 31, lane >> 5);
    if constexpr (D == 256) {
        q8_block_to_f16<IS_V, 2, D>(src, dst, lane & 31, lane >> 5);
        q8_block_to_f16<IS_V, 3, D>(src, dst, lane & 31, lane >> 5);
    }
}

template <int NTW, int RS, int MODE, int D>
__device__ __forceinline__ void decode_piece_wide_q8(const FaArgs& a, WideQ8Lds<NTW, RS, MODE != MODE_FAST, D>& sh,
                                                     int causal, const Piece& pc) {
    using W = WideDim<D>;
    using Q = Q8Dim<D>;
    constexpr int TL = Q::TL;
    constexpr int STEP = q8_step_lds<D>(), SLOTB = q8_slot_bytes<D>();
    constexpr int NSQ = q8_slots<RS>();
    constexpr bool GEN = MODE != MODE_FAST;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = w / TL;
    const int tl = w % TL;
    const int s = pc.s, g = pc.g, tb = pc.tb, te = pc.te;
    const StreamDims sd = table_dims(sh.st, s);
    const int G = a.Gr;
    const int hb = g * a.G + a.hoff;
    const int R = G * sd.ql;
    const int n0 = rg * NTW;
    const int r = lane & 15;
    const int c = lane >> 4;

    f16x8 qv[NTW][W::KS];
    load_q_operands<NTW, W::KS, true>(a, s, g, R, n0, lane, qv);

    RowInfo<NTW> ri;
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        const int row = 16 * (n0 + n) + r;
        const bool valid = row < R;
        const int j = valid ? row / G : 0;
        ri.j[n] = j;
        ri.vis[n] = (valid && causal) ? sd.kl + j + 1 : sd.nc;
        ri.slope[n] = (MODE == MODE_GENERIC) ? alibi_slope(a, hb + (valid ? row % G : 0)) : 1.0f;
    }
    const int t_full = (MODE == MODE_GENERIC) ? 0 : ((causal && MODE == MODE_FAST) ? (sd.kl + 1) / kWide : sd.nc / kWide);
    const char* mrow = nullptr;
    if (MODE != MODE_FAST && a.mask) mrow = a.mask + (int64_t)(s % a.m_ne3) * a.m_nb3;

    Acc<NTW, W::DT> acc;
    acc_clear(acc);

    const uint32_t knb = (uint32_t)a.k_nb1, vnb = (uint32_t)a.v_nb1;
    // K/V of the piece's steps: read offsets of the LB-byte piece t = 64u + lane of a step's
    // rows -- row t / (ROW/LB), piece t % (ROW/LB) -- relative to the step's first cell; row
    // group 0 loads K, row group 1 V (one row group: both)
    constexpr uint32_t PER = Q::ROW / Q::LB;
    uint32_t ko[Q::LOADS], vo[Q::LOADS];
#pragma unroll
    for (int u = 0; u < Q::LOADS; ++u) {
        const uint32_t t = 64u * u + (uint32_t)lane;
        ko[u] = (t / PER) * knb + (t % PER) * (uint32_t)Q::LB;
        vo[u] = (t / PER) * vnb + (t % PER) * (uint32_t)Q::LB;
    }
    uint32_t kofs[W::KS];
#pragma unroll
    for (int ks = 0; ks < W::KS; ++ks) kofs[ks] = (uint32_t)W::ROW * r + 16u * (uint32_t)((4 * ks + c) ^ r);
    const uint32_t vrow = (uint32_t)(4 * c + (r >> 2)) * (uint32_t)W::ROW + 32u * (4 * (c & 1) + (r >> 2)) + 8u * (r & 3);

    const int t0 = tb + tl;
    const int n_my = t0 < te ? (te - t0 + TL - 1) / TL : 0;
    const int n_iter = (te - tb + TL - 1) / TL;
    u32x4* f16buf = sh.t.f16buf + (size_t)tl * 2 * (W::SLOT / 16);
    const uint32_t* q8ring = reinterpret_cast<const uint32_t*>(sh.t.q8ring + (size_t)tl * NSQ * (SLOTB / 16));
    const uint32_t q8_base = lds_addr(sh.t.q8ring) + (uint32_t)tl * NSQ * SLOTB;

    const buf_rsrc mrs = make_rsrc_uniform(mrow, GEN && a.mask_stage ? a.m_bytes : 0u);
    const uint32_t mring_base = lds_addr(sh.mring) + (uint32_t)tl * NSQ * kMaskTile;
    PageIds pages = page_ids_load(a, s, (t0 * kWide) >> 8);
    auto issue = [&](int i) {
        const int slot = i % NSQ;
        const uint32_t c0 = (uint32_t)(t0 + i * TL) * kWide;
        const uint32_t base = q8_base + (uint32_t)slot * SLOTB;
        const int page = (int)c0 < sd.nc ? page_id(pages, a, s, (int)(c0 >> 8)) : 0;
        if constexpr (GEN) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                if (RS == 1 || rg == half) {
                    const uint32_t j = 16u * half + (uint32_t)lane / 4;
                    dma16x1_to_lds(mrs, j * (uint32_t)a.m_nb1 + (c0 + 8u * (lane & 3)) * 2u,
                                   mring_base + (uint32_t)slot * kMaskTile + 1024u * half);
                }
            }
        }
        auto rows = [&](const buf_rsrc& rs, const uint32_t (&o)[Q::LOADS], uint32_t dst) {
            uint32_t o8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) o8[u] = o[u];
            if constexpr (Q::LB == 4) {
                uint32_t o9[9];
#pragma unroll
                for (int u = 0; u < 9; ++u) o9[u] = o[8 + u];
                dma4x8_to_lds(rs, o8, dst);
                dma4x9_to_lds(rs, o9, dst + 8 * 256);
            } else {
                dma16x8_to_lds(rs, o8, dst);
                dma16x1_to_lds(rs, o[8], dst + 8 * 1024);
            }
        };
        if (rg == 0) {
            const KvSpan sp = kv_span(a, a.k, a.k_nb1, a.k_nb2, a.k_nb3, s, g, (int)c0, sd.nc, Q::ROW, page);
            rows(make_rsrc_uniform(sp.p, sp.bytes), ko, base);
        }
        if (rg == (RS == 1 ? 0 : 1)) {
            const KvSpan sp = kv_span(a, a.v, a.v_nb1, a.v_nb2, a.v_nb3, s, g, (int)c0, sd.nc, Q::ROW, page);
            rows(make_rsrc_uniform(sp.p, sp.bytes), vo, base + STEP);
        }
    };
    // step i's q8_0 rows -> f16 buffer i % 2
    auto convert = [&](int i) {
        const uint32_t* src = q8ring + (size_t)(i % NSQ) * (SLOTB / 4);
        char* dst = reinterpret_cast<char*>(f16buf + (size_t)(i & 1) * (W::SLOT / 16));
        if constexpr (RS == 3 && D == 256) {
            // three row groups: the eight passes (K blocks 4h + m, m < 4, then V's) go round robin
            // over them (3, 3 and 2 passes) instead of four each to row groups 0 and 1 -- the step
            // waits for the slowest wave.  Every wave's loads of the step landed before the barrier
            // that precedes this conversion, so any wave may convert K or V.
            const int x = lane & 31, h = lane >> 5;
            const uint32_t* sv = src + STEP / 4;
            char* dv = dst + 32 * W::ROW;
            if (rg == 0) {
                q8_block_to_f16<false, 0, D>(src, dst, x, h);
                q8_block_to_f16<false, 3, D>(src, dst, x, h);
                q8_block_to_f16<true, 2, D>(sv, dv, x, h);
            } else if (rg == 1) {
                q8_block_to_f16<false, 1, D>(src, dst, x, h);
                q8_block_to_f16<true, 0, D>(sv, dv, x, h);
                q8_block_to_f16<true, 3, D>(sv, dv, x, h);
            } else {
                q8_block_to_f16<false, 2, D>(src, dst, x, h);
                q8_block_to_f16<true, 1, D>(sv, dv, x, h);
            }
        } else {
            if (rg == 0) q8_step_to_f16<false, D>(src, dst, lane);
            if (rg == (RS == 1 ? 0 : 1)) q8_step_to_f16<true, D>(src + STEP / 4, dst + 32 * W::ROW, lane);
        }
    };
    constexpr int LPW = (RS == 1 ? 2 : 1) * (Q::LOADS + (GEN ? 1 : 0));
    const int n_plain = min(max((t_full - tb) / TL, 0), (te - tb) / TL);
    {
        // Issue order: steps 0 .. NSQ-2 up front, then step i+NSQ-1 after the barrier of step i
        // (into the slot of step i-1, converted during step i-2).  Before the barrier of step i
        // each wave waits for step i+1's loads, which the conversion during step i reads; the
        // batches issued after it may stay in flight.
        // own loads of step j landed, with steps 0 .. issued-1 issued so far
        auto wait_for = [&](int j, int issued) {
            wait_batches<LPW, NSQ - 2>(min(issued, n_my) - (j + 1));
        };
#pragma unroll
        for (int q = 0; q < NSQ - 1; ++q)
            if (q < n_my) issue(q);
#pragma unroll
        for (int n = 0; n < NTW; ++n)
#pragma unroll
            for (int ks = 0; ks < W::KS; ++ks) asm volatile("" ::"v"(qv[n][ks]));
        if (n_my > 0) wait_for(0, NSQ - 1);
        __syncthreads();
        if (n_my > 0) convert(0);
        auto scores = [&](int i, auto masked, WideStep<NTW, D>& ws) -> bool {
            if (i + 1 < n_my) wait_for(i + 1, i + NSQ - 1);
            __syncthreads();
            if (i + NSQ - 1 < n_my) issue(i + NSQ - 1);
            if (i + 1 < n_my) convert(i + 1);
            if (!decltype(masked)::value || i < n_my) {
                const int t = t0 + i * TL;
                const u32x4* kslot = f16buf + (size_t)(i & 1) * (W::SLOT / 16);
                const uint32_t vlane = lds_addr(kslot) + 32 * W::ROW + vrow;
                return wide_scores<NTW, MODE, decltype(masked)::value, D>(
                    a, acc, ws, kslot, vlane, kofs, qv, t * kWide, ri, mrow,
                    mring_base + (uint32_t)(i % NSQ) * kMaskTile, sd.nc, lane);
            }
            return false;
        };
        auto finish = [&](int i, auto masked, const WideStep<NTW, D>& ws) {
            if (!decltype(masked)::value || i < n_my)
                wide_pv<NTW, MODE, D>(a, acc, ws, lds_addr(f16buf + (size_t)(i & 1) * (W::SLOT / 16)) + 32 * W::ROW + vrow,
                                        lane);
        };
        int i = 0;
        auto run = [&](int end, auto masked) {
#pragma unroll 1
            for (; i < end; ++i) {
                WideStep<NTW, D> ws;
                if (scores(i, masked, ws)) wide_rescale<NTW, MODE, D>(a, acc, ws);
                finish(i, masked, ws);
            }
        };
        run(n_plain, std::false_type{});
        run(n_iter, std::true_type{});
    }
    acc_settle(acc.o);

#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        acc.l[n] = sum4_rowgroups(acc.l[n]);
        if (raw_units<MODE>() && acc.m[n] != neg_inf()) acc.m[n] *= a.scale_log2;
    }

    __syncthreads();
    if (merge_lanes<NTW, TL>(sh.mg, acc, rg, tl, lane)) {
        if (tb == 0 && te == pc.nt_seg)
            write_rows_wide(a, acc, n0, s, g, R, lane);
        else
            write_partial_wide(a.part + pc.slot * a.slot_floats, NTW * RS * 16, n0, R, acc, lane);
    }
    __syncthreads();
}

// Work-group -> range of the cost line (segments laid end to end, each seg_cost units of
// start-up followed by its tiles).  Returns false for a work-group without a range.
struct Partition {
    int64_t T, P, x0, x1;
    int p_log;
};

// HS: the kernel may run a head-aligned split (a.head_split); kernels launched without one
// leave the branch out (it costs registers in the tile loop of the 16-cell kernel).
template <bool HS>
__device__ __forceinline__ bool partition(const FaArgs& a, const int* ps, int b, Partition& pt) {
    // logical index: with the remap, consecutive tile ranges land on one XCD (work-groups
    // are dealt round-robin over the XCDs)
    pt.p_log = a.xcd_remap ? (b % kXcds) * (a.P / kXcds) + b / kXcds : b;
    if (HS && a.head_split) {
        // ranges over the streams' cost line, each taken by the Hkv work-groups Hkv*q .. +Hkv-1
        pt.T = ps[a.S];
        const int64_t Q = a.P / a.Hkv;
        pt.P = pt.T < Q ? pt.T : Q;
        const int64_t q = pt.p_log / a.Hkv;
        if (q >= pt.P) return false;
        pt.x0 = q * pt.T / pt.P;
        pt.x1 = (q + 1) * pt.T / pt.P;
        return true;
    }
    pt.T = (int64_t)a.Hkv * ps[a.S];
    pt.P = pt.T < a.P ? pt.T : a.P;  // active work-groups: every one owns >= 1 unit
    if (pt.p_log >= pt.P) return false;
    pt.x0 = pt.p_log * pt.T / pt.P;
    pt.x1 = (pt.p_log + 1) * pt.T / pt.P;
    return true;
}

// Runs fn(piece) for every piece of this work-group's tile range, in order.
template <bool HS, typename F>
__device__ __forceinline__ void for_each_piece(const FaArgs& a, const int* ps, F&& fn) {
    Partition pt;
    if (!partition<HS>(a, ps, blockIdx.x, pt)) return;
    const int64_t Hkv = a.Hkv;
    if (HS && a.head_split) {
        // this work-group's kv-head over the cells of its range of every stream it touches;
        // piece q of segment k sits in slot k + q * Hkv
        const int g = (int)(pt.p_log % Hkv);
        const int64_t q = pt.p_log / Hkv;
        int lo = 0, hi = a.S;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (ps[mid] <= pt.x0) lo = mid; else hi = mid - 1;
        }
        for (int s = lo; s < a.S && ps[s] < pt.x1; ++s) {
            const int ct = ps[s + 1] - ps[s];
            const int64_t t0 = (int64_t)ps[s] + a.seg_cost;
            const int64_t xb = pt.x0 > t0 ? pt.x0 : t0;
            const int64_t xe = pt.x1 < ps[s + 1] ? pt.x1 : ps[s + 1];
            if (xb >= xe) continue;
            Piece pc;
            pc.s = __builtin_amdgcn_readfirstlane(s);
            pc.g = __builtin_amdgcn_readfirstlane(g);
            pc.tb = __builtin_amdgcn_readfirstlane((int)(xb - t0));
            pc.te = __builtin_amdgcn_readfirstlane((int)(xe - t0));
            pc.nt_seg = __builtin_amdgcn_readfirstlane(ct - a.seg_cost);
            pc.slot = __builtin_amdgcn_readfirstlane((int)(((int64_t)s + q) * Hkv + g));
            if (threadIdx.x == 0) {
                const int64_t seg = (int64_t)s * Hkv + g;
                if (pc.tb == 0) a.seg_pieces[2 * seg] = (int)q;
                if (pc.te == pc.nt_seg) a.seg_pieces[2 * seg + 1] = (int)q;
            }
            fn(pc);
        }
        return;
    }

    // stream holding unit x0: the largest s with Hkv*ps[s] <= x0
    int lo = 0, hi = a.S;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (Hkv * ps[mid] <= pt.x0) lo = mid; else hi = mid - 1;
    }
    int s = lo;
    int64_t x = pt.x0;
    while (x < pt.x1) {
        while (Hkv * ps[s + 1] <= x) ++s;
        const int ct = ps[s + 1] - ps[s];  // segment cost: seg_cost + tiles
        const int64_t cs = Hkv * ps[s];
        const int g = (int)((x - cs) / ct);
        const int64_t ck = cs + (int64_t)g * ct;
        const int64_t t0 = ck + a.seg_cost;  // unit of the segment's first tile
        const int64_t xb = x > t0 ? x : t0;
        const int64_t xe = pt.x1 < ck + ct ? pt.x1 : ck + ct;
        if (xb < xe) {
            // the walk reads the LDS table, so the compiler cannot see that these values are
            // uniform; readfirstlane keeps them, and the addresses built on them, in SGPRs
            Piece pc;
            pc.s = __builtin_amdgcn_readfirstlane(s);
            pc.g = __builtin_amdgcn_readfirstlane(g);
            pc.tb = __builtin_amdgcn_readfirstlane((int)(xb - t0));
            pc.te = __builtin_amdgcn_readfirstlane((int)(xe - t0));
            pc.nt_seg = __builtin_amdgcn_readfirstlane(ct - a.seg_cost);
            pc.slot = __builtin_amdgcn_readfirstlane((int)((int64_t)s * Hkv + g + pt.p_log));
            // the segment's first and last piece tell the merge which slots to combine
            if (threadIdx.x == 0) {
                const int64_t seg = (int64_t)s * Hkv + g;
                if (pc.tb == 0) a.seg_pieces[2 * seg] = pt.p_log;
                if (pc.te == pc.nt_seg) a.seg_pieces[2 * seg + 1] = pt.p_log;
            }
            fn(pc);
        }
        x = ck + ct;
    }
}

// The 16-cell kernel.  At 256-dim heads (q8_0) it runs the head-aligned split of the 32-cell
// q8_0 kernel: neighbouring heads' 272-byte rows share cache lines.
template <int NTW, int KV, int MODE, int D>
__global__ __launch_bounds__((Shape<KV>::waves * 64), (Shape<KV>::waves * t16_groups_per_cu(D) / 4)) void
decode_t16(FaArgs a, int causal) {
    __shared__ DecodeLds<NTW, KV, D> sh;
    if (threadIdx.x < 64) build_tile_prefix(a, sh.ps);
    __syncthreads();
    for_each_piece<D == 256>(a, sh.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece<NTW, KV, MODE, D>(a, sh, causal, pc); });
}

template <int NTW, int RS, int MODE, int D>
__global__ __launch_bounds__((RS * wide_lanes<RS, D>() * 64), (RS * wide_lanes<RS, D>() * WideShape::groups_per_cu + 3) / 4)
void decode_wide(FaArgs a, int causal) {
    __shared__ WideLds<NTW, RS, D, MODE != MODE_FAST> sh;
    if (threadIdx.x < 64) build_tile_prefix(a, sh.st.ps, sh.st.dims);
    __syncthreads();
    for_each_piece<MODE == MODE_FAST>(a, sh.st.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece_wide<NTW, RS, MODE, D>(a, sh, causal, pc); });
}

template <int NTW, int RS, int MODE, int D>
__global__ __launch_bounds__((RS * Q8Dim<D>::TL * 64), (RS * Q8Dim<D>::TL + 3) / 4)
void decode_wide_q8(FaArgs a, int causal) {
    __shared__ WideQ8Lds<NTW, RS, MODE != MODE_FAST, D> sh;
    if (threadIdx.x < 64) build_tile_prefix(a, sh.st.ps, sh.st.dims);
    __syncthreads();
    for_each_piece<true>(a, sh.st.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece_wide_q8<NTW, RS, MODE, D>(a, sh, causal, pc); });
}

// Explicit masks after the pre-pass (fa_mask.hip): the lengths-only block-causal body over the
// offsets the rows imply when every row passed it, the staged-mask (or per-cell) body
// otherwise.  Both run one grid, one slot layout and one merge, so the choice needs no host
// round trip; the LDS is the union of the two bodies'.
template <int NTW, int RS, int D>
union WideDualLds {
    WideLds<NTW, RS, D, false> fast;
    WideLds<NTW, RS, D, true> mask;
};
template <int NTW, int RS, int D>
__global__ __launch_bounds__((RS * wide_lanes<RS, D>() * 64), (RS * wide_lanes<RS, D>() * WideShape::groups_per_cu + 3) / 4)
void decode_wide_dual(FaArgs a) {
    __shared__ WideDualLds<NTW, RS, D> sh;
    __shared__ int wbad[RS * wide_lanes<RS, D>()];
    static_assert(RS * wide_lanes<RS, D>() >= 2, "the table is read by the waves after the first");
    // the first wave builds the lengths body's cost line while the others read the table
    const FaArgs b = mask_as_lengths(a);
    if (threadIdx.x < 64) build_tile_prefix(b, sh.fast.st.ps, sh.fast.st.dims);
    if (mask_rows_block_causal(a, wbad, 64)) {
        for_each_piece<true>(b, sh.fast.st.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece_wide<NTW, RS, MODE_FAST, D>(b, sh.fast, 1, pc); });
    } else {
        if (threadIdx.x < 64) build_tile_prefix(a, sh.mask.st.ps, sh.mask.st.dims);
        __syncthreads();
        for_each_piece<true>(a, sh.mask.st.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece_wide<NTW, RS, MODE_MASK, D>(a, sh.mask, 0, pc); });
    }
}

template <int NTW, int RS, int D>
union WideQ8DualLds {
    WideQ8Lds<NTW, RS, false, D> fast;
    WideQ8Lds<NTW, RS, true, D> mask;
};
template <int NTW, int RS, int D>
__global__ __launch_bounds__((RS * Q8Dim<D>::TL * 64), (RS * Q8Dim<D>::TL + 3) / 4)
void decode_wide_q8_dual(FaArgs a) {
    __shared__ WideQ8DualLds<NTW, RS, D> sh;
    __shared__ int wbad[RS * Q8Dim<D>::TL];
    static_assert(RS * Q8Dim<D>::TL >= 2, "the table is read by the waves after the first");
    const FaArgs b = mask_as_lengths(a);
    if (threadIdx.x < 64) build_tile_prefix(b, sh.fast.st.ps, sh.fast.st.dims);
    if (mask_rows_block_causal(a, wbad, 64)) {
        for_each_piece<true>(b, sh.fast.st.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece_wide_q8<NTW, RS, MODE_FAST, D>(b, sh.fast, 1, pc); });
    } else {
        if (threadIdx.x < 64) build_tile_prefix(a, sh.mask.st.ps, sh.mask.st.dims);
        __syncthreads();
        for_each_piece<true>(a, sh.mask.st.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece_wide_q8<NTW, RS, MODE_MASK, D>(a, sh.mask, 0, pc); });
    }
}

// The 16-cell kernel's dual: the lengths-only body, or per row tile the per-cell body (one
// row tile at a time fits the registers of two work-groups per CU; a mask that is not a
// block-causal prefix then reads the piece's K/V once per row tile).
template <int NTW, int KV, int D>
__global__ __launch_bounds__((Shape<KV>::waves * 64), (Shape<KV>::waves * t16_groups_per_cu(D) / 4)) void
decode_t16_dual(FaArgs a) {
    __shared__ DecodeLds<NTW, KV, D> sh;
    __shared__ int wbad[Shape<KV>::waves];
    static_assert(Shape<KV>::waves >= 2, "the table is read by the waves after the first");
    const FaArgs b = mask_as_lengths(a);
    if (threadIdx.x < 64) build_tile_prefix(b, sh.ps);
    if (mask_rows_block_causal(a, wbad, 64)) {
        for_each_piece<D == 256>(b, sh.ps, [&](const Piece& pc) __attribute__((always_inline)) { decode_piece<NTW, KV, MODE_FAST, D>(b, sh, 1, pc); });
    } else {
        if (threadIdx.x < 64) build_tile_prefix(a, sh.ps);
        __syncthreads();
        for_each_piece<D == 256>(a, sh.ps, [&](const Piece& pc) __attribute__((always_inline)) {
#pragma unroll 1
            for (int n0 = 0; n0 < NTW; ++n0) decode_piece<1, KV, MODE_GENERIC, D, NTW>(a, sh, 0, pc, n0);
        });
    }
}

// Combines the pieces of every segment that more than one work-group touched, for segments of
// many pieces (a few long streams: single-stream decode and verify).  grid = (S*Hkv segments,
// rows); 256 threads = PG piece groups x D/4 threads of four dims.  Group pg folds
// pieces p_first + pg, + PG, ... in increasing order, eight loads per step, all independent, so
// up to 8 PG pieces (64 at 128-dim heads) cost one memory latency; group 0 then folds the
// groups' partials in group order through LDS.  The order is fixed, so the result is
// deterministic.  The split kernel recorded the segment's first and last piece; the stream
// extents come in the same round trip.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_pieces(FaArgs a, int rows_slot) {
    constexpr int TPR = D / 4;     // threads per piece group (4 dims each)
    constexpr int PG = 256 / TPR;  // piece groups: 8 (128-dim heads) or 4 (256)
    __shared__ f32x4 lo[PG][TPR];
    __shared__ float lm[PG], ll[PG];
    const int64_t k = blockIdx.x;
    const int s = (int)(k / a.Hkv);
    const int g = (int)(k % a.Hkv);
    const StreamDims sd = stream_dims(a, s);
    const int p_first = a.seg_pieces[2 * k], p_last = a.seg_pieces[2 * k + 1];
    const int row = blockIdx.y;
    if (row >= a.Gr * sd.ql) return;  // (a segment without rows has stale entries)

    const int pg = (int)(threadIdx.x / TPR), c = (int)(threadIdx.x % TPR);
    const int d0 = c * 4;
    const int j = row / a.Gr;
    const int h = g * a.G + a.hoff + row % a.Gr;
    char* dst = a.out + (int64_t)j * a.o_nb2 + (int64_t)h * a.o_nb1 + (int64_t)s * a.o_nb3 + d0 * 4;
    const f32x4 gv = gate_load(a, s, j, h, d0);  // (fused gate: loaded beside the partials)
    if (p_first == p_last) {
        // written whole by its only work-group; with the fused gate, gated here
        if (a.gate && pg == 0) st16(dst, gated(a, *reinterpret_cast<const f32x4*>(dst), gv));
        return;
    }
    const float* base = a.part + k * a.slot_floats;
    float M = neg_inf(), L = 0.0f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    for (int p0 = p_first + pg; p0 <= p_last; p0 += 8 * PG) {
        f32x4 ov[8];
        float mv[8], lv[8];
        u32x2 hv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int p = p0 + PG * u <= p_last ? p0 + PG * u : p_last;
            const float* sl = base + (int64_t)p * a.piece_stride * a.slot_floats;
            hv[u] = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(sl) + (int64_t)row * (2 * D) + d0 * 2);
            mv[u] = sl[(int64_t)rows_slot * (D / 2) + row];
            lv[u] = sl[(int64_t)rows_slot * (D / 2 + 1) + row];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const f16x4 h = __builtin_bit_cast(f16x4, hv[u]);
            ov[u] = f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]} * lv[u];  // back to O = l * (O/l)
            if (p0 + PG * u <= p_last) merge_row<1>(M, L, &o, mv[u], lv[u], &ov[u]);
        }
    }
    lo[pg][c] = o;
    if (c == 0) {
        lm[pg] = M;
        ll[pg] = L;
    }
    __syncthreads();
    if (pg != 0) return;
#pragma unroll
    for (int q = 1; q < PG; ++q) {
        const f32x4 oq = lo[q][c];
        merge_row<1>(M, L, &o, lm[q], ll[q], &oq);  // a group without pieces adds l = 0, o = 0
    }
    const float inv = L == 0.0f ? 0.0f : 1.0f / L;
    st16(dst, gated(a, o * inv, gv));
}

// Combines the pieces of every segment that more than one work-group touched, for segments of
// few pieces (at most eight on average), in the order of the work-groups.  grid = (S*Hkv
// segments, row blocks of 256 / (D/8) rows); 256 threads = rows x eight-dim chunks, so every
// (row, chunk) is one thread.  The split kernel recorded the
// segment's first and last piece; the stream extents come in the same round trip.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_rows(FaArgs a, int rows_slot) {
    constexpr int DPT = 8;        // dims per thread: one 16-byte partial load, two 16-byte stores
    constexpr int TPR = D / DPT;  // threads per row
    const int64_t k = blockIdx.x;
    const int s = (int)(k / a.Hkv);
    const int g = (int)(k % a.Hkv);
    const StreamDims sd = stream_dims(a, s);
    const int p_first = a.seg_pieces[2 * k], p_last = a.seg_pieces[2 * k + 1];
    const int row = blockIdx.y * (256 / TPR) + (int)(threadIdx.x / TPR);
    if (row >= a.Gr * sd.ql) return;  // (a segment without rows has stale entries)

    const int d0 = (int)(threadIdx.x % TPR) * DPT;
    const int j = row / a.Gr;
    const int h = g * a.G + a.hoff + row % a.Gr;
    char* dst = a.out + (int64_t)j * a.o_nb2 + (int64_t)h * a.o_nb1 + (int64_t)s * a.o_nb3 + d0 * 4;
    // (fused gate: its values load beside the partials)
    const f32x4 gv0 = gate_load(a, s, j, h, d0);
    const f32x4 gv1 = gate_load(a, s, j, h, d0 + 4);
    if (p_first == p_last) {
        // written whole by its only work-group; with the fused gate, gated here
        if (a.gate) {
            const f32x4 w0 = *reinterpret_cast<const f32x4*>(dst), w1 = *reinterpret_cast<const f32x4*>(dst + 16);
            st16(dst, gated(a, w0, gv0));
            st16(dst + 16, gated(a, w1, gv1));
        }
        return;
    }
    const float* base = a.part + k * a.slot_floats;
    float M = neg_inf(), L = 0.0f;
    f32x4 o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    // N pieces per step, their loads independent, so a step costs one memory latency: two or
    // four for the usual segment (no loads beyond its pieces), eight per step beyond
    auto merge_step = [&](auto NC, int p0) {
        constexpr int N = decltype(NC)::value;
        f32x4 ov[N][2];
        float mv[N], lv[N];
        u32x4 hv[N];
#pragma unroll
        for (int u = 0; u < N; ++u) {
            const int p = p0 + u <= p_last ? p0 + u : p_last;
            const float* sl = base + (int64_t)p * a.piece_stride * a.slot_floats;
            hv[u] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(sl) + (int64_t)row * (2 * D) + d0 * 2);
            mv[u] = sl[(int64_t)rows_slot * (D / 2) + row];
            lv[u] = sl[(int64_t)rows_slot * (D / 2 + 1) + row];
        }
#pragma unroll
        for (int u = 0; u < N; ++u) {
            const f16x8 h = as_f16x8(hv[u]);
            // back to O = l * (O/l)
            ov[u][0] = f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]} * lv[u];
            ov[u][1] = f32x4{(float)h[4], (float)h[5], (float)h[6], (float)h[7]} * lv[u];
            if (p0 + u <= p_last) merge_row<2>(M, L, o, mv[u], lv[u], ov[u]);
        }
    };
    if (p_last - p_first < 2) {
        merge_step(std::integral_constant<int, 2>{}, p_first);
    } else if (p_last - p_first < 4) {
        merge_step(std::integral_constant<int, 4>{}, p_first);
    } else {
        for (int p0 = p_first; p0 <= p_last; p0 += 8) merge_step(std::integral_constant<int, 8>{}, p0);
    }
    const float inv = L == 0.0f ? 0.0f : 1.0f / L;
    st16(dst, gated(a, o[0] * inv, gv0));
    st16(dst + 16, gated(a, o[1] * inv, gv1));
}

// The merge form for a split launch: the piece-parallel one once segments average more than
// eight pieces (the row-block form then needs several dependent load steps per row).
template <int D>
void launch_merge(const FaArgs& a, int rows_slot, hipStream_t stream) {
    if ((int64_t)a.P > 8 * (int64_t)a.S * a.Hkv) {
        hipLaunchKernelGGL(decode_merge_pieces<D>, dim3((unsigned)(a.S * a.Hkv), (unsigned)rows_slot), dim3(256), 0,
                           stream, a, rows_slot);
    } else {
        const int rows_wg = 256 / (D / 8);
        hipLaunchKernelGGL(decode_merge_rows<D>,
                           dim3((unsigned)(a.S * a.Hkv), (unsigned)((rows_slot + rows_wg - 1) / rows_wg)), dim3(256), 0,
                           stream, a, rows_slot);
    }
}

// A launch writes partial slots of `rows` rows of D dims: the workspace must hold them.
inline bool slot_fits(const FaArgs& a, int rows, int D) {
    return (int64_t)rows * (D / 2 + 2) <= a.slot_floats;
}

// Head-aligned split: the kv-heads of a cell range go to Hkv work-groups of one XCD that start
// together, so one XCD requests a cell's whole row (all heads) at about the same time.  For
// q8_0 (34*D/32 bytes per head row) neighbouring heads share L2 lines, which are then fetched
// from HBM once, not once per XCD; for f16 the four 256-byte slices of a row are requested
// together (measured 2-3% faster on the 32 x 16 verify).  The grid becomes a multiple of 8 * Hkv.
inline FaArgs head_split_args(const FaArgs& a) {
    FaArgs b = a;
    const int64_t unit = (int64_t)kXcds * a.Hkv;
    if (a.P >= unit) {
        b.P = (int)(a.P / unit * unit);
        b.head_split = 1;
        b.piece_stride = a.Hkv;
        b.xcd_remap = 1;
    }
    return b;
}

// FAST_BUILT: whether the launch shape has a fast-mode kernel (the 32-cell kernel takes f16
// explicit-mask and softcap calls of up to 48 rows as well, whose fast calls run decode_t16).
template <int NTW, int RS, int D, bool FAST_BUILT = true>
hipError_t launch_wide(const FaArgs& a_in, int mode, int causal, hipStream_t stream) {
    // the fast kernels with the head-aligned split
    const FaArgs a = (mode == MODE_FAST) ? head_split_args(a_in) : a_in;
    if (!slot_fits(a, NTW * RS * 16, D)) return hipErrorInvalidValue;
    const dim3 grid(a.P), block(RS * wide_lanes<RS, D>() * 64);
    if (mode == MODE_GENERIC)
        hipLaunchKernelGGL((decode_wide<NTW, RS, MODE_GENERIC, D>), grid, block, 0, stream, a, causal);
    else if (mode == MODE_MASK)
        hipLaunchKernelGGL((decode_wide<NTW, RS, MODE_MASK, D>), grid, block, 0, stream, a, causal);
    else if constexpr (FAST_BUILT)
        hipLaunchKernelGGL((decode_wide<NTW, RS, MODE_FAST, D>), grid, block, 0, stream, a, causal);
    else
        return hipErrorNotSupported;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_merge<D>(a, NTW * RS * 16, stream);
    return hipGetLastError();
}

template <int NTW, int RS, int D = 128>
hipError_t launch_wide_q8(const FaArgs& a_in, int mode, int causal, hipStream_t stream) {
    const FaArgs a = head_split_args(a_in);
    if (!slot_fits(a, NTW * RS * 16, D)) return hipErrorInvalidValue;
    const dim3 grid(a.P), block(RS * Q8Dim<D>::TL * 64);
    if (mode == MODE_GENERIC)
        hipLaunchKernelGGL((decode_wide_q8<NTW, RS, MODE_GENERIC, D>), grid, block, 0, stream, a, causal);
    else if (mode == MODE_MASK)
        hipLaunchKernelGGL((decode_wide_q8<NTW, RS, MODE_MASK, D>), grid, block, 0, stream, a, causal);
    else
        hipLaunchKernelGGL((decode_wide_q8<NTW, RS, MODE_FAST, D>), grid, block, 0, stream, a, causal);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_merge<D>(a, NTW * RS * 16, stream);
    return hipGetLastError();
}

template <int NTW, int KV, int D = 128>
hipError_t launch_nt(const FaArgs& a_in, int mode, int causal, hipStream_t stream) {
    const FaArgs a = (D == 256) ? head_split_args(a_in) : a_in;
    if (!slot_fits(a, NTW * 16, D)) return hipErrorInvalidValue;
    const dim3 grid(a.P), block(Shape<KV>::waves * 64);
    if (mode == MODE_FAST) {
        hipLaunchKernelGGL((decode_t16<NTW, KV, MODE_FAST, D>), grid, block, 0, stream, a, causal);
    } else if constexpr (KV == SIXI_TYPE_Q8_0 && NTW == 1 && D == 128) {
        // (f16 explicit-mask and softcap calls, and q8_0 ones of more than 16 rows or of 256-dim
        // heads, run the 32-cell kernels)
        hipLaunchKernelGGL((decode_t16<NTW, KV, MODE_GENERIC, D>), grid, block, 0, stream, a, causal);
    } else {
        return hipErrorNotSupported;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_merge<D>(a, NTW * 16, stream);
    return hipGetLastError();
}

// The launches of the dual kernels: the fast launches' head-aligned split where they use it.
template <int NTW, int RS, int D>
hipError_t launch_wide_dual(const FaArgs& a_in, hipStream_t stream) {
    const FaArgs a = head_split_args(a_in);
    if (!slot_fits(a, NTW * RS * 16, D)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((decode_wide_dual<NTW, RS, D>), dim3(a.P), dim3(RS * wide_lanes<RS, D>() * 64), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_merge<D>(a, NTW * RS * 16, stream);
    return hipGetLastError();
}

template <int NTW, int RS, int D>
hipError_t launch_wide_q8_dual(const FaArgs& a_in, hipStream_t stream) {
    const FaArgs a = head_split_args(a_in);
    if (!slot_fits(a, NTW * RS * 16, D)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((decode_wide_q8_dual<NTW, RS, D>), dim3(a.P), dim3(RS * Q8Dim<D>::TL * 64), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_merge<D>(a, NTW * RS * 16, stream);
    return hipGetLastError();
}

template <int NTW, int KV, int D>
hipError_t launch_t16_dual(const FaArgs& a_in, hipStream_t stream) {
    const FaArgs a = (D == 256) ? head_split_args(a_in) : a_in;
    if (!slot_fits(a, NTW * 16, D)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((decode_t16_dual<NTW, KV, D>), dim3(a.P), dim3(Shape<KV>::waves * 64), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_merge<D>(a, NTW * 16, stream);
    return hipGetLastError();
}

// Explicit-mask launches with the pre-pass's table (a.row_kl), planned as the lengths-only
// call of the same shape: the 16-cell kernel's dual up to 48 rows (f16 and q8_0 at 128-dim
// heads, q8_0 at 256), the 32-cell kernels' duals beyond (and for f16 at 256-dim heads).
hipError_t launch_decode_dual(const FaArgs& a, int kv_type, int head_dim, int row_tiles, hipStream_t stream) {
    if (!decode_wide_kernel(kv_type, row_tiles, head_dim, false)) {
        if (kv_type == SIXI_TYPE_F16 && head_dim == 128) {
            switch (row_tiles) {
                case 1: return launch_t16_dual<1, SIXI_TYPE_F16, 128>(a, stream);
                case 2: return launch_t16_dual<2, SIXI_TYPE_F16, 128>(a, stream);
                case 3: return launch_t16_dual<3, SIXI_TYPE_F16, 128>(a, stream);
                default: return hipErrorNotSupported;
            }
        }
        if (kv_type == SIXI_TYPE_Q8_0 && head_dim == 128) {
            switch (row_tiles) {
                case 1: return launch_t16_dual<1, SIXI_TYPE_Q8_0, 128>(a, stream);
                case 2: return launch_t16_dual<2, SIXI_TYPE_Q8_0, 128>(a, stream);
                case 3: return launch_t16_dual<3, SIXI_TYPE_Q8_0, 128>(a, stream);
                default: return hipErrorNotSupported;
            }
        }
        if (kv_type == SIXI_TYPE_Q8_0 && head_dim == 256) {
            switch (row_tiles) {
                case 1: return launch_t16_dual<1, SIXI_TYPE_Q8_0, 256>(a, stream);
                case 2: return launch_t16_dual<2, SIXI_TYPE_Q8_0, 256>(a, stream);
                case 3: return launch_t16_dual<3, SIXI_TYPE_Q8_0, 256>(a, stream);
                default: return hipErrorNotSupported;
            }
        }
        return hipErrorNotSupported;
    }
    if (kv_type == SIXI_TYPE_F16 && head_dim == 128) {
        switch (row_tiles) {
            case 4: return launch_wide_dual<kWide64.ntw, kWide64.rs, 128>(a, stream);
            case 6: return launch_wide_dual<kWide96.ntw, kWide96.rs, 128>(a, stream);
            default: return hipErrorNotSupported;
        }
    }
    if (kv_type == SIXI_TYPE_F16 && head_dim == 256) {
        switch (row_tiles) {
            case 1: return launch_wide_dual<1, 1, 256>(a, stream);
            case 2: return launch_wide_dual<2, 1, 256>(a, stream);
            case 4: return launch_wide_dual<2, 2, 256>(a, stream);
            case 6: return launch_wide_dual<2, 3, 256>(a, stream);
            default: return hipErrorNotSupported;
        }
    }
    if (kv_type == SIXI_TYPE_Q8_0 && head_dim == 128) {
        switch (row_tiles) {
            case 4: return launch_wide_q8_dual<kWide64.ntw, kWide64.rs, 128>(a, stream);
            case 6: return launch_wide_q8_dual<kWide96.ntw, kWide96.rs, 128>(a, stream);
            default: return hipErrorNotSupported;
        }
    }
    if (kv_type == SIXI_TYPE_Q8_0 && head_dim == 256) {
        switch (row_tiles) {
            case 4: return launch_wide_q8_dual<2, 2, 256>(a, stream);
            case 6: return launch_wide_q8_dual<2, 3, 256>(a, stream);
            default: return hipErrorNotSupported;
        }
    }
    return hipErrorNotSupported;
}

}  // namespace

int decode_num_groups(const FaArgs& a, int cu_count, int per_cu) {
    const int64_t tiles_max = (int64_t)a.S * a.Hkv * ((a.n_kv + a.tile_cells - 1) / a.tile_cells + a.seg_cost);
    int64_t P = (int64_t)(cu_count > 0 ? cu_count : 256) * per_cu;
    if (P > kMaxSplitGroups) P = kMaxSplitGroups;
    if (P > tiles_max) P = tiles_max;
    // at most about kMaxPieces pieces per segment when the segments are full: more split
    // work-groups would only lengthen the merge of a few long streams
    const int64_t cap = (int64_t)kMaxPieces * a.S * a.Hkv;
    if (P > cap) P = cap;
    return (int)(P < 1 ? 1 : P);
}

hipError_t launch_decode(const FaArgs& a, int kv_type, int mask_mode, int head_dim, int row_tiles,
                         hipStream_t stream) {
    if (a.row_kl || a.mask_inline) return launch_decode_dual(a, kv_type, head_dim, row_tiles, stream);
    // the 32-cell kernel's MASK mode: a staged explicit mask, no softcap, no ALiBi
    const int mode = (mask_mode == SIXI_MASK_EXPLICIT || a.softcap != 0.0f)
                         ? ((mask_mode == SIXI_MASK_EXPLICIT && a.softcap == 0.0f && a.alibi_nlog2 == 0 && a.mask_stage)
                                ? MODE_MASK : MODE_GENERIC)
                         : MODE_FAST;
    const int causal = mask_mode == SIXI_MASK_BLOCK_CAUSAL;
    if (head_dim == 256 && kv_type == SIXI_TYPE_Q8_0) {
        // q8_0 at 256-dim heads, up to 48 rows and lengths only: the 16-cell kernel (four
        // waves per CU, each dequantising its tiles in registers)
        if (mode == MODE_FAST && row_tiles <= 3) {
            switch (row_tiles) {
                case 1: return launch_nt<1, SIXI_TYPE_Q8_0, 256>(a, mode, causal, stream);
                case 2: return launch_nt<2, SIXI_TYPE_Q8_0, 256>(a, mode, causal, stream);
                case 3: return launch_nt<3, SIXI_TYPE_Q8_0, 256>(a, mode, causal, stream);
                default: return hipErrorNotSupported;
            }
        }
        // the rest: the 32-cell q8_0 kernel on one lane, up to two row tiles per wave (33-48
        // rows run as 64)
        switch (row_tiles) {
            case 1: return launch_wide_q8<1, 1, 256>(a, mode, causal, stream);
            case 2: return launch_wide_q8<2, 1, 256>(a, mode, causal, stream);
            case 4: return launch_wide_q8<2, 2, 256>(a, mode, causal, stream);
            case 6: return launch_wide_q8<2, 3, 256>(a, mode, causal, stream);
            default: return hipErrorNotSupported;
        }
    }
    if (head_dim == 256) {
        // 256-dim heads: every row count runs the 32-cell kernel (one or two row groups)
        if (kv_type != SIXI_TYPE_F16) return hipErrorNotSupported;
        // at most two row tiles per wave (three spill the 256-dim accumulators), so 33-48 rows
        // run as 64 (decode_row_tiles maps 3 to 4); 96 rows run as three row groups of one lane
        switch (row_tiles) {
            case 1: return launch_wide<1, 1, 256>(a, mode, causal, stream);
            case 2: return launch_wide<2, 1, 256>(a, mode, causal, stream);
            case 4: return launch_wide<2, 2, 256>(a, mode, causal, stream);
            case 6: return launch_wide<2, 3, 256>(a, mode, causal, stream);
            default: return hipErrorNotSupported;
        }
    }
    if (head_dim != 128) return hipErrorNotSupported;
    if (kv_type == SIXI_TYPE_F16 && mode != MODE_FAST && row_tiles <= 3) {
        // explicit mask or softcap, up to 48 rows: the 32-cell kernel with one row group per lane
        // (its per-cell mask work fits the 512 registers of one wave per SIMD)
        switch (row_tiles) {
            case 1: return launch_wide<1, 1, 128, false>(a, mode, causal, stream);
            case 2: return launch_wide<2, 1, 128, false>(a, mode, causal, stream);
            case 3: return launch_wide<3, 1, 128, false>(a, mode, causal, stream);
            default: return hipErrorNotSupported;
        }
    }
    if (kv_type == SIXI_TYPE_F16) {
        switch (row_tiles) {
            case 1: return launch_nt<1, SIXI_TYPE_F16>(a, mode, causal, stream);
            case 2: return launch_nt<2, SIXI_TYPE_F16>(a, mode, causal, stream);
            case 3: return launch_nt<3, SIXI_TYPE_F16>(a, mode, causal, stream);
            case 4: return launch_wide<kWide64.ntw, kWide64.rs, 128>(a, mode, causal, stream);
            case 6: return launch_wide<kWide96.ntw, kWide96.rs, 128>(a, mode, causal, stream);
            default: return hipErrorNotSupported;
        }
    }
    if (kv_type == SIXI_TYPE_Q8_0) {
        switch (row_tiles) {
            case 1: return launch_nt<1, SIXI_TYPE_Q8_0>(a, mode, causal, stream);
            case 2: return mode == MODE_FAST ? launch_nt<2, SIXI_TYPE_Q8_0>(a, mode, causal, stream)
                                             : launch_wide_q8<2, 1>(a, mode, causal, stream);
            case 3: return mode == MODE_FAST ? launch_nt<3, SIXI_TYPE_Q8_0>(a, mode, causal, stream)
                                             : launch_wide_q8<3, 1>(a, mode, causal, stream);
            case 4: return launch_wide_q8<kWide64.ntw, kWide64.rs>(a, mode, causal, stream);
            case 6: return launch_wide_q8<kWide96.ntw, kWide96.rs>(a, mode, causal, stream);
            default: return hipErrorNotSupported;
        }
    }
    return hipErrorNotSupported;
}

}  // namespace sixi
