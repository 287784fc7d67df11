// fa_prefill.hip -- chunked causal prefill (and any block of more than 96 rows per GQA group)
// on gfx950 f16 MFMA (head_dim 128 and 256 over f16 KV; head_dim 128 over q8_0 KV).
//
// Work decomposition.  One work-group computes 128 consecutive rows (block rows j) of one
// q-head of one stream, over every KV cell those rows see.  The grid is ordered heaviest
// row block first (the last rows of a causal chunk see the most cells), so the long blocks
// start first and the short ones fill in behind them.  Four waves own 32 rows each.
//
// Per 64-cell KV tile (double-buffered in LDS, one barrier per tile), both K and V arrive by
// direct global->LDS loads issued one tile ahead:
//   K   [64 cells][16 chunks of 16 B], chunk q of cell c stored at slot q ^ (c & 15) (each
//       lane fetches the global chunk that lands in its slot), read back conflict-free as
//       MFMA A operands;
//   V   [64 cells][8 chunks of 32 B], chunk q of cell c stored at position q ^ 2(c & 3); the
//       V^T A operands come out of it with ds_read_b64_tr_b16 (within each 16-lane group,
//       lane i receives element i%4 of the 8 bytes addressed by lane 4e + i/4), so no
//       transpose runs through registers.  The 32 lanes of a read pass address 4 cells
//       (c & 3 = 0..3) x 2 chunks: the swizzle spreads them over all 8 positions of a row,
//       i.e. 256 distinct bytes, conflict-free (with c & 7 they covered 4 positions).
//   S^T = K Q^T on v_mfma_f32_32x32x16_f16: A = 32 cells x 16 dims from LDS, B = Q^T held in
//       registers for the whole work-group (lane l: row l%32, dims 16ks + 8(l/32)..+7);
//       lane l receives cells 8b + 4(l/32) + e (b, e < 4) of row l%32, so a row's 64 cells
//       live in lanes l and l^32 and the row max needs one v_permlane32_swap.
//   softmax: lazy exponent reference (moves only when the tile max exceeds it by 2^8),
//       p = 2^(s*c - m*c) in one FMA.
//   O^T += V^T P^T on v_mfma_f32_32x32x16_f16: for the 16-cell step kk the lane's eight
//       values i = 8(kk%2) .. +7 of S^T block kk/2 are exactly its B operand, so the
//       reduction index k = 8(l/32) + e stands for cell 8(e/4) + 4(l/32) + e%4 of the step;
//       the transposed V reads follow the same order.
// Only tiles that reach past the first row's causal boundary (or the stream's end) mask.
//
// Explicit masks without softcap or ALiBi (the ggml hook: MODE_MASK) keep the fast mode's raw
// units and read the mask from LDS: each wave stages its 32 rows x 64 cells of a tile (4 KB)
// by LDS-DMA, the next tile's as soon as it has read the current one.  A wave whose 32 rows
// see none of a tile's cells (a causal mask's upper triangle) skips the tile's MFMAs; a tile
// whose mask is zero for all of them skips the per-cell work.
//
// q8_0 KV (128-dim heads) runs the same tiles: each wave moves 32 q8_0 rows of the next tile
// (K or V, 4352 bytes) by LDS-DMA into the start of the 8 KB of the f16 buffer that those rows
// will occupy, and at the end of the tile rewrites them there as f16 (f16(q * d)), so the LDS
// and the occupancy are the f16 kernel's and the workspace does not grow with the cache.  Q
// goes through ggml's conversion to the q8_0 dot type first, as in the decode kernels.
#include <type_traits>

#include "fa_device.hpp"

namespace sixi {
namespace {

constexpr int kBM = 128;           // rows per work-group
constexpr int kBN = 64;            // cells per KV tile
constexpr int kThreads = 256;      // 4 waves x 32 rows
// Per head dim D: ROW-byte rows, KS k-steps of 16 dims, DB output blocks of 32 dims; a tile of
// K (or V) is kBN rows; LW 1 KB LDS-DMA loads per wave per tile; CPL cells per load.
template <int D>
struct PfDim {
    static constexpr int ROW = 2 * D, KS = D / 16, DB = D / 32, CPR = ROW / 16, CPL = 1024 / ROW;
    static constexpr int TILE = kBN * ROW;            // bytes of a K (or V) tile: 16 KB at 128 dims
    static constexpr int LW = TILE / 1024 / 4;        // loads per wave per tile (4 waves)
    static constexpr int GROUPS = D == 128 ? 2 : 1;   // work-groups per CU (LDS: 4 tiles each)
};
constexpr float kLazyLog2 = 8.0f;

enum { MODE_FAST = 0, MODE_GENERIC = 1, MODE_MASK = 2 };
constexpr int kMaskWave = 32 * kBN * 2;  // bytes of one wave's mask rows of a tile (f16)

// (128-dim heads with the mask: 80 KB, so two work-groups still share a CU's 160 KB)
template <int D, bool MASK>
struct PrefillLds {
    u32x4 k[2][PfDim<D>::TILE / 16];
    u32x4 v[2][PfDim<D>::TILE / 16];
    u32x4 m[MASK ? 4 * kMaskWave / 16 : 1];  // MASK: wave w's rows at kMaskWave * w
};

// q8_0 KV (128-dim heads): block 2h + M of cell c (f16 scale bits d, 32 int8 quants as eight
// little-endian dwords) into a tile's f16 layout at dst: K chunk j (dims 8j .. 8j+7) at slot
// j ^ (c % 16), V's 32-byte chunk j/2 at position (j/2) ^ 2(c % 4).  `key` is the lane's part
// of those slots, (8h) ^ (c % 16) for K and (4h) ^ 2(c % 4) for V, so that each store address
// is one XOR with a constant.  The values are f16(q * d), one rounding, as every q8_0 path of
// this library dequantises.
template <bool IS_V, int M>
__device__ __forceinline__ void pf_q8_block_store(char* dst, int c, int key, uint16_t d, const uint32_t (&w)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int pos = IS_V ? 32 * (key ^ (2 * M + (k >> 1))) + 16 * (k & 1) : 16 * (key ^ (4 * M + k));
        *reinterpret_cast<u32x4*>(dst + c * 256 + pos) = dequant_q8x8(w[2 * k], w[2 * k + 1], d);
    }
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// QQ8: Q goes through ggml's conversion to the q8_0 dot type (a q8_0 cache, read as q8_0 tiles or
// staged as f16 rows).
template <int MODE, int D, int KV, bool QQ8>
__device__ __forceinline__ void prefill_body(const FaArgs& a, int causal, int nrb, int n_cu,
                                             PrefillLds<D, MODE == MODE_MASK>& sh) {
    using P = PfDim<D>;
    constexpr bool Q8 = KV == SIXI_TYPE_Q8_0;
    static_assert(QQ8 || !Q8, "q8_0 tiles take a q8_0-converted Q");
    constexpr int GROUPS = P::GROUPS;
    constexpr int kKBytes = P::TILE, kVBytes = P::TILE;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int hl = lane >> 5;      // lane half
    const int rl = lane & 31;      // row inside the wave / M index inside an MFMA block

    // Work-group order.  (row block, head) items are ranked heaviest first (the last rows of
    // a causal chunk see the most cells).  The first n_cu work-groups take a CU each and the
    // next ones (up to n_cu more) join the earliest of them, where both run slower than a
    // work-group alone on its CU; so the heaviest ranks go to the positions that keep a CU to
    // themselves, the next ranks to the positions that will be joined, the lightest last.
    const int SH = a.S * a.H;
    const int b = blockIdx.x;
    const int N = gridDim.x;
    int rank = b;
    if (GROUPS == 2 && N > n_cu && N <= 2 * n_cu) {
        const int npair = N - n_cu;
        const int alone = n_cu - npair;
        if (b < npair) rank = alone + b;
        else if (b < n_cu) rank = b - npair;
    }
    const int rb = nrb - 1 - rank / SH;
    const int s = (rank % SH) / a.H;
    const int h = (rank % SH) % a.H;
    const int g = h / a.G;
    const StreamDims sd = stream_dims(a, s);
    const int j0 = rb * kBM;
    if (j0 >= sd.ql) return;
    const int j_last = min(j0 + kBM, sd.ql) - 1;
    const int j = j0 + 32 * w + rl;  // this lane's row
    const bool row_ok = j < sd.ql;

    // cells each row sees; tiles below t_full are unmasked for every row of the group
    const int vis = causal ? sd.kl + min(j, j_last) + 1 : sd.nc;
    const int vis_max = causal ? sd.kl + j_last + 1 : sd.nc;
    const int vis_min = causal ? sd.kl + j0 + 1 : sd.nc;
    const int n_tiles = (vis_max + kBN - 1) / kBN;
    const int t_full = (MODE == MODE_GENERIC) ? 0 : vis_min / kBN;
    constexpr bool RAW = MODE != MODE_GENERIC;  // scores in raw dot-product units
    const int t_beg = 0, t_end = n_tiles;  // the tiles walked

    // ---- Q^T B operands in registers: lane l -> row j, dims 16ks + 8*hl .. +7 ----
    // (every load issued before any is used; rows past the block read its first row)
    f16x8 qop[P::KS];
    if constexpr (QQ8) {
        // ggml's conversion of Q to the q8_0 dot type: per 32-dim block (ks = 2bq, 2bq + 1 of
        // lanes l and l^32) d = amax/127, q = round-half-away(x * 127/amax) clamped to +-127,
        // and the MFMA takes f16(q * f16(d))
        const char* src = a.q + (int64_t)(row_ok ? j : j0) * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)s * a.q_nb3;
        float xq[P::KS][8];
        if (a.q_f16) {
            u32x4 raw[P::KS];
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks) raw[ks] = ld16(src + (16 * ks + 8 * hl) * 2);
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) xq[ks][e] = (float)as_f16x8(raw[ks])[e];
        } else {
            f32x4 lo[P::KS], hi[P::KS];
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks) {
                lo[ks] = *reinterpret_cast<const f32x4*>(src + (16 * ks + 8 * hl) * 4);
                hi[ks] = *reinterpret_cast<const f32x4*>(src + (16 * ks + 8 * hl) * 4 + 16);
            }
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xq[ks][e] = lo[ks][e];
                    xq[ks][4 + e] = hi[ks][e];
                }
        }
#pragma unroll
        for (int bq = 0; bq < P::KS / 2; ++bq) {
            float am = 0.0f;
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(xq[2 * bq + k2][e]));
            am = fmaxf(am, __shfl_xor(am, 32, 64));
            const float d = am / 127.0f;
            const float id = d != 0.0f ? 127.0f / am : 0.0f;
            const float dh = (float)(_Float16)d;
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                f16x8 hv;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    hv[e] = (_Float16)(fminf(fmaxf(roundf(xq[2 * bq + k2][e] * id), -127.0f), 127.0f) * dh);
                qop[2 * bq + k2] = row_ok ? hv : f16x8{};
            }
        }
    } else {
        const char* src = a.q + (int64_t)(row_ok ? j : j0) * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)s * a.q_nb3;
        if (a.q_f16) {
            u32x4 raw[P::KS];
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks) raw[ks] = ld16(src + (16 * ks + 8 * hl) * 2);
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks) qop[ks] = row_ok ? as_f16x8(raw[ks]) : f16x8{};
        } else {
            f32x4 lo[P::KS], hi[P::KS];
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks) {
                lo[ks] = *reinterpret_cast<const f32x4*>(src + (16 * ks + 8 * hl) * 4);
                hi[ks] = *reinterpret_cast<const f32x4*>(src + (16 * ks + 8 * hl) * 4 + 16);
            }
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks) {
                f16x8 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hv[e] = (_Float16)lo[ks][e];
                    hv[4 + e] = (_Float16)hi[ks][e];
                }
                qop[ks] = row_ok ? hv : f16x8{};
            }
        }
    }

    // K/V of (stream, kv-head): every tile gets its own range-checked buffer resource whose
    // base is the tile's first cell (in its page, for paged caches), so cells >= nc read as
    // zero and no load can fault
    const int64_t rowb = P::ROW;
    const uint32_t knb = (uint32_t)a.k_nb1, vnb = (uint32_t)a.v_nb1;

    // ---- per-lane LDS byte offsets, fixed for the whole loop ----
    char* lds = reinterpret_cast<char*>(&sh);
    const uint32_t lds0 = lds_addr(&sh);
    constexpr int kVBase = 2 * kKBytes;  // the V buffers follow the two K buffers
    // K A operand of (cb, ks): cell 32cb + rl, chunk (2ks + hl) stored at slot chunk ^ (rl & 15)
    uint32_t koff[P::KS];
#pragma unroll
    for (int ks = 0; ks < P::KS; ++ks) koff[ks] = rl * P::ROW + ((((2 * ks + hl) ^ (rl & 15)) & (P::CPR - 1)) << 4);
    // K staging: wave w's load u fills cells CPL(LW w + u) + l/CPR; lane fetches chunk (l%CPR)^cell
    // (the XOR touches the low four bits of the chunk index)
    uint32_t kdo[P::LW];
#pragma unroll
    for (int u = 0; u < P::LW; ++u) {
        const int cell = P::CPL * (P::LW * w + u) + lane / P::CPR;
        kdo[u] = (uint32_t)cell * knb + (uint32_t)(((lane % P::CPR) ^ (cell & 15)) * 16);
    }
    // V staging: wave w's load u fills LDS row CPL(LW w + u) + t/CPR at 16-byte position
    // t%CPR, i.e. 32-byte chunk position (t%CPR)/2 of the row, which holds dims
    // 16 * (position ^ 2(row % 4))
    uint32_t vdo[P::LW];
#pragma unroll
    for (int u = 0; u < P::LW; ++u) {
        const int cell = P::CPL * (P::LW * w + u) + lane / P::CPR;
        const int pos = lane % P::CPR;
        vdo[u] = (uint32_t)cell * vnb + 32u * (uint32_t)((pos >> 1) ^ (2 * (cell & 3))) + 16u * (uint32_t)(pos & 1);
    }
    // V^T A operand of (db, kk), half h: lane (G = l/16, q = l%16) addresses cell
    // 16kk + 8h + x, x = 4(G/2) + q/4, dims 32db + 16(G%2) + 4(q%4) .. +3, which sits in chunk
    // position (2db + G%2) ^ 2(x % 4).  The row offset has the bits that 64db touches clear,
    // so the address is (row + 32*((G%2) ^ 2(x % 4)) + 8(q%4)) ^ 64db + (16kk + 8h)*ROW.
    uint32_t vtr[P::DB];
    {
        const int G = lane >> 4, q = lane & 15;
        const int x = 4 * (G >> 1) + (q >> 2);
        const uint32_t base = (uint32_t)x * (uint32_t)P::ROW + 32u * (uint32_t)((G & 1) ^ (2 * (x & 3))) + 8u * (uint32_t)(q & 3);
#pragma unroll
        for (int db = 0; db < P::DB; ++db) vtr[db] = lds0 + kVBase + (base ^ (64u * db));
    }

    PageIds pages = page_ids_load(a, s, 0);
    auto issue_kv = [&](int t, int buf) {
        const int page = t * kBN < sd.nc ? page_id(pages, a, s, (t * kBN) >> 8) : 0;
        const KvSpan ksp = kv_span(a, a.k, a.k_nb1, a.k_nb2, a.k_nb3, s, g, t * kBN, sd.nc, rowb, page);
        const KvSpan vsp = kv_span(a, a.v, a.v_nb1, a.v_nb2, a.v_nb3, s, g, t * kBN, sd.nc, rowb, page);
        const buf_rsrc krs = make_rsrc_uniform(ksp.p, ksp.bytes);
        const buf_rsrc vrs = make_rsrc_uniform(vsp.p, vsp.bytes);
        if constexpr (P::LW == 4) {
            dma16x4_to_lds(krs, kdo, lds0 + buf * kKBytes + 4 * w * 1024);
            dma16x4_to_lds(vrs, vdo, lds0 + kVBase + buf * kVBytes + 4 * w * 1024);
        } else {
            dma16x8_to_lds(krs, kdo, lds0 + buf * kKBytes + 8 * w * 1024);
            dma16x8_to_lds(vrs, vdo, lds0 + kVBase + buf * kVBytes + 8 * w * 1024);
        }
    };

    // Q8: wave w moves the q8_0 rows of K cells 32(w % 2) .. +31 (w < 2) or V cells (w >= 2)
    // of the next tile by 17 dword LDS-DMA loads (two row heads of 128 contiguous bytes per
    // load, then the rows' last 8 bytes) into the start of its own 8 KB of that tile's f16
    // buffer -- the rows it later writes as f16 -- and converts them there in place: no other
    // wave reads or writes that slice before the barrier, so the f16 tiles are all the LDS it
    // takes.
    const int wq = __builtin_amdgcn_readfirstlane(w);
    const uint32_t q8nb = (uint32_t)__builtin_amdgcn_readfirstlane((int)(wq >= 2 ? a.v_nb1 : a.k_nb1));
    // byte offset of this wave's slice in f16 buffer `buf`
    auto q8_slice = [&](int buf) { return (wq >= 2 ? kVBase + buf * kVBytes : buf * kKBytes) + (wq & 1) * 32 * P::ROW; };
    auto issue_q8 = [&](int t, int buf) {
        if constexpr (Q8) {
            const int page = t * kBN < sd.nc ? page_id(pages, a, s, (t * kBN) >> 8) : 0;
            constexpr int Q8ROW = D / 32 * 34;
            const KvSpan sp = wq >= 2 ? kv_span(a, a.v, a.v_nb1, a.v_nb2, a.v_nb3, s, g, t * kBN, sd.nc, Q8ROW, page)
                                      : kv_span(a, a.k, a.k_nb1, a.k_nb2, a.k_nb3, s, g, t * kBN, sd.nc, Q8ROW, page);
            const buf_rsrc rs = make_rsrc_uniform(sp.p, sp.bytes);
            // (the lane offsets are recomputed here, not kept in registers across the tile)
            uint32_t l = (uint32_t)lane;
            asm volatile("" : "+v"(l));
            const uint32_t r0 = 32u * (uint32_t)(wq & 1);
            if constexpr (D == 128) {
                const uint32_t v = (r0 + (l >> 5)) * q8nb + 4u * (l & 31);
                const uint32_t vx = (r0 + (l >> 1)) * q8nb + 128u + 4u * (l & 1);
                dma_q8rows32_to_lds(rs, v, vx, 2u * q8nb, lds0 + (uint32_t)q8_slice(buf));
            } else {
                // 272-byte rows (16-byte aligned): 16-byte piece c = 64u + l of the 32 rows --
                // row c / 17, piece c % 17 -- lands at 16c, so row x occupies bytes 272x ..
                // 272x + 271 of the slice (the ninth load's upper half runs past the rows,
                // inside the slice)
                uint32_t o[9];
#pragma unroll
                for (int u = 0; u < 9; ++u) {
                    const uint32_t c = 64u * (uint32_t)u + l;
                    o[u] = (r0 + c / 17u) * q8nb + 16u * (c % 17u);
                }
                uint32_t o8[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) o8[u] = o[u];
                const uint32_t dst = lds0 + (uint32_t)q8_slice(buf);
                dma16x8_to_lds(rs, o8, dst);
                dma16x1_to_lds(rs, o[8], dst + 8u * 1024u);
            }
        }
    };
    // this wave's q8_0 rows in f16 buffer BUF (landed) -> f16 rows of the same slice.  Lane
    // (x = l % 32, h = l / 32) reads blocks 2h and 2h + 1 of row x, dwords 17h .. 17h + 16 --
    // dword c < 32 at byte 264(x/2) + 128(x%2) + 4c, dwords 32, 33 at 4224 + 8x, so the 64
    // lanes of each read hit 64 distinct banks -- every read before any write.
    auto convert_q8 = [&](auto BUF) {
        if constexpr (Q8 && D == 256) {
            constexpr int buf = decltype(BUF)::value;
            char* sl = lds + q8_slice(buf);
            // lane (x = l % 32, h = l / 32) takes blocks 4h .. 4h+3 of row x: the 136 bytes at
            // 272x + 136h (8-byte aligned), all read before any write
            int lx = lane;
            asm volatile("" : "+v"(lx));
            const int x = lx & 31, hx = lx >> 5;
            const u32x2* src = reinterpret_cast<const u32x2*>(sl + 272 * x + 136 * hx);
            uint32_t r[34];
#pragma unroll
            for (int i = 0; i < 17; ++i) {
                const u32x2 v2 = src[i];
                r[2 * i] = v2[0];
                r[2 * i + 1] = v2[1];
            }
            asm volatile("" ::: "memory");
            // block m at byte 34m: m even -> scale in the low half of dword 17m/2, quants 2 bytes
            // past the following dwords; m odd -> scale in the high half, quants dword-aligned
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int d0 = (34 * m) >> 2;
                uint32_t wq8[8];
                uint16_t dh;
                if (m & 1) {
                    dh = (uint16_t)(r[d0] >> 16);
#pragma unroll
                    for (int i = 0; i < 8; ++i) wq8[i] = r[d0 + 1 + i];
                } else {
                    dh = (uint16_t)(r[d0] & 0xffffu);
#pragma unroll
                    for (int i = 0; i < 8; ++i) wq8[i] = __builtin_amdgcn_alignbyte(r[d0 + i + 1], r[d0 + i], 2);
                }
                const int bk = 4 * hx + m;  // block: dims 32bk .. 32bk+31
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const u32x4 f = dequant_q8x8(wq8[2 * k], wq8[2 * k + 1], dh);
                    const int j = 4 * bk + k;  // 16-byte chunk: dims 8j .. 8j+7
                    const int pos = wq >= 2 ? 32 * ((j >> 1) ^ (2 * (x & 3))) + 16 * (j & 1) : 16 * (j ^ (x & 15));
                    *reinterpret_cast<u32x4*>(sl + x * P::ROW + pos) = f;
                }
            }
        } else if constexpr (Q8) {
            constexpr int buf = decltype(BUF)::value;
            char* sl = lds + q8_slice(buf);
            // (addresses and store keys are recomputed here, not kept in registers across the tile)
            int lx = lane;
            asm volatile("" : "+v"(lx));
            const int x = lx & 31, hx = lx >> 5;
            const int bx = 264 * (x >> 1) + 128 * (x & 1);
            const uint32_t* src = reinterpret_cast<const uint32_t*>(sl + bx + 68 * hx);
            const uint32_t* src2 = reinterpret_cast<const uint32_t*>(sl + (hx ? 4224 + 8 * x : bx + 60));
            uint32_t r[17];
#pragma unroll
            for (int i = 0; i < 15; ++i) r[i] = src[i];
            r[15] = src2[0];
            r[16] = src2[1];
            asm volatile("" ::: "memory");
            // block 2h: scale in the low half of dword 0, quants 2 bytes past dwords 0..8;
            // block 2h + 1: scale in the high half of dword 8, quants dwords 9..16
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);
                hi[i] = r[9 + i];
            }
            const uint16_t dlo = (uint16_t)(r[0] & 0xffffu), dhi = (uint16_t)(r[8] >> 16);
            const int key = wq < 2 ? (8 * hx) ^ (x & 15) : (4 * hx) ^ (2 * (x & 3));
            if (wq < 2) {
                pf_q8_block_store<false, 0>(sl, x, key, dlo, lo);
                pf_q8_block_store<false, 1>(sl, x, key, dhi, hi);
            } else {
                pf_q8_block_store<true, 0>(sl, x, key, dlo, lo);
                pf_q8_block_store<true, 1>(sl, x, key, dhi, hi);
            }
        }
    };

    f32x16 acc[P::DB];  // O^T blocks: dims 32db + 8(i/4) + 4hl + i%4 of row j
#pragma unroll
    for (int db = 0; db < P::DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[db][i] = 0.0f;
    float m_ref = neg_inf();  // raw score (FAST) or log2 units (GENERIC)
    float l_sum = 0.0f;
    const float c2 = a.scale_log2;
    const float thr = RAW ? kLazyLog2 / c2 : kLazyLog2;
    const float slope = (MODE == MODE_GENERIC) ? alibi_slope(a, h) : 1.0f;
    const char* mrow = nullptr;
    if (MODE == MODE_GENERIC && a.mask)
        mrow = a.mask + (int64_t)(s % a.m_ne3) * a.m_nb3 + (int64_t)min(j, j_last) * a.m_nb1;
    const f32x16 zero16 = {};

    // MODE_MASK: the stream's mask rows through a range-checked resource (exactly its n_q rows);
    // wave w's load u stages its rows 8u + l/8, the 16-byte piece at slot l%8 of a row
    // holding cells 8((l%8) ^ ((row >> 1) & 7)) .. +7 of the tile, so that the 32 lanes of a
    // read (one row each, same piece) spread over the banks
    buf_rsrc mrs = make_rsrc(a.q, 0u);  // (empty unless MODE_MASK)
    uint32_t mdo[4] = {0u, 0u, 0u, 0u};
    const uint32_t m_lds = lds0 + 4 * kKBytes + (uint32_t)w * kMaskWave;
    const float inv_scale = 1.0f / a.scale;
    if constexpr (MODE == MODE_MASK) {
        mrs = make_rsrc_uniform(a.mask + (int64_t)(s % a.m_ne3) * a.m_nb3, (uint32_t)a.m_span);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = 8 * u + lane / 8;
            const int jr = min(j0 + 32 * w + r, j_last);
            mdo[u] = (uint32_t)((int64_t)jr * a.m_nb1) + 16u * (uint32_t)((lane % 8) ^ ((r >> 1) & 7));
        }
    }
    auto issue_mask = [&](int t) {
        if constexpr (MODE == MODE_MASK) {
            uint32_t o[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) o[u] = mdo[u] + (uint32_t)(t * kBN) * 2u;
            dma16x4_to_lds(mrs, o, m_lds);
        }
    };

    // One tile from LDS buffer BUF (compile-time, so every LDS offset is an immediate).
    auto tile = [&](int t, auto BUF, auto MASKED) {
        constexpr int buf = decltype(BUF)::value;
        constexpr bool masked = decltype(MASKED)::value;
        const bool more = t + 1 < t_end;
        if (more) {
            if constexpr (Q8) issue_q8(t + 1, buf ^ 1);
            else issue_kv(t + 1, buf ^ 1);
        }
        const int c0 = t * kBN;
        const char* kt = lds + buf * kKBytes;

        // MODE_MASK: this wave's mask values of the lane's 32 cells (row rl, cells
        // 32cb + 8b + 4hl .. +3: piece 4cb + b, half hl), then the next tile's rows into the
        // same place (once the reads have returned)
        u32x2 mv[2][4];
        bool mask_any = false, live = true;
        if constexpr (MODE == MODE_MASK) {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    mv[cb][b] = lds_ld8(m_lds + 128u * (uint32_t)rl +
                                        16u * (uint32_t)((4 * cb + b) ^ ((rl >> 1) & 7)) + 8u * (uint32_t)hl);
            uint32_t nz = 0, alive = 0;
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        nz |= mv[cb][b][e] & 0x7fff7fffu;
                        // a cell is seen unless its value is -inf (0xfc00) or it lies past the stream
                        const int cell = c0 + 32 * cb + 8 * b + 4 * hl + 2 * e;
                        alive |= ((mv[cb][b][e] & 0xffffu) != 0xfc00u && cell < sd.nc) ? 1u : 0u;
                        alive |= ((mv[cb][b][e] >> 16) != 0xfc00u && cell + 1 < sd.nc) ? 1u : 0u;
                    }
            mask_any = __builtin_amdgcn_ballot_w64(nz != 0) != 0;
            live = __builtin_amdgcn_ballot_w64(row_ok && alive != 0) != 0;
            wait_lgkmcnt0();
            if (t + 1 < t_end) issue_mask(t + 1);
        }
        if (live) {

        // ---- S^T = K Q^T: two 32-cell blocks ----
        // (the MFMA phases run at raised wave priority, so that the SIMD feeds the matrix core of
        // the wave in an MFMA phase first while the other wave on the SIMD works its softmax)
        __builtin_amdgcn_s_setprio(1);
        f32x16 st[2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            st[cb] = mfma32x32x16(as_f16x8(*reinterpret_cast<const u32x4*>(kt + cb * 32 * P::ROW + koff[0])), qop[0],
                                  zero16);
#pragma unroll
            for (int ks = 1; ks < P::KS; ++ks)
                st[cb] = mfma32x32x16(as_f16x8(*reinterpret_cast<const u32x4*>(kt + cb * 32 * P::ROW + koff[ks])),
                                      qop[ks], st[cb]);
        }

        __builtin_amdgcn_s_setprio(0);

        // ---- scores, row max (lanes l and l^32 hold the row's 64 cells) ----
        float mx = neg_inf();
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int cell = c0 + 32 * cb + 8 * (i >> 2) + 4 * hl + (i & 3);
                float x = st[cb][i];
                if (MODE == MODE_GENERIC) {
                    x *= a.scale;
                    if (a.softcap != 0.0f) x = a.softcap * tanhf(x);
                    if (a.mask) {
                        float mv = neg_inf();
                        if (cell < sd.nc)
                            mv = slope * half_bits_to_float(*reinterpret_cast<const uint16_t*>(mrow + (int64_t)cell * 2));
                        x = (mv == neg_inf()) ? neg_inf() : x + mv;
                    } else if (cell >= vis) {
                        x = neg_inf();
                    }
                    x *= kLog2e;
                } else if (MODE == MODE_MASK) {
                    // raw units: s = dot + mask / scale; -inf (or a cell past the stream) skips it
                    if (mask_any) {
                        const uint32_t wv = mv[cb][i >> 2][(i & 3) >> 1];
                        const float m = half_bits_to_float((uint16_t)((i & 1) ? (wv >> 16) : (wv & 0xffffu)));
                        x = (m == neg_inf() || (masked && cell >= sd.nc)) ? neg_inf() : fmaf(m, inv_scale, x);
                    } else if (masked && cell >= sd.nc) {
                        x = neg_inf();
                    }
                } else if (masked) {
                    if (cell >= vis) x = neg_inf();
                }
                st[cb][i] = x;
            }
#pragma unroll
            for (int i = 0; i < 16; i += 8)
                mx = max3f(mx, max3f(st[cb][i], st[cb][i + 1], st[cb][i + 2]),
                           max3f(max3f(st[cb][i + 3], st[cb][i + 4], st[cb][i + 5]), st[cb][i + 6], st[cb][i + 7]));
        }
        {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }

        // ---- lazy exponent reference ----
        const bool need = mx > m_ref + thr;
        if (__builtin_amdgcn_ballot_w64(need) != 0) {
            float alpha = 1.0f;
            if (need) {
                alpha = fast_exp2(RAW ? (m_ref - mx) * c2 : m_ref - mx);
                m_ref = mx;
            }
            l_sum *= alpha;
#pragma unroll
            for (int db = 0; db < P::DB; ++db) acc[db] *= alpha;
        }

        // ---- probabilities ----
        const float mc = (m_ref == neg_inf()) ? 0.0f : (RAW ? m_ref * c2 : m_ref);
        // B operands of the four 16-cell steps (f16 pairs by packed RNE conversion) and the
        // row sum of exactly those f16 probabilities, two per v_dot2_f32_f16
        f16x8 pb[4];
        float part[4] = {0.f, 0.f, 0.f, 0.f};
        const f16x2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                f32x2 pp;
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    pp[e] = fast_exp2(RAW ? fmaf(st[cb][i + e], c2, -mc) : st[cb][i + e] - mc);
                const f16x2 ph = __builtin_convertvector(pp, f16x2);
                pb[2 * cb + (i >> 3)][i & 7] = ph[0];
                pb[2 * cb + (i >> 3)][(i & 7) + 1] = ph[1];
                part[(i >> 1) & 3] = __builtin_amdgcn_fdot2(ph, one2, part[(i >> 1) & 3], false);
            }
        l_sum += (part[0] + part[1]) + (part[2] + part[3]);

        // Explicit masks: a cell that none of this wave's 32 rows sees may hold NaN bits, so
        // its V^T entries are zeroed in this wave's operands (0 * NaN must not reach O).
        uint32_t keep[4][4];
        const bool use_keep = (MODE == MODE_GENERIC && a.mask) || (MODE == MODE_MASK && mask_any);
        if (use_keep) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int m2 = 0; m2 < 4; ++m2) {
                    const uint64_t b0 = __builtin_amdgcn_ballot_w64((float)pb[kk][2 * m2] != 0.0f);
                    const uint64_t b1 = __builtin_amdgcn_ballot_w64((float)pb[kk][2 * m2 + 1] != 0.0f);
                    keep[kk][m2] = ((((b0 >> (32 * hl)) & 0xffffffffull) != 0) ? 0x0000ffffu : 0u) |
                                   ((((b1 >> (32 * hl)) & 0xffffffffull) != 0) ? 0xffff0000u : 0u);
                }
        }

        // ---- O^T += V^T P^T, V^T by transposed reads of the V rows ----
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int db = 0; db < P::DB; ++db) {
                const lds_char* vp = lds_ptr(vtr[db] + buf * kVBytes + kk * 16 * P::ROW);
                const u32x2 lo = ld_tr16(vp);
                const u32x2 hi = ld_tr16(vp + 8 * P::ROW);
                u32x4 vop = {lo[0], lo[1], hi[0], hi[1]};
                if (use_keep) {
#pragma unroll
                    for (int m2 = 0; m2 < 4; ++m2) vop[m2] &= keep[kk][m2];
                }
                acc[db] = mfma32x32x16(as_f16x8(vop), pb[kk], acc[db]);
            }
        }

        __builtin_amdgcn_s_setprio(0);
        }  // live
        if (more) {
            // this wave's share of tile t+1 (and, masked, its mask rows) is in LDS; Q8: it
            // becomes f16 in place
            wait_vmcnt<0>();
            if constexpr (Q8) convert_q8(std::integral_constant<int, buf ^ 1>{});
        }
        __syncthreads();
    };
    // (256-dim heads run every tail tile masked: two bodies per buffer in one loop would merge
    // their accumulator sets, and the registers are all taken; at most one tail tile is
    // unmasked, and the mask passes its cells)
    auto run_tile = [&](int t, auto BUF) {
        if (D == 128 && RAW && t < t_full)
            tile(t, BUF, std::integral_constant<bool, false>{});
        else
            tile(t, BUF, std::integral_constant<bool, true>{});
    };

    // prologue: the first tile into buffer 0
    if (t_beg < t_end) {
        if constexpr (Q8) issue_q8(t_beg, 0);
        else issue_kv(t_beg, 0);
        issue_mask(t_beg);
        wait_vmcnt<0>();
        if constexpr (Q8) convert_q8(std::integral_constant<int, 0>{});
    }
    __syncthreads();

    // the unmasked tiles in pairs (buffers 0, 1), then the tail with the masked tiles, so
    // each loop holds one copy of the tile body per buffer
    const int t_fast = RAW ? min(t_full, t_end) : 0;
    int t = t_beg;
#pragma unroll 1
    for (; t + 2 <= t_fast; t += 2) {
        tile(t, std::integral_constant<int, 0>{}, std::integral_constant<bool, false>{});
        tile(t + 1, std::integral_constant<int, 1>{}, std::integral_constant<bool, false>{});
    }
#pragma unroll 1
    for (; t < t_end; t += 2) {
        run_tile(t, std::integral_constant<int, 0>{});
        if (t + 1 < t_end) run_tile(t + 1, std::integral_constant<int, 1>{});
    }

    // ---- normalise and write: lane holds dims 32db + 8b + 4hl .. +3 of row j ----
    {
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_sum), __float_as_uint(l_sum), false, false);
        l_sum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    if (row_ok) {
        // (the row and its address are recomputed from the lane here rather than held across
        // the tile loop)
        int lx = lane;
        asm volatile("" : "+v"(lx));
        const int jw = j0 + 32 * wq + (lx & 31), hw = lx >> 5;
        const float inv = l_sum == 0.0f ? 0.0f : 1.0f / l_sum;
        char* dst = a.out + (int64_t)jw * a.o_nb2 + (int64_t)h * a.o_nb1 + (int64_t)s * a.o_nb3;
#pragma unroll
        for (int db = 0; db < P::DB; ++db)
#pragma unroll
            for (int bq = 0; bq < 4; ++bq)
                st16(dst + (32 * db + 8 * bq + 4 * hw) * 4,
                     gated(a, f32x4{acc[db][4 * bq], acc[db][4 * bq + 1], acc[db][4 * bq + 2], acc[db][4 * bq + 3]} * inv,
                           gate_load(a, s, jw, h, 32 * db + 8 * bq + 4 * hw)));
    }
}

template <int MODE, int D>
__global__ __launch_bounds__(kThreads, PfDim<D>::GROUPS) void prefill_f16(FaArgs a, int causal, int nrb, int n_cu) {
    __shared__ PrefillLds<D, MODE == MODE_MASK> sh;
    prefill_body<MODE, D, SIXI_TYPE_F16, false>(a, causal, nrb, n_cu, sh);
}

// f16 rows staged from a q8_0 cache: Q converted to the q8_0 dot type in the kernel
template <int MODE, int D>
__global__ __launch_bounds__(kThreads, PfDim<D>::GROUPS) void prefill_f16_qq8(FaArgs a, int causal, int nrb, int n_cu) {
    __shared__ PrefillLds<D, MODE == MODE_MASK> sh;
    prefill_body<MODE, D, SIXI_TYPE_F16, true>(a, causal, nrb, n_cu, sh);
}

// q8_0 KV: the same tiles, converted from q8_0 rows in place in LDS
template <int MODE, int D>
__global__ __launch_bounds__(kThreads, PfDim<D>::GROUPS) void prefill_q8(FaArgs a, int causal, int nrb, int n_cu) {
    __shared__ PrefillLds<D, MODE == MODE_MASK> sh;
    prefill_body<MODE, D, SIXI_TYPE_Q8_0, true>(a, causal, nrb, n_cu, sh);
}

// Explicit masks after the pre-pass (fa_mask.hip).  GATE 1 runs the lengths-only block-causal
// body over the offsets the rows imply when every row passed the pre-pass, GATE 2 the
// staged-mask body when one did not; each returns after reading the pre-pass's table when the
// other one's case holds, and the two run as a pair of launches at 128-dim heads (one kernel
// holding both bodies needs more than the 256 registers per wave of two work-groups per CU).
// GATE 0 holds both bodies (the LDS of the larger), one launch: 256-dim heads, which run one
// work-group per CU either way.
template <int D>
union PrefillDualLds {
    PrefillLds<D, false> fast;
    PrefillLds<D, true> mask;
};
template <int D, int GATE>
using GatedLds = std::conditional_t<GATE == 0, PrefillDualLds<D>, PrefillLds<D, GATE == 2>>;
template <int D, int KV, bool QQ8, int GATE>
__global__ __launch_bounds__(kThreads, PfDim<D>::GROUPS) void prefill_gated(FaArgs a, int nrb, int n_cu) {
    __shared__ GatedLds<D, GATE> sh;
    const bool lengths = mask_rows_block_causal(a, reinterpret_cast<int*>(&sh));
    if constexpr (GATE == 0) {
        if (lengths)
            prefill_body<MODE_FAST, D, KV, QQ8>(mask_as_lengths(a), 1, nrb, n_cu, sh.fast);
        else
            prefill_body<MODE_MASK, D, KV, QQ8>(a, 0, nrb, n_cu, sh.mask);
    } else {
        if (lengths != (GATE == 1)) return;
        if constexpr (GATE == 1)
            prefill_body<MODE_FAST, D, KV, QQ8>(mask_as_lengths(a), 1, nrb, n_cu, sh);
        else
            prefill_body<MODE_MASK, D, KV, QQ8>(a, 0, nrb, n_cu, sh);
    }
}

template <int MODE, int D, int KV>
void launch_prefill_mode(const FaArgs& a, int causal, int nrb, hipStream_t stream) {
    const dim3 grid((unsigned)((int64_t)a.S * a.H * nrb)), block(kThreads);
    if constexpr (KV == SIXI_TYPE_Q8_0)
        hipLaunchKernelGGL((prefill_q8<MODE, D>), grid, block, 0, stream, a, causal, nrb, a.P);
    else if (a.q_q8)
        hipLaunchKernelGGL((prefill_f16_qq8<MODE, D>), grid, block, 0, stream, a, causal, nrb, a.P);
    else
        hipLaunchKernelGGL((prefill_f16<MODE, D>), grid, block, 0, stream, a, causal, nrb, a.P);
}

template <int D, int KV, bool QQ8>
void launch_gated(const FaArgs& a, int nrb, hipStream_t stream) {
    const dim3 grid((unsigned)((int64_t)a.S * a.H * nrb)), block(kThreads);
    if constexpr (PfDim<D>::GROUPS == 1) {
        hipLaunchKernelGGL((prefill_gated<D, KV, QQ8, 0>), grid, block, 0, stream, a, nrb, a.P);
    } else {
        hipLaunchKernelGGL((prefill_gated<D, KV, QQ8, 1>), grid, block, 0, stream, a, nrb, a.P);
        hipLaunchKernelGGL((prefill_gated<D, KV, QQ8, 2>), grid, block, 0, stream, a, nrb, a.P);
    }
}

template <int D, int KV>
void launch_prefill_gated(const FaArgs& a, int nrb, hipStream_t stream) {
    if constexpr (KV == SIXI_TYPE_Q8_0)
        launch_gated<D, SIXI_TYPE_Q8_0, true>(a, nrb, stream);
    else if (a.q_q8)
        launch_gated<D, SIXI_TYPE_F16, true>(a, nrb, stream);
    else
        launch_gated<D, SIXI_TYPE_F16, false>(a, nrb, stream);
}

}  // namespace

template <int D, int KV>
hipError_t launch_prefill_d(const FaArgs& a, int mask_mode, hipStream_t stream) {
    const bool generic = mask_mode == SIXI_MASK_EXPLICIT || a.softcap != 0.0f;
    const int causal = mask_mode == SIXI_MASK_BLOCK_CAUSAL;
    const int nrb = (a.n_q + kBM - 1) / kBM;
    // an explicit mask alone, with 16-byte aligned rows that one 32-bit range covers: LDS-staged
    const bool mask_only = mask_mode == SIXI_MASK_EXPLICIT && a.mask && a.softcap == 0.0f && a.alibi_nlog2 == 0 &&
                           reinterpret_cast<uintptr_t>(a.mask) % 16 == 0 && a.m_nb1 % 16 == 0 &&
                           (a.m_ne3 == 1 || a.m_nb3 % 16 == 0) && a.m_span < (int64_t)UINT32_MAX;
    if (mask_only && a.row_kl)
        launch_prefill_gated<D, KV>(a, nrb, stream);
    else if (mask_only)
        launch_prefill_mode<MODE_MASK, D, KV>(a, causal, nrb, stream);
    else if (generic)
        launch_prefill_mode<MODE_GENERIC, D, KV>(a, causal, nrb, stream);
    else
        launch_prefill_mode<MODE_FAST, D, KV>(a, causal, nrb, stream);
    return hipGetLastError();
}

hipError_t launch_prefill(const FaArgs& a, int kv_type, int mask_mode, int head_dim, hipStream_t stream) {
    if (kv_type == SIXI_TYPE_Q8_0)
        return head_dim == 128   ? launch_prefill_d<128, SIXI_TYPE_Q8_0>(a, mask_mode, stream)
               : head_dim == 256 ? launch_prefill_d<256, SIXI_TYPE_Q8_0>(a, mask_mode, stream)
                                 : hipErrorNotSupported;
    if (kv_type != SIXI_TYPE_F16) return hipErrorNotSupported;
    if (head_dim == 128) return launch_prefill_d<128, SIXI_TYPE_F16>(a, mask_mode, stream);
    if (head_dim == 256) return launch_prefill_d<256, SIXI_TYPE_F16>(a, mask_mode, stream);
    return hipErrorNotSupported;
}

}  // namespace sixi
