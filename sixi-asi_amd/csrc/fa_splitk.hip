// fa_splitk.hip -- split-K flash-decoding for decode and speculative verify (gfx950).
//
// Work decomposition ("stream-K" over KV tiles):
//   A segment is one (stream s, kv-head g); it has nt_s = ceil(cells_s / 32) tiles of 32
//   KV cells, and all G*q_len_s query rows of the group ride along with every tile, so
//   each K/V byte is read from HBM once for the whole GQA group.  Segments are laid end to
//   end (stream-major, then kv-head) and the P work-groups take equal shares
//   [floor(p*T/P), floor((p+1)*T/P)) of the T tiles, so any mix of lengths balances.  The
//   share of work-group p inside segment k is a "piece"; it goes to partial slot k + p,
//   which is unique because pieces are ordered in both k and p.  A segment owned by one
//   work-group is finished in place; the others are combined by splitk_merge_d128.
//
// Inside a work-group of 4 waves, K/V tiles are staged in LDS with direct global->LDS
// 16-byte loads (buffer_load_dwordx4 ... lds), so the bytes in flight cost no VGPRs:
//   RS = 1 (<= 48 rows): the 4 waves take the piece's tiles round-robin, each through a
//          private 2-slot ring (2 tiles = 32 KB in flight per wave, no barriers);
//   RS = 2 (49..96 rows): waves (rg, tl) split the rows in two halves rg and the tiles
//          over two tile lanes tl; the two waves of a lane share a 4-slot ring (3 tiles in
//          flight per lane), each issuing half of every tile, one barrier per tile.
// Per tile a wave computes
//   S^T = K Q^T   on v_mfma_f32_16x16x32_f16: A = 16 cells x 32 dims (lane (r, c) holds
//                 cell 16mt+r, dims 32ks+8c..+7), B = Q^T from LDS;
//   online softmax in the log2 domain, row max across the 4 lane groups;
//   O^T += V^T P^T  with B = P^T taken from the lane's own S^T values (cell order
//                 16*(e/4) + 4c + e%4) and A = V^T built by an in-register 8x8 16-bit
//                 transpose (v_perm_b32) of the eight 16-byte V rows the lane staged: lane
//                 (r, c) stages dims 8r..8r+7 of its 8 cells, so output M-tile t holds
//                 dims 8r + t.
// Every 16-byte chunk is read back by the lane index that staged it.
#include "fa_device.hpp"

namespace sixi {
namespace {

constexpr int kTile = kSplitTile;
constexpr int kWaves = kSplitWaves;
constexpr int kThreads = kWaves * 64;
constexpr int kSlotChunks = 16;  // 8 K chunks + 8 V chunks of 1 KB (64 lanes x 16 B)
constexpr int kRingChunks = 128; // 8 slots of 16 KB: 4 waves x 2 (RS=1) or 2 lanes x 4 (RS=2)

// Inclusive tile prefix over streams into ps[0..S] (run by one wave).
__device__ void build_tile_prefix(const FaArgs& a, int* ps) {
    const int lane = threadIdx.x & 63;
    if (lane == 0) ps[0] = 0;
    int carry = 0;
    for (int base = 0; base < a.S; base += 64) {
        const int s = base + lane;
        int x = 0;
        if (s < a.S) x = (stream_dims(a, s).nc + kTile - 1) / kTile;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (s < a.S) ps[s + 1] = carry + x;
        carry += __shfl(x, 63, 64);
    }
}

template <int NT>
struct MergeLds {
    f32x4 o[2][NT * 8 * 64];  // [slot][n][t][lane]
    float m[2][NT * 64];
    float l[2][NT * 64];
};

template <int NTW, int RS>
struct SplitLds {
    union {
        u32x4 ring[kRingChunks * 64];  // K/V staging, 16 KB slots
        MergeLds<NTW> mg;              // reused after the tile loop
    };
    u32x4 q[NTW * RS * 4 * 64];  // Q^T B-operands: [n][ks][lane] 8 f16 each
    int ps[kMaxStreams + 1];
};

template <int NT>
struct WaveAcc {
    f32x4 o[8][NT];  // O^T tiles: lane (r,c) holds row 16n+r, dims 32c + 8i + t at o[t][n][i]
    float m[NT];     // running row max (log2 domain), equal across the 4 lane groups
    float l[NT];     // this lane's share of the row sum (summed over groups at the end)
};

template <int NT>
__device__ __forceinline__ void acc_to_lds(MergeLds<NT>& mg, int slot, const WaveAcc<NT>& acc,
                                           int lane) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int t = 0; t < 8; ++t) mg.o[slot][(n * 8 + t) * 64 + lane] = acc.o[t][n];
        mg.m[slot][n * 64 + lane] = acc.m[n];
        mg.l[slot][n * 64 + lane] = acc.l[n];
    }
}

template <int NT>
__device__ __forceinline__ void acc_merge_lds(const MergeLds<NT>& mg, int slot, WaveAcc<NT>& acc,
                                              int lane) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const float m2 = mg.m[slot][n * 64 + lane];
        const float l2 = mg.l[slot][n * 64 + lane];
        const float mn = fmaxf(acc.m[n], m2);
        const float ms = (mn == neg_inf()) ? 0.0f : mn;
        const float a1 = fast_exp2(acc.m[n] - ms);
        const float a2 = fast_exp2(m2 - ms);
        acc.l[n] = acc.l[n] * a1 + l2 * a2;
        acc.m[n] = mn;
#pragma unroll
        for (int t = 0; t < 8; ++t)
            acc.o[t][n] = acc.o[t][n] * a1 + mg.o[slot][(n * 8 + t) * 64 + lane] * a2;
    }
}

// One piece: tiles [t_begin, t_end) of segment (s, g).  NTW = 16-row tiles per wave,
// RS = row groups (1 or 2); the group has up to NTW*RS*16 rows.
template <int NTW, int RS, int MASK>
__device__ void splitk_piece(const FaArgs& a, SplitLds<NTW, RS>& sh, int s, int g, int t_begin,
                             int t_end, bool whole, int64_t slot) {
    constexpr int NT = NTW * RS;
    constexpr int TL = kWaves / RS;           // tile lanes
    constexpr int NSLOT = (RS == 1) ? 2 : 4;  // ring slots per wave (RS=1) or lane (RS=2)
    constexpr int DMA = kSlotChunks / RS;     // DMA instructions per tile per wave
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int rg = (RS == 2) ? (w >> 1) : 0;
    const int tl = (RS == 2) ? (w & 1) : w;
    const int r = lane & 15;
    const int c = lane >> 4;
    const StreamDims sd = stream_dims(a, s);
    const int G = a.G;
    const int R = G * sd.ql;

    // ---- Q rows of the group -> f16 B operands in LDS (row 16n+r, dims 32ks+8c..+7) ----
    for (int idx = tid; idx < NT * 16 * 16; idx += kThreads) {
        const int row = idx >> 4;
        const int chunk = idx & 15;  // 8-dim chunk: ks = chunk/4, c = chunk%4
        u32x4 val = {0u, 0u, 0u, 0u};
        if (row < R) {
            const int j = row / G;
            const int h = g * G + row % G;
            const char* src = a.q + (int64_t)j * a.q_nb1 + (int64_t)h * a.q_nb2 +
                              (int64_t)s * a.q_nb3 + (int64_t)chunk * 8 * a.q_es;
            f16x8 hv;
            if (a.q_f16) {
#pragma unroll
                for (int e = 0; e < 8; ++e) hv[e] = reinterpret_cast<const _Float16*>(src)[e];
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) hv[e] = (_Float16)reinterpret_cast<const float*>(src)[e];
            }
            val = as_u32x4(hv);
        }
        const int n = row >> 4, rr = row & 15, ks = chunk >> 2, cc = chunk & 3;
        sh.q[(n * 4 + ks) * 64 + cc * 16 + rr] = val;
    }
    __syncthreads();

    // ---- per-row constants for this lane (its rows are 16*(rg*NTW + n) + r) ----
    int vis[NTW];      // cells visible to the row
    float slope[NTW];  // ALiBi slope (EXPLICIT mode)
    int jrow[NTW];
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        const int row = 16 * (rg * NTW + n) + r;
        const int j = row < R ? row / G : 0;
        jrow[n] = j;
        vis[n] = (MASK == SIXI_MASK_BLOCK_CAUSAL) ? sd.kl + j + 1 : sd.nc;
        slope[n] = (MASK == SIXI_MASK_EXPLICIT) ? alibi_slope(a, g * G + (row % G)) : 1.0f;
    }
    const int vis_min = (MASK == SIXI_MASK_BLOCK_CAUSAL) ? sd.kl + 1 : sd.nc;

    WaveAcc<NTW> acc;
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
        acc.m[n] = neg_inf();
        acc.l[n] = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) acc.o[t][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // K/V of this (stream, kv-head) through range-checked buffer resources: cells >= nc
    // read as zeros and are masked, so the tail tile needs no clamping.
    const int64_t rowb = 128 * 2;
    const i32x4 krs = make_rsrc_sgpr(a.k + (int64_t)s * a.k_nb3 + (int64_t)g * a.k_nb2,
                                     (uint32_t)((int64_t)(sd.nc - 1) * a.k_nb1 + rowb));
    const i32x4 vrs = make_rsrc_sgpr(a.v + (int64_t)s * a.v_nb3 + (int64_t)g * a.v_nb2,
                                     (uint32_t)((int64_t)(sd.nc - 1) * a.v_nb1 + rowb));
    const uint32_t knb = (uint32_t)a.k_nb1, vnb = (uint32_t)a.v_nb1;
    const char* mrow = nullptr;
    if (MASK == SIXI_MASK_EXPLICIT) mrow = a.mask + (int64_t)(s % a.m_ne3) * a.m_nb3;

    // tiles of this lane: t_begin + tl + TL*i, i < n_my; n_iter is the same for the group
    const int n_tiles = t_end - t_begin;
    const int n_iter = (n_tiles + TL - 1) / TL;
    const int t0 = t_begin + tl;
    const int n_my = t0 < t_end ? (t_end - t0 + TL - 1) / TL : 0;
    u32x4* ring = sh.ring + (size_t)tl * NSLOT * kSlotChunks * 64;
    const uint32_t ring_base = lds_addr(ring);

    // Stage tile i of this lane into slot i % NSLOT.  RS = 1: all 16 chunks; RS = 2: row
    // group 0 stages the 8 K chunks and row group 1 the 8 V chunks.
    auto issue = [&](int i) {
        const uint32_t c0 = (uint32_t)(t0 + i * TL) * kTile;
        const uint32_t base = ring_base + (uint32_t)(i % NSLOT) * (kSlotChunks * 1024);
        if (RS == 1 || rg == 0) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const uint32_t off = (c0 + 16 * mt + r) * knb + c * 16;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    dma16_to_lds(krs, off + ks * 64, base + (mt * 4 + ks) * 1024);
            }
        }
        if (RS == 1 || rg == 1) {
            const uint32_t vo = (c0 + 4 * c) * vnb + r * 16;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                dma16_to_lds(vrs, vo + (16 * (e >> 2) + (e & 3)) * vnb, base + (8 + e) * 1024);
        }
    };

    // One tile from a staged slot; `after_reads` runs once the slot has been read.
    auto compute = [&](int i, auto&& after_reads) {
        const u32x4* slot_p = ring + (i % NSLOT) * (kSlotChunks * 64);
        const int c0 = (t0 + i * TL) * kTile;
        const int ql = opaque(lane);

        // S^T = K Q^T
        f32x4 st[2][NTW];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            f16x8 kop[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) kop[ks] = as_f16x8(slot_p[(mt * 4 + ks) * 64 + ql]);
#pragma unroll
            for (int n = 0; n < NTW; ++n) {
                f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    x = mfma16x16x32(kop[ks], as_f16x8(sh.q[((rg * NTW + n) * 4 + ks) * 64 + ql]), x);
                st[mt][n] = x;
            }
        }
        u32x4 vr[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vr[e] = slot_p[(8 + e) * 64 + ql];
        after_reads();

        if (c0 + kTile > sd.nc) {
            // tail tile: cells past the stream read as zero or stale; make V exactly zero
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (c0 + 16 * (e >> 2) + 4 * c + (e & 3) >= sd.nc) vr[e] = u32x4{0u, 0u, 0u, 0u};
        }

        const bool need_mask = (MASK == SIXI_MASK_EXPLICIT) || (c0 + kTile > vis_min);
        f16x8 pf[NTW];
        bool rescale = false;
        float alpha[NTW];
#pragma unroll
        for (int n = 0; n < NTW; ++n) {
            float sv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float x = st[e >> 2][n][e & 3];
                if (a.softcap != 0.0f) x = a.softcap * tanhf(x * a.scale) * kLog2e;
                else x *= a.scale_log2;
                sv[e] = x;
            }
            if (need_mask) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int cell = c0 + 16 * (e >> 2) + 4 * c + (e & 3);
                    if (MASK == SIXI_MASK_EXPLICIT) {
                        float mv = neg_inf();
                        if (cell < sd.nc) {
                            const uint16_t bits = *reinterpret_cast<const uint16_t*>(
                                mrow + (int64_t)jrow[n] * a.m_nb1 + (int64_t)cell * 2);
                            mv = slope[n] * half_bits_to_float(bits);
                        }
                        sv[e] = (mv == neg_inf()) ? neg_inf() : sv[e] + mv * kLog2e;
                    } else if (cell >= vis[n]) {
                        sv[e] = neg_inf();
                    }
                }
            }
            float mx = sv[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
            mx = max4_rowgroups(mx);
            const float mnew = fmaxf(acc.m[n], mx);
            const float ms = (mnew == neg_inf()) ? 0.0f : mnew;
            alpha[n] = fast_exp2(acc.m[n] - ms);
            rescale |= (alpha[n] != 1.0f);
            float psum = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pv = fast_exp2(sv[e] - ms);
                psum += pv;
                pf[n][e] = (_Float16)pv;
            }
            acc.l[n] = acc.l[n] * alpha[n] + psum;
            acc.m[n] = mnew;
        }
        if (__any(rescale)) {
#pragma unroll
            for (int n = 0; n < NTW; ++n)
#pragma unroll
                for (int tt = 0; tt < 8; ++tt) acc.o[tt][n] *= alpha[n];
        }

        // EXPLICIT mode: a cell that none of this wave's rows sees may hold NaN; zero its
        // V row (other waves make their own decision for their rows).
        if (MASK == SIXI_MASK_EXPLICIT) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                bool seen = false;
#pragma unroll
                for (int n = 0; n < NTW; ++n) seen |= ((float)pf[n][e] != 0.0f);
                const uint64_t b = __ballot(seen);
                if (((b >> (16 * c)) & 0xffffull) == 0) vr[e] = u32x4{0u, 0u, 0u, 0u};
            }
        }

        // O^T += V^T P^T
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) {
            const int d2 = tt >> 1;
            const uint32_t sel = (tt & 1) ? 0x07060302u : 0x05040100u;
            u32x4 vt;
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2)
                vt[e2] = __builtin_amdgcn_perm(vr[2 * e2 + 1][d2], vr[2 * e2][d2], sel);
#pragma unroll
            for (int n = 0; n < NTW; ++n) acc.o[tt][n] = mfma16x16x32(as_f16x8(vt), pf[n], acc.o[tt][n]);
        }
    };

    if constexpr (RS == 1) {
        // private ring: refill the slot just read with tile i+2
        if (n_my > 0) issue(0);
        if (n_my > 1) issue(1);
        for (int i = 0; i < n_my; ++i) {
            if (i + 1 < n_my) wait_vmcnt<DMA>();
            else wait_vmcnt<0>();
            compute(i, [&] {
                wait_lgkmcnt0();
                if (i + 2 < n_my) issue(i + 2);
            });
        }
    } else {
        // shared ring: tile i+3 goes into the slot of tile i-1, which every reader left
        // before the barrier of iteration i
#pragma unroll
        for (int i = 0; i < NSLOT - 1; ++i)
            if (i < n_my) issue(i);
        for (int i = 0; i < n_iter; ++i) {
            const int ahead = n_my - 1 - i;  // own tiles issued after tile i, capped at 2
            if (ahead >= 2) wait_vmcnt<2 * DMA>();
            else if (ahead == 1) wait_vmcnt<DMA>();
            else wait_vmcnt<0>();
            __syncthreads();
            if (i + NSLOT - 1 < n_my) issue(i + NSLOT - 1);
            if (i < n_my) compute(i, [] {});
        }
    }
    // rows' sums over the 4 lane groups
#pragma unroll
    for (int n = 0; n < NTW; ++n) acc.l[n] = sum4_rowgroups(acc.l[n]);

    // ---- combine the waves that share rows (LDS reused from the rings) ----
    __syncthreads();
    bool owner;
    if constexpr (RS == 1) {
        // (2,3) -> (0,1), then 1 -> 0
        if (w >= 2) acc_to_lds(sh.mg, w - 2, acc, lane);
        __syncthreads();
        if (w < 2) acc_merge_lds(sh.mg, w, acc, lane);
        __syncthreads();
        if (w == 1) acc_to_lds(sh.mg, 0, acc, lane);
        __syncthreads();
        if (w == 0) acc_merge_lds(sh.mg, 0, acc, lane);
        owner = (w == 0);
    } else {
        // lane 1 -> lane 0 within each row group
        if (tl == 1) acc_to_lds(sh.mg, rg, acc, lane);
        __syncthreads();
        if (tl == 0) acc_merge_lds(sh.mg, rg, acc, lane);
        owner = (tl == 0);
    }
    if (owner) {
        // ---- write: final rows, or the piece's partial (m, l, unnormalised O) ----
#pragma unroll
        for (int n = 0; n < NTW; ++n) {
            const int row = 16 * (rg * NTW + n) + r;
            if (row >= R) continue;
            if (whole) {
                const int j = row / G;
                const int h = g * G + row % G;
                const float inv = acc.l[n] == 0.0f ? 0.0f : 1.0f / acc.l[n];
                char* dst = a.out + (int64_t)j * a.o_nb2 + (int64_t)h * a.o_nb1 +
                            (int64_t)s * a.o_nb3 + c * 32 * 4;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    st16(dst + i * 32, f32x4{acc.o[0][n][i], acc.o[1][n][i], acc.o[2][n][i], acc.o[3][n][i]} * inv);
                    st16(dst + i * 32 + 16, f32x4{acc.o[4][n][i], acc.o[5][n][i], acc.o[6][n][i], acc.o[7][n][i]} * inv);
                }
            } else {
                float* base = a.part + slot * a.slot_floats;
                char* dst = reinterpret_cast<char*>(base + (int64_t)row * 128 + c * 32);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    st16(dst + i * 32, f32x4{acc.o[0][n][i], acc.o[1][n][i], acc.o[2][n][i], acc.o[3][n][i]});
                    st16(dst + i * 32 + 16, f32x4{acc.o[4][n][i], acc.o[5][n][i], acc.o[6][n][i], acc.o[7][n][i]});
                }
                if (c == 0) {
                    base[(int64_t)a.rows_max * 128 + row] = acc.m[n];
                    base[(int64_t)a.rows_max * 128 + a.rows_max + row] = acc.l[n];
                }
            }
        }
    }
    __syncthreads();  // LDS (q, merge slots, rings) is reused by the next piece
}

template <int NTW, int RS, int MASK>
__global__ __launch_bounds__(kThreads, 1) void splitk_f16_d128(FaArgs a) {
    __shared__ SplitLds<NTW, RS> sh;
    const int tid = threadIdx.x;
    if (tid < 64) build_tile_prefix(a, sh.ps);
    __syncthreads();
    const int S = a.S;
    const int64_t Hkv = a.Hkv;
    const int64_t T = Hkv * sh.ps[S];
    if (blockIdx.x == 0)
        for (int i = tid; i <= S; i += kThreads) a.meta[i] = sh.ps[i];
    const int64_t P = a.P;
    const int64_t p = blockIdx.x;
    const int64_t x0 = p * T / P;
    const int64_t x1 = (p + 1) * T / P;
    if (x0 >= x1) return;

    // stream holding tile x0: the largest s with Hkv*ps[s] <= x0
    int lo = 0, hi = S;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (Hkv * sh.ps[mid] <= x0) lo = mid; else hi = mid - 1;
    }
    int s = lo;
    int64_t x = x0;
    while (x < x1) {
        while (Hkv * sh.ps[s + 1] <= x) ++s;
        const int nt = sh.ps[s + 1] - sh.ps[s];
        const int64_t cs = Hkv * sh.ps[s];
        const int g = (int)((x - cs) / nt);
        const int64_t ck = cs + (int64_t)g * nt;
        const int tb = (int)(x - ck);
        const int te = (int)(min(x1, ck + nt) - ck);
        const int64_t k = (int64_t)s * Hkv + g;
        splitk_piece<NTW, RS, MASK>(a, sh, s, g, tb, te, tb == 0 && te == nt, k + p);
        x = ck + te;
    }
}

// Combines the pieces of every segment that more than one work-group touched.
// grid = (S*Hkv segments, rows_max/16); 256 threads = 16 rows x 16 chunks of 8 dims.
__global__ __launch_bounds__(256) void splitk_merge_d128(FaArgs a) {
    const int64_t k = blockIdx.x;
    const int s = (int)(k / a.Hkv);
    const int g = (int)(k % a.Hkv);
    const int32_t* ps = a.meta;
    const int nt = ps[s + 1] - ps[s];
    if (nt == 0) return;
    const int64_t T = (int64_t)a.Hkv * ps[a.S];
    const int64_t P = a.P;
    const int64_t ck = (int64_t)a.Hkv * ps[s] + (int64_t)g * nt;
    const int64_t p_first = ((ck + 1) * P - 1) / T;
    const int64_t p_last = ((ck + nt) * P - 1) / T;
    if (p_first == p_last) return;  // finished in place by its only work-group

    const StreamDims sd = stream_dims(a, s);
    const int row = blockIdx.y * 16 + (threadIdx.x >> 4);
    const int d0 = (threadIdx.x & 15) * 8;
    if (row >= a.G * sd.ql) return;

    const int64_t moff = (int64_t)a.rows_max * 128 + row;
    const int64_t loff = moff + a.rows_max;
    float M = neg_inf();
    for (int64_t p = p_first; p <= p_last; ++p) {
        if (p * T / P == (p + 1) * T / P) continue;  // empty work-group
        M = fmaxf(M, a.part[(k + p) * a.slot_floats + moff]);
    }
    const float Ms = (M == neg_inf()) ? 0.0f : M;
    float L = 0.0f;
    f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
    for (int64_t p = p_first; p <= p_last; ++p) {
        if (p * T / P == (p + 1) * T / P) continue;
        const float* base = a.part + (k + p) * a.slot_floats;
        const float wgt = fast_exp2(base[moff] - Ms);
        L += base[loff] * wgt;
        const f32x4* src = reinterpret_cast<const f32x4*>(base + (int64_t)row * 128 + d0);
        o0 += src[0] * wgt;
        o1 += src[1] * wgt;
    }
    const float inv = L == 0.0f ? 0.0f : 1.0f / L;
    const int j = row / a.G;
    const int h = g * a.G + row % a.G;
    char* dst = a.out + (int64_t)j * a.o_nb2 + (int64_t)h * a.o_nb1 + (int64_t)s * a.o_nb3 + d0 * 4;
    st16(dst, o0 * inv);
    st16(dst + 16, o1 * inv);
}

template <int NTW, int RS>
hipError_t launch_nt(const FaArgs& a, int mask_mode, hipStream_t stream) {
    const dim3 grid(a.P), block(kThreads);
    switch (mask_mode) {
        case SIXI_MASK_NONE:
            hipLaunchKernelGGL((splitk_f16_d128<NTW, RS, SIXI_MASK_NONE>), grid, block, 0, stream, a); break;
        case SIXI_MASK_BLOCK_CAUSAL:
            hipLaunchKernelGGL((splitk_f16_d128<NTW, RS, SIXI_MASK_BLOCK_CAUSAL>), grid, block, 0, stream, a); break;
        default:
            hipLaunchKernelGGL((splitk_f16_d128<NTW, RS, SIXI_MASK_EXPLICIT>), grid, block, 0, stream, a); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 mgrid((unsigned)(a.S * a.Hkv), (unsigned)(a.rows_max / 16));
    hipLaunchKernelGGL(splitk_merge_d128, mgrid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

int splitk_num_groups(const FaArgs& a, int cu_count) {
    const int64_t tiles_max = (int64_t)a.S * a.Hkv * ((a.n_kv + kTile - 1) / kTile);
    int64_t P = cu_count > 0 ? cu_count : 256;
    if (P > kMaxSplitGroups) P = kMaxSplitGroups;
    if (P > tiles_max) P = tiles_max;
    return (int)(P < 1 ? 1 : P);
}

hipError_t launch_splitk(const FaArgs& a, int kv_type, int mask_mode, int head_dim,
                         hipStream_t stream) {
    if (kv_type != SIXI_TYPE_F16 || head_dim != 128) return hipErrorNotSupported;
    const int nt = a.rows_max / 16;
    switch (nt) {
        case 1: return launch_nt<1, 1>(a, mask_mode, stream);
        case 2: return launch_nt<2, 1>(a, mask_mode, stream);
        case 3: return launch_nt<3, 1>(a, mask_mode, stream);
        case 4: return launch_nt<2, 2>(a, mask_mode, stream);
        case 5: case 6: return launch_nt<3, 2>(a, mask_mode, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace sixi
