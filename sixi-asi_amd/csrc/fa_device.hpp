// fa_device.hpp -- device helpers shared by the gfx950 attention kernels.
#pragma once

#include "fa_internal.hpp"

namespace sixi {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }

// 2^x with the hardware v_exp_f32 (2^-inf = 0).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(f16x8 v) { return __builtin_bit_cast(u32x4, v); }

// D = A(16x32) * B(32x16) + C on f16 inputs, f32 accumulate.  Lane l supplies row l%16
// of A (resp. column l%16 of B) at k = 8*(l/16) .. +7, and receives D[4*(l/16)+i][l%16].
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// D = A(16x16) * B(16x16) + C on f16 inputs, f32 accumulate.  Lane l supplies row l%16
// of A (resp. column l%16 of B) at k = 4*(l/16) .. +3, and receives D[4*(l/16)+i][l%16].
__device__ __forceinline__ f32x4 mfma16x16x16(f16x4 a, f16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Accumulators carried across a step loop that also has a rare rescale (a VALU use of them).
// With the builtin MFMA the register allocator either keeps a VGPR copy of every accumulator
// and re-reads it each step, or splits the loop-carried value from the MFMA result and copies
// it back each step.  These asm forms pin the accumulator in place in AGPRs (D = C).
//
// Inline asm is outside the hazard recognizer, so the wait states are explicit:
//  - acc_mfma8 opens with more than the 2 that an MFMA read of a VGPR or AGPR just written by a
//    VALU instruction needs (P converted to f16, V^T masked, a rescaled accumulator);
//  - acc_settle8 stands between the last asm MFMA on a tile and any other read of it: more
//    than the 11 an 8-pass MFMA result needs before a VALU or accvgpr read.  Being an asm
//    statement on the tiles themselves, nothing that reads them can be scheduled before it.
// o[t0 + t][n] += a[t] * b (v_mfma_f32_16x16x32_f16), t < 8: eight output tiles of row tile n.
template <int DT, int NT>
__device__ __forceinline__ void acc_mfma8(f32x4 (&o)[DT][NT], int n, int t0, const u32x4 (&a)[8], f16x8 b) {
    asm("s_nop 2\n\t"
        "v_mfma_f32_16x16x32_f16 %0, %8, %16, %0\n\t"
        "v_mfma_f32_16x16x32_f16 %1, %9, %16, %1\n\t"
        "v_mfma_f32_16x16x32_f16 %2, %10, %16, %2\n\t"
        "v_mfma_f32_16x16x32_f16 %3, %11, %16, %3\n\t"
        "v_mfma_f32_16x16x32_f16 %4, %12, %16, %4\n\t"
        "v_mfma_f32_16x16x32_f16 %5, %13, %16, %5\n\t"
        "v_mfma_f32_16x16x32_f16 %6, %14, %16, %6\n\t"
        "v_mfma_f32_16x16x32_f16 %7, %15, %16, %7"
        : "+a"(o[t0][n]), "+a"(o[t0 + 1][n]), "+a"(o[t0 + 2][n]), "+a"(o[t0 + 3][n]), "+a"(o[t0 + 4][n]),
          "+a"(o[t0 + 5][n]), "+a"(o[t0 + 6][n]), "+a"(o[t0 + 7][n])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]), "v"(b));
}
// Wait states after the asm MFMAs on the accumulator tiles o[t0 .. t0+7][n], before anything
// else reads them.
template <int DT, int NT>
__device__ __forceinline__ void acc_settle8(f32x4 (&o)[DT][NT], int n, int t0) {
    asm volatile("s_nop 7\n\ts_nop 7"
                 : "+a"(o[t0][n]), "+a"(o[t0 + 1][n]), "+a"(o[t0 + 2][n]), "+a"(o[t0 + 3][n]), "+a"(o[t0 + 4][n]),
                   "+a"(o[t0 + 5][n]), "+a"(o[t0 + 6][n]), "+a"(o[t0 + 7][n]));
}
// All tiles of an accumulator set.
template <int DT, int NT>
__device__ __forceinline__ void acc_settle(f32x4 (&o)[DT][NT]) {
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int t0 = 0; t0 < DT; t0 += 8) acc_settle8(o, n, t0);
}

// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes return 0, so the
// tail of a stream needs no clamping and can never fault.  Word 3 = 0x00020000 is the
// gfx9-family raw-buffer format.
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// The same for a base and size that are uniform but that the compiler cannot prove so
// (the inline-asm LDS-DMA loads need the resource in SGPRs).
__device__ __forceinline__ buf_rsrc make_rsrc_uniform(const void* base, uint32_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
    return make_rsrc(reinterpret_cast<const void*>((hi << 32) | lo), (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes));
}
__device__ __forceinline__ u32x4 buf_ld16(buf_rsrc r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ u32x2 buf_ld8(buf_rsrc r, uint32_t off) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_ld4(buf_rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// Batches of direct global->LDS loads (gfx950 buffer_load_dword{,x4} ... lds).  Load u of a
// batch reads buffer offset v[u] into LDS at lds + stride*u + (bytes per lane)*lane.  They are
// issued from asm so that the compiler does not drain every LDS-DMA load before each LDS
// read; the caller waits with wait_vmcnt<N>.  One asm block per batch, so nothing is
// scheduled between its loads: the block opens with the five wait states a VMEM read of an
// SGPR written by a VALU instruction needs (v_readfirstlane, SGPR-spill restores: the
// compiler does not see the resource read inside the asm), and the s_nop after each M0
// write covers the M0 -> LDS-DMA hazard.  M0 is restored at the end.
// NT sets the loads' non-temporal policy (nt): for K/V rows that no other work-group reads,
// i.e. f16 head rows (256 or 512 bytes, whole cache lines) streamed once by the decode
// kernels, so that they leave L2 first and the lines the kernel does reuse stay.  Not for
// q8_0 rows (136-byte head rows share lines with the neighbouring head's work-group) nor for
// the prefill tiles (every row block of a head reads them).
#define SIXI_DMA16X4_ASM(POL) \
    "s_nop 4\n\t" \
    "s_mov_b32 %0, m0\n\t" \
    "s_mov_b32 m0, %1\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %2, %6, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %3, %6, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %4, %6, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %5, %6, 0 offen " POL "lds\n\t" \
    "s_mov_b32 m0, %0"
template <bool NT = false>
__device__ __forceinline__ void dma16x4_to_lds(buf_rsrc rs, const uint32_t (&v)[4], uint32_t lds) {
    int saved;
    if constexpr (NT)
        asm volatile(SIXI_DMA16X4_ASM("nt ")
                     : "=&s"(saved)
                     : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "s"(rs)
                     : "memory", "scc");
    else
        asm volatile(SIXI_DMA16X4_ASM("")
                     : "=&s"(saved)
                     : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "s"(rs)
                     : "memory", "scc");
}
#define SIXI_DMA16X8_ASM(POL) \
    "s_nop 4\n\t" \
    "s_mov_b32 %0, m0\n\t" \
    "s_mov_b32 m0, %1\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %2, %10, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %3, %10, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %4, %10, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %5, %10, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %6, %10, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %7, %10, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %8, %10, 0 offen " POL "lds\n\t" \
    "s_add_u32 m0, m0, 1024\n\t" \
    "s_nop 0\n\t" \
    "buffer_load_dwordx4 %9, %10, 0 offen " POL "lds\n\t" \
    "s_mov_b32 m0, %0"
template <bool NT = false>
__device__ __forceinline__ void dma16x8_to_lds(buf_rsrc rs, const uint32_t (&v)[8], uint32_t lds) {
    int saved;
    if constexpr (NT)
        asm volatile(SIXI_DMA16X8_ASM("nt ")
                     : "=&s"(saved)
                     : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]),
                       "v"(v[5]), "v"(v[6]), "v"(v[7]), "s"(rs)
                     : "memory", "scc");
    else
        asm volatile(SIXI_DMA16X8_ASM("")
                     : "=&s"(saved)
                     : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]),
                       "v"(v[5]), "v"(v[6]), "v"(v[7]), "s"(rs)
                     : "memory", "scc");
}
// Five 16-byte-per-lane loads (5 KB): 16 q8_0 rows of 256 dims (17 x 256 B) and a spare tail.
__device__ __forceinline__ void dma16x5_to_lds(buf_rsrc rs, const uint32_t (&v)[5], uint32_t lds) {
    int saved;
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %7, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 1024\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %3, %7, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 1024\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %4, %7, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 1024\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %5, %7, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 1024\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %6, %7, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "s"(rs)
        : "memory", "scc");
}
// One 16-byte-per-lane load (1 KB).
__device__ __forceinline__ void dma16x1_to_lds(buf_rsrc rs, uint32_t v, uint32_t lds) {
    int saved;
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v), "s"(rs)
        : "memory", "scc");
}
// 4 bytes per lane, LDS stride 256: q8_0 rows, whose alignment is only 4 bytes.
__device__ __forceinline__ void dma4x9_to_lds(buf_rsrc rs, const uint32_t (&v)[9], uint32_t lds) {
    int saved;
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %2, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %3, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %4, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %5, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %6, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %7, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %8, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %9, %11, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %10, %11, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]), "v"(v[8]), "s"(rs)
        : "memory", "scc");
}
// The same with eight loads (a 32-cell step of q8_0 rows takes 17: eight, then nine).
__device__ __forceinline__ void dma4x8_to_lds(buf_rsrc rs, const uint32_t (&v)[8], uint32_t lds) {
    int saved;
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %2, %10, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %3, %10, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %4, %10, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %5, %10, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %6, %10, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %7, %10, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %8, %10, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 256\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %9, %10, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]), "s"(rs)
        : "memory", "scc");
}
// 32 q8_0 rows of 128 dims (34 dwords each) by seventeen 4-byte-per-lane loads.  Loads
// u = 0..15 move dwords 0..31 of rows 2u and 2u + 1 (lane l: row 2u + l/32, dword l%32, offset
// v + u * step with v = (l/32) * stride + 4(l%32) and step = 2 * stride) to LDS lds + 264u +
// 4l; the last moves dwords 32, 33 (lane l: row l/2, dword 32 + l%2, offset vx) to lds + 4224
// + 4l.  So dword c < 32 of row x sits at byte 264(x/2) + 128(x%2) + 4c, dword 32 + e at
// 4224 + 8x + 4e.  The offset steps inside the block, so it costs no registers across it.
__device__ __forceinline__ void dma_q8rows32_to_lds(buf_rsrc rs, uint32_t v, uint32_t vx, uint32_t step,
                                                    uint32_t lds) {
    int saved;
    uint32_t o;
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %6\n\t"
        "v_mov_b32 %1, %2\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "v_add_u32 %1, %4, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 264\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %5, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved), "=&v"(o)
        : "v"(v), "s"(rs), "s"(__builtin_amdgcn_readfirstlane(step)), "v"(vx),
          "s"(__builtin_amdgcn_readfirstlane(lds))
        : "memory", "scc");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt counts at most 63 loads");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most min(later, KMAX) batches of PER loads each are in flight (a ring's own
// loads issued after the one needed; KMAX: the most the ring can have).
template <int PER, int KMAX>
__device__ __forceinline__ void wait_batches(int later) {
    static_assert(PER * KMAX <= 63, "vmcnt counts at most 63 loads");
    if constexpr (KMAX >= 4) {
        if (later >= 4) return wait_vmcnt<4 * PER>();
    }
    if constexpr (KMAX >= 3) {
        if (later >= 3) return wait_vmcnt<3 * PER>();
    }
    if constexpr (KMAX >= 2) {
        if (later >= 2) return wait_vmcnt<2 * PER>();
    }
    if constexpr (KMAX >= 1) {
        if (later >= 1) return wait_vmcnt<PER>();
    }
    wait_vmcnt<0>();
}
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Transposed LDS read (gfx950 ds_read_b64_tr_b16).  Within each group of 16 lanes, lane i
// receives as element e the 16-bit value i%4 of the 8 bytes addressed by lane 4e + i/4 of
// the group; `p` must be 8-byte aligned.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;
__device__ __forceinline__ u32x2 ld_tr16(const lds_char* p) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)const_cast<lds_char*>(p)));
}

// LDS pointer from an LDS byte address.
__device__ __forceinline__ const lds_char* lds_ptr(uint32_t addr) { return (const lds_char*)(size_t)addr; }

// 8-byte LDS load at an LDS byte address (8-byte aligned).
__device__ __forceinline__ u32x2 lds_ld8(uint32_t addr) {
    typedef __attribute__((address_space(3))) const u32x2 lds_u32x2;
    return *(lds_u32x2*)(size_t)addr;
}

// LDS byte address of a __shared__ object.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) T*)p);
}

// Hides a value from the optimizer so LDS reads inside a loop are not hoisted into
// registers (they are re-read every tile on purpose, to keep VGPRs for K/V in flight).
__device__ __forceinline__ int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

// 16-byte global load / store.
__device__ __forceinline__ u32x4 ld16(const char* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(char* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }

// The fused output gate of a call with SIXI_ATTN_FLAG_GATE: the four gate values of dims
// d .. d+3 of head h, row j, stream s (zeros without the gate; load them early, use them with
// gated()).
__device__ __forceinline__ f32x4 gate_load(const FaArgs& a, int s, int j, int h, int d) {
    if (!a.gate) return f32x4{0.f, 0.f, 0.f, 0.f};
    return *reinterpret_cast<const f32x4*>(a.gate + (int64_t)s * a.g_nb3 + (int64_t)j * a.g_nb2 +
                                           (int64_t)h * a.g_nb1 + (int64_t)d * 4);
}
// o * sigmoid(g) per element, in the arithmetic of the separate gate (sixi_attn_gate,
// layer_prologue.hip), so a gated call equals the attention followed by the gate bit for bit;
// o unchanged without the gate.
__device__ __forceinline__ f32x4 gated(const FaArgs& a, f32x4 o, f32x4 g) {
    if (!a.gate) return o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = o[i] * (1.0f / (1.0f + expf(-g[i])));
    return o;
}

// Reductions over the four lanes l, l^16, l^32, l^48 (the lane groups of one MFMA column)
// with the gfx950 row-swap permutes (VALU only, no LDS round trip).  Each swap returns both
// halves, so max/sum of the pair is the reduction over {l, l^32} (resp. {l, l^16}).
// Maxima with IEEE-754 2019 `maximum` semantics (NaN propagates), which gfx950 issues as one
// v_maximum3_f32 with no operand canonicalisation (fmaxf would first canonicalise every
// MFMA result).  These are compiler builtins, not inline asm, so the hazard recognizer adds
// the wait states a read of a fresh MFMA result needs.
__device__ __forceinline__ float max2f(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max3f(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float max4_rowgroups(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = max2f(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max2f(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum4_rowgroups(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Per-stream extents resolved on the device from the length arrays.
struct StreamDims {
    int ql;     // rows of the stream
    int kl;     // cached cells before the block (causal offset)
    int nc;     // cells scanned: kl + ql (0 when the stream has no rows)
};

__device__ __forceinline__ StreamDims stream_dims_from(const FaArgs& a, int q_raw, int kv_raw) {
    StreamDims d;
    d.ql = a.q_len ? min(max(q_raw, 0), a.n_q) : a.n_q;
    if (a.kv_len) {
        d.kl = min(max(kv_raw, 0), a.n_kv - d.ql);
        d.nc = d.ql > 0 ? d.kl + d.ql : 0;
    } else {
        d.kl = a.n_kv - d.ql;
        d.nc = d.ql > 0 ? a.n_kv : 0;
    }
    return d;
}
// Both length loads go through buffer resources that are empty when an array is absent
// (such a load returns 0 and touches no memory), so they issue together, without a branch.
__device__ __forceinline__ StreamDims stream_dims(const FaArgs& a, int s) {
    const buf_rsrc qr = make_rsrc(a.q_len, a.q_len ? (uint32_t)a.S * 4u : 0u);
    const uint32_t ks = (uint32_t)a.kv_len_stride;
    const buf_rsrc kr = make_rsrc(a.kv_len, a.kv_len ? (uint32_t)a.S * 4u * ks : 0u);
    const int q_raw = (int)buf_ld4(qr, (uint32_t)s * 4u);
    const int kv_raw = (int)buf_ld4(kr, (uint32_t)s * 4u * ks);
    return stream_dims_from(a, q_raw, kv_raw);
}

// Explicit masks: whether every row of every stream is a block-causal prefix with one kv offset
// per stream.  With the pre-pass's table (a.row_kl): each active row's entry >= 0 and equal to
// its stream's row 0 (rows past q_len marked idle).  Without it (a.mask_inline: one stream, one
// row, a short row, which every work-group reads itself): the row is +0 or -0 on all of its
// scanned cells [0, nc), i.e. it shows exactly the cells the lengths show.  Called by the whole
// work-group; the threads from t_first on do the reading, eight loads per thread and round, all
// issued before any is used (table entries past the table read 0, as does their row 0, which
// passes), so the waves below t_first can do other work meanwhile (the decode kernels' first
// wave builds the lengths body's cost line).  `wbad` is LDS of one int per wave, free for other
// use again when this returns (it ends with a barrier, which also publishes what the other
// waves wrote to LDS before it).  The result is uniform (an SGPR), so the callers branch on it
// without divergence.
__device__ __forceinline__ bool mask_rows_block_causal(const FaArgs& a, int* wbad, int t_first = 0) {
    constexpr int U = 8;
    const int nt = (int)blockDim.x - t_first;
    bool bad = false;
    if (a.row_kl) {
        const int n = a.S * a.n_q;
        const buf_rsrc r = make_rsrc(a.row_kl, (uint32_t)n * 4u);
        for (int i0 = (int)threadIdx.x - t_first; i0 >= 0 && i0 < n; i0 += U * nt) {
            int v[U], v0[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = i0 + u * nt;
                v[u] = (int)buf_ld4(r, 4u * (uint32_t)i);
                v0[u] = (int)buf_ld4(r, 4u * (uint32_t)(i / a.n_q * a.n_q));
            }
#pragma unroll
            for (int u = 0; u < U; ++u) bad |= !(v[u] == kMaskRowIdle || (v[u] == v0[u] && v[u] >= 0));
        }
    } else {
        // stream 0, row 0: 16-byte pieces of eight cells through a resource over the row's bytes
        // (m_span); a piece that would run past them (the row's last cells) is read cell by cell
        const StreamDims sd = stream_dims(a, 0);
        const buf_rsrc r = make_rsrc(a.mask, (uint32_t)a.m_span);
        const uint16_t* row = reinterpret_cast<const uint16_t*>(a.mask);
        for (int c0 = 8 * ((int)threadIdx.x - t_first); c0 >= 0 && c0 < a.n_kv; c0 += 8 * U * nt) {
            u32x4 w[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 8 * u * nt;
                w[u] = (c < a.n_kv && 2 * (int64_t)c + 16 <= a.m_span) ? buf_ld16(r, 2u * (uint32_t)c)
                                                                         : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 8 * u * nt;
                if (c < sd.nc && 2 * (int64_t)c + 16 > a.m_span) {
                    for (int e = 0; e < 8 && c + e < sd.nc; ++e) bad |= (row[c + e] & 0x7fffu) != 0u;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint32_t bits = (e & 1) ? (w[u][e >> 1] >> 16) : (w[u][e >> 1] & 0xffffu);
                        bad |= c + e < sd.nc && (bits & 0x7fffu) != 0u;
                    }
                }
            }
        }
    }
    const bool wave_bad = __builtin_amdgcn_ballot_w64(bad) != 0;
    if ((threadIdx.x & 63) == 0) wbad[threadIdx.x >> 6] = wave_bad ? 1 : 0;
    __syncthreads();
    int any = 0;
    for (int w = 0; w < (int)blockDim.x / 64; ++w) any |= wbad[w];
    any = __builtin_amdgcn_readfirstlane(any);
    __syncthreads();
    return any == 0;
}
// The arguments of the lengths-only body of a mask whose rows passed that test: each stream's
// cached length is the offset its mask implies (row 0's entry of the table; without the table
// the call's own lengths, which the single row matched), block-causal.
__device__ __forceinline__ FaArgs mask_as_lengths(const FaArgs& a) {
    FaArgs b = a;
    if (a.row_kl) {
        b.kv_len = a.row_kl;
        b.kv_len_stride = a.n_q;
    }
    b.mask = nullptr;
    return b;
}

// Page ids of a paged cache for one stream, 64 consecutive page indices at a time, one per
// lane: a tile's page comes from a register (v_readlane) rather than a load per tile.  Ids
// are clamped to [0, n_pages).  Unused for contiguous caches (pt null).
struct PageIds {
    int first;  // page index that lane 0 holds
    int id;     // lane l: id of page index first + l
};
__device__ __forceinline__ PageIds page_ids_load(const FaArgs& a, int s, int first) {
    PageIds p{__builtin_amdgcn_readfirstlane(first), 0};
    first = p.first;
    if (a.pt) {
        const int64_t idx = (int64_t)first + (threadIdx.x & 63);
        if (idx < a.pt_stride) p.id = min(max(a.pt[(int64_t)s * a.pt_stride + idx], 0), a.n_pages - 1);
    }
    return p;
}
// Id of page index `page` (uniform) of stream s; reloads the window when it moves past it.
__device__ __forceinline__ int page_id(PageIds& p, const FaArgs& a, int s, int page) {
    if (!a.pt) return 0;
    if (page < p.first || page >= p.first + 64) {
        p = page_ids_load(a, s, page);
        // use the load on this (rare) path: a first use after the paths join would put the
        // compiler's wait for it -- which also drains the ring's DMA loads -- on every step
        asm volatile("" ::"v"(p.id));
    }
    return __builtin_amdgcn_readlane(p.id, page - p.first);
}

// K or V rows of (stream s, kv-head g) from cell c0 on, for a range-checked buffer resource:
// the address of cell c0's row, and the bytes from there to the end of the last row a load may
// use -- rows up to cell nc - 1 that lie in c0's page (paged caches, page id `page` of c0's
// page) or in the stream (contiguous).  Offsets from the address are (c - c0) * nb1.  0 bytes
// when c0 >= nc.  Every tile of the kernels lies in one page: tiles of 16, 32 and 64 cells
// start at multiples of their size, and pages hold 256 cells.
struct KvSpan {
    const char* p;
    uint32_t bytes;
};
__device__ __forceinline__ KvSpan kv_span(const FaArgs& a, const char* kv, int64_t nb1, int64_t nb2, int64_t nb3, int s,
                                          int g, int c0, int nc, int64_t rowb, int page) {
    if (c0 >= nc) return {kv, 0u};
    int64_t off;
    int last = nc;
    if (a.pt) {
        off = (int64_t)page * nb3 + (int64_t)(c0 & (kPageCells - 1)) * nb1;
        last = min(nc, (c0 | (kPageCells - 1)) + 1);
    } else {
        off = (int64_t)s * nb3 + (int64_t)c0 * nb1;
    }
    return {kv + off + (int64_t)g * nb2, (uint32_t)((int64_t)(last - 1 - c0) * nb1 + rowb)};
}

// ALiBi slope of q-head h (ggml's rule); 1 when ALiBi is off.
__device__ __forceinline__ float alibi_slope(const FaArgs& a, int h) {
    if (a.alibi_nlog2 == 0) return 1.0f;
    return h < a.alibi_nlog2 ? powf(a.alibi_m0, (float)(h + 1))
                             : powf(a.alibi_m1, (float)(2 * (h - a.alibi_nlog2) + 1));
}

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Eight int8 values (two dwords, little-endian) times the f16 block scale `dbits`, as eight
// f16 (u32x4).  Each byte becomes the f16 1024 + (b ^ 0x80) = 1152 + b through v_perm_b32,
// an exact f16 subtraction recovers b, and one f16 multiply rounds b * d once.
__device__ __forceinline__ u32x4 dequant_q8x8(uint32_t w0, uint32_t w1, uint16_t dbits) {
    const _Float16 d = __builtin_bit_cast(_Float16, dbits);
    const f16x2 dd = {d, d};
    const f16x2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
    u32x4 out;
    out[0] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) - off) * dd);
    out[1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) - off) * dd);
    out[2] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) - off) * dd);
    out[3] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) - off) * dd);
    return out;
}

// The 8 bytes at byte offset `a` of a dword array whose element `a` lies 2 bytes past a
// dword boundary (odd2 = true) or on one.
__device__ __forceinline__ void ld8_at(const uint32_t* base, int a, bool odd2, uint32_t& w0, uint32_t& w1) {
    if (odd2) {
        const int d0 = (a - 2) >> 2;
        const uint32_t x0 = base[d0], x1 = base[d0 + 1], x2 = base[d0 + 2];
        w0 = __builtin_amdgcn_alignbyte(x1, x0, 2);
        w1 = __builtin_amdgcn_alignbyte(x2, x1, 2);
    } else {
        w0 = base[a >> 2];
        w1 = base[(a >> 2) + 1];
    }
}

// The 16 bytes at byte offset `a` (even; its parity over dwords may differ between lanes) of
// a dword array: five dword reads from the dword holding `a`, realigned by a & 3.  Reads up to
// 4 bytes past the 16 when `a` is dword-aligned.
__device__ __forceinline__ void ld16_at_any(const uint32_t* base, int a, uint32_t (&w)[4]) {
    const int d0 = a >> 2;
    const uint32_t sh = (uint32_t)(a & 3);
    uint32_t x[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) x[i] = base[d0 + i];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __builtin_amdgcn_alignbyte(x[i + 1], x[i], sh);
}

// The f16 bits at an even byte offset `a` of a dword array.
__device__ __forceinline__ uint16_t ld_half_at(const uint32_t* base, int a) {
    const uint32_t w = base[a >> 2];
    return (uint16_t)((a & 2) ? (w >> 16) : (w & 0xffffu));
}

// One q8_0 block (34 bytes: f16 scale, 32 int8) at byte offset `a` (even) of a dword array:
// the scale bits and the 32 quants as eight little-endian dwords.
template <bool ODD2>  // a % 4 == 2
__device__ __forceinline__ void ld_q8_block(const uint32_t* base, int a, uint16_t& d, uint32_t (&w)[8]) {
    if constexpr (ODD2) {  // scale in the upper half of a dword, quants dword-aligned
        d = (uint16_t)(base[(a - 2) >> 2] >> 16);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = base[((a + 2) >> 2) + i];
    } else {      // scale in the lower half, quants 2 bytes past each dword boundary
        uint32_t x[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) x[i] = base[(a >> 2) + i];
        d = (uint16_t)(x[0] & 0xffffu);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = __builtin_amdgcn_alignbyte(x[i + 1], x[i], 2);
    }
}

}  // namespace sixi
