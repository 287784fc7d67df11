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

// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes return 0, so the
// tail of a stream needs no clamping and can never fault.  Word 3 = 0x00020000 is the
// gfx9-family raw-buffer format.
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
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

// 16 bytes per lane from buffer offset `voff` straight into LDS at `lds_addr` + 16*lane
// (gfx950 buffer_load_dwordx4 ... lds).  Issued from asm so that the compiler does not
// drain every LDS-DMA load before each LDS read; the caller waits with wait_vmcnt<N>.
// m0 is saved and restored; the s_nop covers the m0-write -> LDS-DMA hazard.
__device__ __forceinline__ void dma16_to_lds(buf_rsrc rsrc, uint32_t voff, uint32_t lds_addr) {
    int saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(rsrc)
        : "memory");
}
// 4 bytes per lane from buffer offset `voff` into LDS at `lds_addr` + 4*lane
// (buffer_load_dword ... lds); used for rows whose alignment is only 4 bytes (q8_0).
__device__ __forceinline__ void dma4_to_lds(buf_rsrc rsrc, uint32_t voff, uint32_t lds_addr) {
    int saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(rsrc)
        : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

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

// Reductions over the four lanes l, l^16, l^32, l^48 (the lane groups of one MFMA column)
// with the gfx950 row-swap permutes (VALU only, no LDS round trip).  Each swap returns both
// halves, so max/sum of the pair is the reduction over {l, l^32} (resp. {l, l^16}).
__device__ __forceinline__ float max4_rowgroups(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
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

__device__ __forceinline__ StreamDims stream_dims(const FaArgs& a, int s) {
    StreamDims d;
    d.ql = a.q_len ? min(max(a.q_len[s], 0), a.n_q) : a.n_q;
    if (a.kv_len) {
        d.kl = min(max(a.kv_len[s], 0), a.n_kv - d.ql);
        d.nc = d.ql > 0 ? d.kl + d.ql : 0;
    } else {
        d.kl = a.n_kv - d.ql;
        d.nc = d.ql > 0 ? a.n_kv : 0;
    }
    return d;
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

// The f16 bits at an even byte offset `a` of a dword array.
__device__ __forceinline__ uint16_t ld_half_at(const uint32_t* base, int a) {
    const uint32_t w = base[a >> 2];
    return (uint16_t)((a & 2) ? (w >> 16) : (w & 0xffffu));
}

}  // namespace sixi
