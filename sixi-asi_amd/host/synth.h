// synth.h -- seeded synthetic inputs for the attention path (benchmarks and tests).
// Not part of the attention ABI; built into lib/libsixi_synth.so.
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// PCG sequence ids: (tensor << 32) | stream for Q/K/V, a fixed id for the length draw.
#define kSynthTensorQ 1ull
#define kSynthTensorK 2ull
#define kSynthTensorV 3ull
#define kSynthSeqLengths 4ull

void sixi_synth_normal_f32(uint64_t seed, uint64_t seq, float mul, float* out, int64_t n);
void sixi_synth_f32_to_f16(const float* x, uint16_t* y, int64_t n);
void sixi_synth_f16_to_f32(const uint16_t* x, float* y, int64_t n);
int sixi_synth_quantize_q8_0(const float* x, void* dst, int64_t n);
// out[s] = lo + pcg32() % span
void sixi_synth_lengths(uint64_t seed, int64_t S, int32_t lo, int32_t span, int32_t* out);
// Q [S][n_q][H][D] contiguous, f32 (type 0) or f16 (type 1).
int sixi_synth_q(uint64_t seed, int32_t type, float mul, void* dst, int64_t S, int64_t n_q, int64_t H,
                 int64_t D, int n_threads);
// KV cells [0, n_cells[s]) of every stream at dst + s*nb3 + cell*nb1 + head*nb2, f16 (1) or q8_0 (8).
int sixi_synth_kv(uint64_t seed, uint64_t tensor_id, int32_t type, float mul, void* dst, int64_t S,
                  int64_t Hkv, int64_t D, const int32_t* n_cells, int64_t nb1, int64_t nb2, int64_t nb3,
                  int n_threads);

#ifdef __cplusplus
}
#endif
