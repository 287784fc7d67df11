// synth.cpp -- seeded synthetic inputs for the attention path (benchmarks and tests).
//
// Generator: PCG32 XSH-RR (the reference's DeterministicRng, src/core/core_execution.cpp:33-62)
// with 53-bit uniforms and Box-Muller normals in float64; one PCG sequence per (tensor,
// stream) so streams can be filled in parallel.  KV elements are stored as f16
// (round-to-nearest-even via F16C) or as q8_0 blocks (include/sixi_asi/numeric.hpp:32-38,
// quantised with the rule of src/core/numeric.cpp:349-384).
#include "synth.h"

#include <immintrin.h>

#include <cmath>
#include <cstring>
#include <vector>

namespace {

struct Pcg32 {
    uint64_t state = 0, inc = 1;
    uint32_t next() {
        const uint64_t old = state;
        state = old * 6364136223846793005ULL + inc;
        const uint32_t x = static_cast<uint32_t>(((old >> 18u) ^ old) >> 27u);
        const uint32_t rot = static_cast<uint32_t>(old >> 59u);
        return (x >> rot) | (x << ((0u - rot) & 31u));
    }
    Pcg32(uint64_t seed, uint64_t seq) {
        inc = (seq << 1u) | 1u;
        next();
        state += seed;
        next();
    }
    double uniform() {
        const uint64_t hi = next(), lo = next();
        return static_cast<double>(((hi << 32) | lo) >> 11) * (1.0 / 9007199254740992.0);
    }
};

// Normals in pairs: z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), r = sqrt(-2 ln u1).
class NormalStream {
public:
    NormalStream(uint64_t seed, uint64_t seq) : rng_(seed, seq) {}
    double next() {
        if (have_) {
            have_ = false;
            return spare_;
        }
        double u1 = rng_.uniform();
        const double u2 = rng_.uniform();
        if (u1 < 1e-300) u1 = 1e-300;
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double t = 6.283185307179586476925286766559 * u2;
        spare_ = r * std::sin(t);
        have_ = true;
        return r * std::cos(t);
    }

private:
    Pcg32 rng_;
    double spare_ = 0.0;
    bool have_ = false;
};

inline uint16_t to_f16(float x) { return _cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT); }
inline float from_f16(uint16_t h) { return _cvtsh_ss(h); }

void quantize_block_q8_0(const float* x, uint8_t* blk) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(x[i]));
    const float d = amax / 127.0f;
    const uint16_t dh = to_f16(d);
    const float id = d != 0.0f ? 127.0f / amax : 0.0f;
    std::memcpy(blk, &dh, 2);
    for (int i = 0; i < 32; ++i) {
        long q = std::lround(x[i] * id);  // half away from zero, as std::round
        if (q > 127) q = 127;
        if (q < -127) q = -127;
        blk[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(q));
    }
}

}  // namespace

extern "C" {

void sixi_synth_normal_f32(uint64_t seed, uint64_t seq, float mul, float* out, int64_t n) {
    NormalStream ns(seed, seq);
    for (int64_t i = 0; i < n; ++i) out[i] = static_cast<float>(ns.next() * static_cast<double>(mul));
}

void sixi_synth_f32_to_f16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = to_f16(x[i]);
}

void sixi_synth_f16_to_f32(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = from_f16(x[i]);
}

int sixi_synth_quantize_q8_0(const float* x, void* dst, int64_t n) {
    if (n < 0 || n % 32) return -1;
    uint8_t* out = static_cast<uint8_t*>(dst);
    for (int64_t b = 0; b < n / 32; ++b) quantize_block_q8_0(x + 32 * b, out + 34 * b);
    return 0;
}

void sixi_synth_lengths(uint64_t seed, int64_t S, int32_t lo, int32_t span, int32_t* out) {
    Pcg32 r(seed, kSynthSeqLengths);
    for (int64_t s = 0; s < S; ++s) out[s] = lo + static_cast<int32_t>(r.next() % static_cast<uint32_t>(span));
}

int sixi_synth_q(uint64_t seed, int32_t type, float mul, void* dst, int64_t S, int64_t n_q, int64_t H,
                 int64_t D, int n_threads) {
    if (type != 0 && type != 1) return -1;
    const int64_t per = n_q * H * D;
#pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(dynamic, 1)
    for (int64_t s = 0; s < S; ++s) {
        NormalStream ns(seed, (kSynthTensorQ << 32) | static_cast<uint64_t>(s));
        for (int64_t i = 0; i < per; ++i) {
            const float x = static_cast<float>(ns.next() * static_cast<double>(mul));
            if (type == 0) static_cast<float*>(dst)[s * per + i] = x;
            else static_cast<uint16_t*>(dst)[s * per + i] = to_f16(x);
        }
    }
    return 0;
}

int sixi_synth_kv(uint64_t seed, uint64_t tensor_id, int32_t type, float mul, void* dst, int64_t S,
                  int64_t Hkv, int64_t D, const int32_t* n_cells, int64_t nb1, int64_t nb2, int64_t nb3,
                  int n_threads) {
    if (type != 1 && type != 8) return -1;
    if (type == 8 && D % 32) return -1;
#pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(dynamic, 1)
    for (int64_t s = 0; s < S; ++s) {
        NormalStream ns(seed, (tensor_id << 32) | static_cast<uint64_t>(s));
        std::vector<float> row(static_cast<size_t>(D));
        for (int64_t c = 0; c < n_cells[s]; ++c) {
            for (int64_t g = 0; g < Hkv; ++g) {
                for (int64_t d = 0; d < D; ++d) row[d] = static_cast<float>(ns.next() * static_cast<double>(mul));
                uint8_t* p = static_cast<uint8_t*>(dst) + s * nb3 + c * nb1 + g * nb2;
                if (type == 1) {
                    uint16_t* h = reinterpret_cast<uint16_t*>(p);
                    for (int64_t d = 0; d < D; ++d) h[d] = to_f16(row[d]);
                } else {
                    for (int64_t b = 0; b < D / 32; ++b) quantize_block_q8_0(row.data() + 32 * b, p + 34 * b);
                }
            }
        }
    }
    return 0;
}

}  // extern "C"
