// driver.cpp -- host-side exercise of the C ABIs' validation, workspace sizing, the verify
// planner, the page pool and the C oracle, built with AddressSanitizer and
// UndefinedBehaviorSanitizer on the host (tests/test_sanitizers.py builds and runs it; no GPU).
//
// Every descriptor points at host addresses that validation never dereferences.  The
// kernel launchers are replaced by functions that abort: a description that validation
// accepts is never launched here, only sized.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "fa_internal.hpp"
#include "gdn_internal.hpp"
#include "kv_internal.hpp"
#include "layer_internal.hpp"
#include "sixi_attn.h"
#include "sixi_gdn.h"
#include "sixi_kv.h"
#include "sixi_layer.h"
#include "sixi_plan.h"

extern "C" {
#include "fa_oracle.h"
}

namespace sixi {
[[noreturn]] static void no_launch(const char* what) {
    std::fprintf(stderr, "unexpected launch: %s\n", what);
    std::abort();
}
hipError_t launch_q8_stage(const Q8StageArgs&, hipStream_t) { no_launch("q8 stage"); }
hipError_t launch_mask_prefix(const FaArgs&, hipStream_t) { no_launch("mask pre-pass"); }
hipError_t launch_decode(const FaArgs&, int, int, int, int, hipStream_t) { no_launch("decode"); }
hipError_t launch_prefill(const FaArgs&, int, int, int, hipStream_t) { no_launch("prefill"); }
int decode_num_groups(const FaArgs&, int cu_count, int per_cu) { return cu_count * per_cu; }
hipError_t launch_kv_write(const KvWriteArgs&, hipStream_t) { no_launch("kv write"); }
hipError_t launch_kv_copy(const KvCopyArgs&, hipStream_t) { no_launch("kv copy"); }
hipError_t launch_table_store(int32_t*, const int32_t*, int64_t, hipStream_t) { no_launch("table store"); }
hipError_t launch_qk_prologue(const QkPrologueArgs&, hipStream_t) { no_launch("prologue"); }
hipError_t launch_attn_gate(const AttnGateArgs&, hipStream_t) { no_launch("gate"); }
hipError_t launch_gdn_verify(const GdnArgs&, hipStream_t) { no_launch("gdn"); }
}  // namespace sixi

namespace {

std::mt19937_64 rng(0x51A7);
int64_t pick(std::initializer_list<int64_t> v) {
    return *(v.begin() + (int64_t)(rng() % v.size()));
}
// 4-d view with dims ne (innermost first) and contiguous strides of `es`-byte elements
sixi_view dense(const void* data, int32_t type, int64_t es, int64_t n0, int64_t n1, int64_t n2, int64_t n3) {
    sixi_view v{};
    v.data = data;
    v.type = type;
    v.ne[0] = n0; v.ne[1] = n1; v.ne[2] = n2; v.ne[3] = n3;
    v.nb[0] = es; v.nb[1] = n0 * es; v.nb[2] = v.nb[1] * n1; v.nb[3] = v.nb[2] * n2;
    return v;
}
const char* FAKE = reinterpret_cast<const char*>(uintptr_t(0x7F0000000000ull));

int attention_descriptors() {
    int accepted = 0;
    for (int it = 0; it < 20000; ++it) {
        const int64_t D = pick({128, 256, 64, 0, -1});
        const int64_t S = pick({1, 2, 32, 512, 513, 0});
        const int64_t nq = pick({1, 8, 16, 48, 200, 2048, 1 << 21});
        const int64_t Hkv = pick({1, 4, 8, 3});
        const int64_t H = Hkv * pick({1, 6, 8}) + pick({0, 0, 0, 1});
        const int64_t nkv = pick({256, 8192, 65536, 1 << 27, 7});
        const int32_t kt = (int32_t)pick({SIXI_TYPE_F16, SIXI_TYPE_Q8_0, SIXI_TYPE_F32});
        const int64_t row = kt == SIXI_TYPE_Q8_0 ? D / 32 * 34 : D * 2;
        sixi_attn_params p{};
        p.q = dense(FAKE, SIXI_TYPE_F32, 4, D, nq, H, S);
        if (rng() % 8 == 0) p.q.nb[1] = pick({INT64_MAX / 2, 3, -16});
        p.k = dense(FAKE + (1ll << 36), kt, 1, D, nkv, Hkv, S);
        p.k.nb[0] = kt == SIXI_TYPE_Q8_0 ? 34 : 2;
        p.k.nb[1] = Hkv * row; p.k.nb[2] = row; p.k.nb[3] = nkv * Hkv * row;
        if (rng() % 8 == 0) p.k.nb[3] = pick({INT64_MAX, 0, 4});
        p.v = p.k;
        p.v.data = FAKE + (2ll << 36);
        p.out = dense(FAKE + (3ll << 36), SIXI_TYPE_F32, 4, D, H, nq, S);
        p.kv_len = rng() % 4 ? reinterpret_cast<const int32_t*>(FAKE) : nullptr;
        p.q_len = reinterpret_cast<const int32_t*>(FAKE);
        p.mask_mode = (int32_t)pick({SIXI_MASK_BLOCK_CAUSAL, SIXI_MASK_NONE, SIXI_MASK_EXPLICIT, 7});
        if (p.mask_mode == SIXI_MASK_EXPLICIT) {
            p.mask = dense(FAKE + (4ll << 36), SIXI_TYPE_F16, 2, nkv + pick({0, 5}), nq, 1, pick({1, S}));
        }
        p.scale = (float)pick({1, 0}) * 0.088f;
        p.max_bias = (float)pick({0, 0, 8, -1});
        p.logit_softcap = (float)pick({0, 0, 30});
        if (rng() % 3 == 0) {  // paged
            p.page_table = reinterpret_cast<const int32_t*>(FAKE + (5ll << 36));
            p.page_table_stride = pick({1, 32, 0, (1ll << 30)});
            p.k.ne[1] = p.v.ne[1] = pick({256, 128});
            p.k.ne[3] = p.v.ne[3] = pick({1, 100, 1ll << 33});
            p.k.nb[3] = p.v.nb[3] = 256 * Hkv * row;
        }
        const int rc = sixi_attn_validate(&p);
        size_t ws = 0;
        const int rw = sixi_attn_workspace_bytes(&p, &ws);
        if (rc != rw) {
            std::fprintf(stderr, "validate %d vs workspace %d\n", rc, rw);
            return -1;
        }
        if (rc == SIXI_OK) {
            ++accepted;
            if (ws == 0 || ws % 256) {
                std::fprintf(stderr, "workspace %zu\n", ws);
                return -1;
            }
        }
        (void)sixi_attn_strerror(rc);
    }
    return accepted;
}

int kv_write_descriptors() {
    int accepted = 0;
    for (int it = 0; it < 5000; ++it) {
        const int64_t D = pick({128, 256, 96, 0});
        const int64_t S = pick({1, 32}), n = pick({1, 16}), Hkv = pick({4, 1}), cells = pick({4096, 256, 0});
        const int32_t t = (int32_t)pick({SIXI_TYPE_F16, SIXI_TYPE_Q8_0, SIXI_TYPE_F32});
        sixi_kv_write_params p{};
        p.src = dense(FAKE, SIXI_TYPE_F32, 4, D, n, Hkv, S);
        const int64_t row = t == SIXI_TYPE_Q8_0 ? D / 32 * 34 : D * 2;
        p.dst = dense(FAKE + (1ll << 36), t, 1, D, cells, Hkv, S);
        p.dst.nb[0] = t == SIXI_TYPE_Q8_0 ? 34 : 2;
        p.dst.nb[1] = Hkv * row; p.dst.nb[2] = row; p.dst.nb[3] = cells * Hkv * row;
        if (rng() % 2) {
            p.page_table = reinterpret_cast<const int32_t*>(FAKE);
            p.page_table_stride = pick({16, 0, -1});
            p.dst.ne[1] = pick({256, 255});
            p.dst.ne[3] = pick({64, 0});
        }
        if (sixi_kv_write_validate(&p) == SIXI_OK) ++accepted;
    }
    return accepted;
}

int planner() {
    for (int it = 0; it < 5000; ++it) {
        const int n = (int)pick({0, 1, 5, 32, 64});
        std::vector<sixi_verify_stream> in((size_t)std::max(n, 1));
        for (int i = 0; i < n; ++i) {
            in[i].stream = i;
            in[i].cached = (int32_t)(rng() % 5000) - (rng() % 50 == 0 ? 6000 : 0);
            in[i].real = (int32_t)(rng() % 17);
        }
        std::vector<sixi_verify_slot> out((size_t)std::max(n, 1));
        int32_t parts = -1;
        const int rc = sixi_verify_plan(in.data(), n, pick({0, 4096, 300}), (int32_t)pick({0, 1, 2}), out.data(), &parts);
        if (rc == SIXI_OK) {
            for (int i = 0; i < n; ++i)
                if (out[i].part < 0 || out[i].part >= parts || out[i].rows < in[i].real) return -1;
        }
    }
    return 0;
}

int pool_ops() {
    sixi_kv_pool* pool = nullptr;
    if (sixi_kv_pool_create(64, 8, 12, &pool) != SIXI_OK) return -1;
    std::vector<int32_t> table(8 * 12);
    for (int it = 0; it < 20000; ++it) {
        const int32_t s = (int32_t)(rng() % 9) - (rng() % 20 == 0 ? 2 : 0);
        switch (rng() % 5) {
            case 0: (void)sixi_kv_pool_prepare_write(pool, s, (int64_t)(rng() % 3500) - 2, (int64_t)(rng() % 600), nullptr); break;
            case 1: (void)sixi_kv_pool_seq_rm(pool, s, (int64_t)(rng() % 3500) - 1); break;
            case 2: (void)sixi_kv_pool_seq_cp(pool, s, (int32_t)(rng() % 8), (int64_t)(rng() % 3500) - 1); break;
            case 3: (void)sixi_kv_pool_page_table(pool, table.data()); break;
            default: (void)sixi_kv_pool_page_refs(pool, (int32_t)(rng() % 70) - 3); break;
        }
        if (sixi_kv_pool_free_pages(pool) < 0) return -1;
    }
    int32_t held = 0;
    for (int32_t s = 0; s < 8; ++s) held += sixi_kv_pool_stream_pages(pool, s);
    sixi_kv_pool_destroy(pool);
    sixi_kv_pool* bad = nullptr;
    if (sixi_kv_pool_create(0, 1, 1, &bad) == SIXI_OK || bad) return -1;
    if (sixi_kv_pool_create(1, INT32_MAX, INT32_MAX, &bad) == SIXI_OK) return -1;
    return held;
}

int oracle_cases() {
    // small attention cases in both KV types, both accumulators, masks with and without softcap/ALiBi
    for (int it = 0; it < 40; ++it) {
        const int64_t S = 2, nq = 1 + (int64_t)(rng() % 9), H = 4, Hkv = 2, D = 64, nkv = 40 + (int64_t)(rng() % 60);
        const bool q8 = it % 2;
        std::vector<float> q((size_t)(S * nq * H * D)), kf((size_t)(S * nkv * Hkv * D)), vf(kf.size());
        oracle_fill_normal_f32(it, 1, 1.0f, q.data(), (int64_t)q.size());
        oracle_fill_normal_f32(it, 2, 1.0f, kf.data(), (int64_t)kf.size());
        oracle_fill_normal_f32(it, 3, 1.0f, vf.data(), (int64_t)vf.size());
        const int64_t row = q8 ? D / 32 * 34 : D * 2;
        std::vector<uint8_t> k((size_t)(S * nkv * Hkv * row)), v(k.size());
        for (int64_t r = 0; r < S * nkv * Hkv; ++r) {
            if (q8) {
                oracle_quantize_row_q8_0(&kf[(size_t)(r * D)], &k[(size_t)(r * row)], D);
                oracle_quantize_row_q8_0(&vf[(size_t)(r * D)], &v[(size_t)(r * row)], D);
            } else {
                oracle_fp32_to_fp16_row(&kf[(size_t)(r * D)], reinterpret_cast<uint16_t*>(&k[(size_t)(r * row)]), D);
                oracle_fp32_to_fp16_row(&vf[(size_t)(r * D)], reinterpret_cast<uint16_t*>(&v[(size_t)(r * row)]), D);
            }
        }
        const int32_t kl[2] = {(int32_t)(nkv - nq - (int64_t)(rng() % 5)), 0};
        const int32_t ql[2] = {(int32_t)nq, (int32_t)(nq / 2)};
        std::vector<uint16_t> mask((size_t)(S * nq * nkv));
        if (oracle_build_kq_mask(mask.data(), nkv, nq, S, kl, ql, 1) != 0) return -1;
        oracle_view vq{q.data(), 0, {D, nq, H, S}, {4, D * 4, D * 4 * nq, D * 4 * nq * H}};
        oracle_view vk{k.data(), q8 ? 8 : 1, {D, nkv, Hkv, S}, {q8 ? 34 : 2, Hkv * row, row, nkv * Hkv * row}};
        oracle_view vv = vk;
        vv.data = v.data();
        oracle_view vm{mask.data(), 1, {nkv, nq, 1, S}, {2, nkv * 2, nkv * 2 * nq, nkv * 2 * nq}};
        std::vector<float> out((size_t)(S * nq * H * D));
        const float bias = it % 3 == 0 ? 8.0f : 0.0f, cap = it % 5 == 0 ? 30.0f : 0.0f;
        if (oracle_flash_attn_ext(&vq, &vk, &vv, &vm, 0.125f, bias, cap, out.data(), it % 4 < 2, 2) != 0) return -1;
        for (float x : out)
            if (!std::isfinite(x) && x == x) return -1;  // rows without cells are 0, never inf
    }
    // gated delta rule, ragged rows
    const int64_t S = 2, n = 5, G = 3, K = 16, HD = 8;
    std::vector<float> q((size_t)(S * n * G * K)), k(q.size()), v((size_t)(S * n * G * HD)), a((size_t)(S * n * G)),
        b(a.size()), st((size_t)(S * G * HD * K)), y(v.size());
    oracle_fill_normal_f32(7, 1, 0.3f, q.data(), (int64_t)q.size());
    oracle_fill_normal_f32(7, 2, 0.3f, k.data(), (int64_t)k.size());
    oracle_fill_normal_f32(7, 3, 1.0f, v.data(), (int64_t)v.size());
    oracle_fill_normal_f32(7, 4, 1.0f, st.data(), (int64_t)st.size());
    for (size_t i = 0; i < a.size(); ++i) {
        a[i] = 0.9f;
        b[i] = 0.5f;
    }
    const int32_t gq[2] = {5, 2}, snap[2] = {3, 2};
    oracle_gdn_verify(q.data(), k.data(), v.data(), a.data(), b.data(), st.data(), y.data(), S, n, G, K, HD, gq, snap, 1);
    return 0;
}

}  // namespace

int main() {
    const int acc = attention_descriptors();
    std::printf("attention descriptors accepted: %d\n", acc);
    if (acc <= 0) return 1;
    const int kw = kv_write_descriptors();
    std::printf("kv write descriptors accepted: %d\n", kw);
    if (kw <= 0) return 1;
    if (planner() != 0) return 1;
    const int held = pool_ops();
    std::printf("pool: %d pages held after the random operations\n", held);
    if (held < 0) return 1;
    if (oracle_cases() != 0) return 1;
    std::printf("sanitized host run: ok\n");
    return 0;
}
