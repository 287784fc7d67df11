// ref_shim.cpp -- extern "C" entry points over the reference's own codec and metric functions
// (src/core/numeric.cpp), built by oracle/Makefile into oracle/_ref/ together with that
// source file exactly as it lies in the reference tree.  Test infrastructure only: the
// oracle's restated codecs are checked bit-for-bit against these.
#include "sixi_asi/numeric.hpp"

#include <cstdint>

extern "C" {

float ref_fp16_to_fp32(uint16_t h) { return sixi_asi::fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return sixi_asi::fp32_to_fp16(f); }

void ref_fp32_to_fp16_row(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = sixi_asi::fp32_to_fp16(x[i]);
}

// Returns 0 on success, else the reference's ErrorCode value.
int ref_quantize_row_q8_0(const float* x, void* dst, int64_t n) {
    const sixi_asi::Status st =
        sixi_asi::quantize_row_q8_0(x, static_cast<sixi_asi::q8_0_block*>(dst), n);
    return static_cast<int>(st.code);
}

int ref_q8_0_block_bytes(void) { return static_cast<int>(sizeof(sixi_asi::q8_0_block)); }

// compute_diff_metrics (src/core/numeric.cpp:701-791): out[0..7] = max_abs, mean_abs, rmse,
// cosine, kl, top1_match, ref_top1_id, test_top1_id.  Returns 0, else the ErrorCode value.
int ref_diff_metrics(const float* ref, const float* cand, int64_t n, double* out) {
    const auto r = sixi_asi::compute_diff_metrics(ref, cand, n);
    if (!r.ok()) return static_cast<int>(r.status().code);
    const sixi_asi::DiffMetrics& m = r.value();
    out[0] = m.max_abs_error;
    out[1] = m.mean_abs_error;
    out[2] = m.rmse;
    out[3] = m.cosine_similarity;
    out[4] = m.kl_divergence;
    out[5] = m.top1_match ? 1.0 : 0.0;
    out[6] = static_cast<double>(m.ref_top1_id);
    out[7] = static_cast<double>(m.test_top1_id);
    return 0;
}

}  // extern "C"
