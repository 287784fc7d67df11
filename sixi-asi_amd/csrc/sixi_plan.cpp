// sixi_plan.cpp -- the host-side verify batch former of include/sixi_plan.h.
//
// SIXI_PAD_REFERENCE follows LlamaCppBackend::Impl::exec_verify_group
// (src/core/core_execution.cpp:2016-2212):
//   R      = the longest block of the group (:2019-2022);
//   room   = n_ctx_seq - N, or 0 when the stream is full (:2033-2034);
//   rows   = max(real, min(R, room)) (:2035);
//   parts  = streams grouped by equal rows, first fit in input order (:2038-2045);
//   offset = running sum of rows inside a part, stream-major (:2048-2049).
// SIXI_PAD_NONE puts every stream in one part with rows = real.
#include <cstdint>
#include <vector>

#include "sixi_attn.h"
#include "sixi_plan.h"

extern "C" int sixi_verify_plan(const sixi_verify_stream* in, int32_t n, int64_t n_ctx_seq, int32_t pad_mode,
                                sixi_verify_slot* out, int32_t* n_parts) {
    if (!n_parts || n < 0 || (n > 0 && (!in || !out))) return SIXI_E_INVALID_ARGUMENT;
    if (pad_mode != SIXI_PAD_REFERENCE && pad_mode != SIXI_PAD_NONE) return SIXI_E_INVALID_ARGUMENT;
    for (int32_t i = 0; i < n; ++i)
        if (in[i].cached < 0 || in[i].real < 1) return SIXI_E_INVALID_ARGUMENT;
    *n_parts = 0;
    if (n == 0) return SIXI_OK;

    if (pad_mode == SIXI_PAD_NONE) {
        int64_t off = 0;
        for (int32_t i = 0; i < n; ++i) {
            out[i] = sixi_verify_slot{0, i, (int32_t)off, in[i].real};
            off += in[i].real;
        }
        *n_parts = 1;
        return SIXI_OK;
    }

    const int64_t ctx = n_ctx_seq == 0 ? 4096 : n_ctx_seq;
    int64_t R = 0;
    for (int32_t i = 0; i < n; ++i) R = in[i].real > R ? in[i].real : R;
    std::vector<int64_t> part_rows;   // rows of the streams in part p
    std::vector<int64_t> part_total;  // rows of part p so far
    std::vector<int32_t> part_count;  // streams in part p so far
    for (int32_t i = 0; i < n; ++i) {
        const int64_t N = in[i].cached;
        const int64_t room = ctx > N ? ctx - N : 0;
        const int64_t fit = R < room ? R : room;
        const int64_t rows = in[i].real > fit ? in[i].real : fit;
        int32_t p = 0;
        while (p < (int32_t)part_rows.size() && part_rows[p] != rows) ++p;
        if (p == (int32_t)part_rows.size()) {
            part_rows.push_back(rows);
            part_total.push_back(0);
            part_count.push_back(0);
        }
        out[i] = sixi_verify_slot{p, part_count[p], (int32_t)part_total[p], (int32_t)rows};
        part_total[p] += rows;
        part_count[p] += 1;
    }
    *n_parts = (int32_t)part_rows.size();
    return SIXI_OK;
}
