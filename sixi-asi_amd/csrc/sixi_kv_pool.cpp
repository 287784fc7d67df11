// sixi_kv_pool.cpp -- the page pool of include/sixi_kv.h: which 256-cell pages of the K/V
// pools hold each stream's cells, with pages shared between streams.
//
// The reference keeps its KV cells in llama.cpp's memory and drives them with
// llama_memory_seq_cp (share a sequence's cells with another: snapshot save and restore,
// src/core/core_execution.cpp:3215-3216, :3245-3246) and llama_memory_seq_rm (truncate:
// rollback at :4021-4062), with 256-token pages as the layout unit
// (include/sixi_asi/manifest.hpp:124).  Here a stream's cells live in a row of a page table,
// pages are reference counted, and a copy shares pages instead of moving cells; the only
// data moved is the copy of a shared page that a stream is about to write into
// (copy-on-write), one page per write boundary.
//
// Everything here is host bookkeeping under one lock per pool; the page copies go through
// the kv_copy kernel (kv_write.hip) on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <new>
#include <algorithm>
#include <vector>

#include "abi_util.hpp"
#include "kv_internal.hpp"
#include "sixi_kv.h"

struct sixi_kv_pool {
    int32_t n_pages = 0, n_streams = 0, max_pages = 0;
    std::vector<int32_t> refs;   // per page: streams holding it
    std::vector<int32_t> free;   // free page ids (a stack)
    std::vector<int32_t> table;  // n_streams x max_pages, -1 = no page
    std::vector<int32_t> held;   // per stream: pages held, always the prefix of its row
    std::vector<sixi_view> views;
    mutable std::mutex mu;

    // Upload staging: pinned host copies of the table that alternate between uploads, each
    // with the event recorded after its copy, waited on only before that copy is refilled.
    static constexpr int kStages = 2;
    mutable int32_t* stage[kStages] = {};
    mutable hipEvent_t stage_ev[kStages] = {};
    mutable bool stage_busy[kStages] = {};
    mutable int next_stage = 0;

    ~sixi_kv_pool() {
        for (int i = 0; i < kStages; ++i) {
            if (stage_busy[i]) (void)hipEventSynchronize(stage_ev[i]);
            if (stage_ev[i]) (void)hipEventDestroy(stage_ev[i]);
            if (stage[i]) (void)hipHostFree(stage[i]);
        }
    }

    int32_t* row(int32_t s) { return table.data() + (size_t)s * max_pages; }

    void release(int32_t page) {
        if (--refs[page] == 0) free.push_back(page);
    }
    int32_t take() {
        const int32_t page = free.back();
        free.pop_back();
        refs[page] = 1;
        return page;
    }
    // stream s keeps its first `keep` pages
    void truncate(int32_t s, int32_t keep) {
        int32_t* r = row(s);
        for (int32_t i = keep; i < held[s]; ++i) {
            release(r[i]);
            r[i] = -1;
        }
        if (held[s] > keep) held[s] = keep;
    }
};

namespace {

using namespace sixi_abi;

constexpr int kMaxViews = 256;
constexpr int64_t kPage = SIXI_KV_PAGE_CELLS;

bool stream_ok(const sixi_kv_pool* p, int32_t s) { return p && s >= 0 && s < p->n_streams; }

// Copies page `from` to page `to` in every attached view.
int copy_page(const sixi_kv_pool* p, int32_t from, int32_t to, hipStream_t stream) {
    for (const sixi_view& v : p->views) {
        sixi::KvCopyArgs a{};
        a.base = static_cast<char*>(const_cast<void*>(v.data));
        a.nb1 = v.nb[1];
        a.nb2 = v.nb[2];
        a.nb3 = v.nb[3];
        a.row_bytes = row_bytes(v.type, v.ne[0]);
        a.Hkv = v.ne[2];
        a.src_stream = from;
        a.dst_stream = to;
        a.src_cell = 0;
        a.dst_cell = 0;
        a.n_cells = kPage;
        a.word4_aligned = aligned(v.data, 4) && v.nb[1] % 4 == 0 && v.nb[2] % 4 == 0 && v.nb[3] % 4 == 0;
        if (sixi::launch_kv_copy(a, stream) != hipSuccess) return SIXI_E_BACKEND;
    }
    return SIXI_OK;
}

}  // namespace

extern "C" {

int sixi_kv_pool_create(int32_t n_pages, int32_t n_streams, int32_t max_pages, sixi_kv_pool** out) {
    if (!out) return SIXI_E_INVALID_ARGUMENT;
    *out = nullptr;
    if (n_pages <= 0 || n_streams <= 0 || max_pages <= 0) return SIXI_E_INVALID_ARGUMENT;
    // a stream's cells stay addressable with int32 cell indices
    if ((int64_t)max_pages * kPage > INT32_MAX || (int64_t)n_streams * max_pages > ((int64_t)1 << 31))
        return SIXI_E_INTEGER_OVERFLOW;
    sixi_kv_pool* p = new (std::nothrow) sixi_kv_pool;
    if (!p) return SIXI_E_OUT_OF_BOUNDS;
    try {
        p->n_pages = n_pages;
        p->n_streams = n_streams;
        p->max_pages = max_pages;
        p->refs.assign((size_t)n_pages, 0);
        p->free.reserve((size_t)n_pages);
        for (int32_t i = n_pages - 1; i >= 0; --i) p->free.push_back(i);  // page 0 is taken first
        p->table.assign((size_t)n_streams * max_pages, -1);
        p->held.assign((size_t)n_streams, 0);
    } catch (const std::bad_alloc&) {
        delete p;
        return SIXI_E_OUT_OF_BOUNDS;
    }
    *out = p;
    return SIXI_OK;
}

void sixi_kv_pool_destroy(sixi_kv_pool* pool) { delete pool; }

int sixi_kv_pool_attach(sixi_kv_pool* pool, const sixi_view* pages) {
    if (!pool || !pages || !pages->data) return SIXI_E_INVALID_ARGUMENT;
    const sixi_view& v = *pages;
    if (v.type != SIXI_TYPE_F16 && v.type != SIXI_TYPE_Q8_0) return SIXI_E_INVALID_ARGUMENT;
    for (int i = 0; i < 4; ++i)
        if (v.ne[i] <= 0 || v.nb[i] <= 0) return SIXI_E_INVALID_ARGUMENT;
    if (v.ne[1] != kPage || v.ne[3] != pool->n_pages) return SIXI_E_INVALID_ARGUMENT;
    if (v.type == SIXI_TYPE_Q8_0 && v.ne[0] % 32 != 0) return SIXI_E_INVALID_ARGUMENT;
    if (v.nb[0] != (v.type == SIXI_TYPE_F16 ? 2 : 34)) return SIXI_E_INVALID_ARGUMENT;
    const int64_t rb = row_bytes(v.type, v.ne[0]);
    if (view_span(v, rb) < 0) return SIXI_E_INTEGER_OVERFLOW;
    if (!rows_disjoint(v, rb)) return SIXI_E_INVALID_ARGUMENT;
    if (!aligned(v.data, 2) || v.nb[1] % 2 || v.nb[2] % 2 || v.nb[3] % 2) return SIXI_E_ALIGNMENT;
    std::lock_guard<std::mutex> lock(pool->mu);
    if ((int)pool->views.size() >= kMaxViews) return SIXI_E_OUT_OF_BOUNDS;
    pool->views.push_back(v);
    return SIXI_OK;
}

int sixi_kv_pool_prepare_write(sixi_kv_pool* pool, int32_t s, int64_t first, int64_t n, void* stream) {
    if (!stream_ok(pool, s) || first < 0 || n < 0) return SIXI_E_INVALID_ARGUMENT;
    if (n == 0) return SIXI_OK;
    int64_t end = 0;
    if (!add_ok(first, n, &end)) return SIXI_E_INTEGER_OVERFLOW;
    const int64_t last_page = (end - 1) / kPage;
    if (last_page >= pool->max_pages) return SIXI_E_OUT_OF_BOUNDS;
    std::lock_guard<std::mutex> lock(pool->mu);
    int32_t* r = pool->row(s);
    const int32_t held = pool->held[s];
    // pages needed: new ones past the stream's prefix, and private copies of shared ones
    int64_t need = last_page + 1 > held ? last_page + 1 - held : 0;
    for (int64_t i = first / kPage; i <= last_page && i < held; ++i)
        if (pool->refs[r[i]] > 1) ++need;
    if (need > (int64_t)pool->free.size()) return SIXI_E_OUT_OF_BOUNDS;
    for (int64_t i = first / kPage; i <= last_page && i < held; ++i) {
        const int32_t old = r[i];
        if (pool->refs[old] <= 1) continue;
        const int32_t page = pool->take();
        const int rc = copy_page(pool, old, page, static_cast<hipStream_t>(stream));
        if (rc != SIXI_OK) {  // leave the stream on the shared page
            pool->release(page);
            return rc;
        }
        pool->release(old);
        r[i] = page;
    }
    for (int64_t i = held; i <= last_page; ++i) r[i] = pool->take();
    if (last_page + 1 > held) pool->held[s] = (int32_t)(last_page + 1);
    return SIXI_OK;
}

int sixi_kv_pool_seq_rm(sixi_kv_pool* pool, int32_t s, int64_t p0) {
    if (!stream_ok(pool, s)) return SIXI_E_INVALID_ARGUMENT;
    const int64_t keep = p0 <= 0 ? 0 : (p0 + kPage - 1) / kPage;
    std::lock_guard<std::mutex> lock(pool->mu);
    pool->truncate(s, (int32_t)(keep < pool->held[s] ? keep : pool->held[s]));
    return SIXI_OK;
}

int sixi_kv_pool_seq_cp(sixi_kv_pool* pool, int32_t src, int32_t dst, int64_t n) {
    if (!stream_ok(pool, src) || !stream_ok(pool, dst)) return SIXI_E_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(pool->mu);
    const int32_t src_held = pool->held[src];
    const int64_t pages = n < 0 ? src_held : (n + kPage - 1) / kPage;
    if (pages > src_held) return SIXI_E_OUT_OF_BOUNDS;
    if (src == dst) return SIXI_OK;
    pool->truncate(dst, 0);
    const int32_t* a = pool->row(src);
    int32_t* b = pool->row(dst);
    for (int64_t i = 0; i < pages; ++i) {
        b[i] = a[i];
        ++pool->refs[a[i]];
    }
    pool->held[dst] = (int32_t)pages;
    return SIXI_OK;
}

int sixi_kv_pool_page_table(const sixi_kv_pool* pool, int32_t* host_dst) {
    if (!pool || !host_dst) return SIXI_E_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(pool->mu);
    std::copy(pool->table.begin(), pool->table.end(), host_dst);
    return SIXI_OK;
}

int sixi_kv_pool_upload(const sixi_kv_pool* pool, int32_t* dev_dst, void* stream) {
    if (!pool || !dev_dst) return SIXI_E_INVALID_ARGUMENT;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return SIXI_E_BACKEND;
    std::lock_guard<std::mutex> lock(pool->mu);
    const size_t n = pool->table.size();
    if (cs != hipStreamCaptureStatusNone) {
        // under capture: the table travels in kernel arguments, so every replay stores this
        // call's table, and no host buffer has to outlive the call
        return sixi::launch_table_store(dev_dst, pool->table.data(), (int64_t)n, st) == hipSuccess ? SIXI_OK
                                                                                                  : SIXI_E_BACKEND;
    }
    // eager: an asynchronous copy from a pinned snapshot; the only wait is for the copy that
    // last read the same snapshot buffer (two uploads ago), never for the stream's other work
    const int i = pool->next_stage;
    if (!pool->stage[i]) {
        void* h = nullptr;
        if (hipHostMalloc(&h, n * sizeof(int32_t), hipHostMallocDefault) != hipSuccess) return SIXI_E_BACKEND;
        if (hipEventCreateWithFlags(&pool->stage_ev[i], hipEventDisableTiming) != hipSuccess) {
            (void)hipHostFree(h);
            pool->stage_ev[i] = nullptr;
            return SIXI_E_BACKEND;
        }
        pool->stage[i] = static_cast<int32_t*>(h);
    } else if (pool->stage_busy[i]) {
        if (hipEventSynchronize(pool->stage_ev[i]) != hipSuccess) return SIXI_E_BACKEND;
        pool->stage_busy[i] = false;
    }
    std::copy(pool->table.begin(), pool->table.end(), pool->stage[i]);
    if (hipMemcpyAsync(dev_dst, pool->stage[i], n * sizeof(int32_t), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipEventRecord(pool->stage_ev[i], st) != hipSuccess)
        return SIXI_E_BACKEND;
    pool->stage_busy[i] = true;
    pool->next_stage = (i + 1) % sixi_kv_pool::kStages;
    return SIXI_OK;
}

int32_t sixi_kv_pool_free_pages(const sixi_kv_pool* pool) {
    if (!pool) return SIXI_E_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(pool->mu);
    return (int32_t)pool->free.size();
}

int32_t sixi_kv_pool_stream_pages(const sixi_kv_pool* pool, int32_t s) {
    if (!stream_ok(pool, s)) return SIXI_E_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(pool->mu);
    return pool->held[s];
}

int32_t sixi_kv_pool_page_refs(const sixi_kv_pool* pool, int32_t page) {
    if (!pool || page < 0 || page >= pool->n_pages) return SIXI_E_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(pool->mu);
    return pool->refs[page];
}

}  // extern "C"
