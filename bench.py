"""Benchmark of the MI355X attention hot path (one GPU).

Headline workload: batched speculative verify -- 32 streams x 16 drafted rows, block-causal,
per-stream cached lengths drawn from [512, 16384], 24 q-heads / 4 kv-heads x 128, f32 Q, f16
KV in the page pool (every stream's 256-cell pages at shuffled pool positions, read through
the page table; each page head-major, [kv-head][256 cells][D]) -- one attention layer per
step.  The same call over llama.cpp's token-major cell rows (in pages, and as one contiguous
cache per stream) is reported beside it.  A step is one call of the C ABI
(sixi_attn_forward), i.e. the split-K kernel (decode_wide, 32-cell steps) plus its merge
kernel, timed with HIP events on the stream the library launches on, inputs resident in HBM.

Prints one JSON line: value = algorithmic HBM GB/s of the verify call (K/V of every attended
cell + Q + O, counted once) at the mean time of the steps bracketed by synchronisation (the
per-call median and p10/p90 beside it); roofline = that rate against the 8 TB/s HBM peak;
verify_explicit_mask = the same call with the mask handed over as a ggml KQ mask (the drop-in
path); the other
configurations (single-stream decode and verify, long q8_0 decode/verify, chunked prefill)
are reported beside it when their kernels are built; cpu_baseline = the oracle (a
restatement of ggml's CPU flash_attn_ext, f16 V accumulator as upstream) on the host cores,
same inputs.

`--workload copy` instead times a plain 1 GiB device copy: the calibration run for the HBM
byte counters (FETCH_SIZE / WRITE_SIZE) used in the traffic figures.  `--workload prefill`
times only the chunked causal prefill (two 2048-row chunks), for profiling that kernel;
`prefill_q8` and `prefill_d256_q8` the same over a q8_0 cache (128- and 256-dim heads; f16
staging), and their `_bounded` forms with FLAG_BOUNDED_WORKSPACE (q8_0 tiles converted in LDS).
`verify_q8`, `verify_d256` and `verify_d256_q8` time the batched verify alone over a q8_0 cache
(128-dim heads) and at 256-dim heads over an f16 or q8_0 cache; `verify_op` the engine's own
operating point (32 streams x q_len 4 and 6, 256-dim heads, f16 and q8_0 caches); `headline`
the headline call alone (for the profiler); `verify_mask` and `prefill_mask` the verify (over
the contiguous cache) and the prefill with their masks handed over as llama.cpp's explicit f16
KQ mask (the mask pre-pass, then the kernels it chooses between).
"""
from __future__ import annotations

import argparse
import json
import pathlib
import re
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "sixi-asi_amd"))

METRIC = "verify-attn µs/layer & HBM GB/s (32 streams×16 tok, 8k ctx); prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3  # published dense FP32 (vector) peak
TRAFFIC_PROFILE = ROOT / "profiles" / "verify_b32_headmajor_pages.txt"


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Untimed sustained load before each timed series.  After any idle period (input generation,
# host work between configurations) the MI355X runs the first ~10 calls of a sustained
# HBM + MFMA load at full speed, then ~50-90 calls up to 35% slower while its power
# management settles (measured on the headline verify: 145 us, then 165-197 us for calls
# 11-60, back to 143-146 us after ~100 calls / 15 ms; the same after a 50 ms or 2 s pause).
# The timed steps measure the settled state, which is what a loaded server sees: the call
# runs for PRECONDITION_S of wall time first, then the W warm-up steps, then the K timed ones.
PRECONDITION_S = 0.06


def _precondition(fn, seconds: float = PRECONDITION_S) -> None:
    """Runs fn back to back (batches of 8, then a synchronisation) for `seconds` of wall time."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def _timed(call, steps: int, warmup: int):
    """(ms per call, per-call ms list): after the preconditioning and `warmup` untimed calls,
    `steps` calls bracketed by synchronisation and one event pair -- the timed region, whose
    mean is the rate reported -- then the same number of calls again with an event after each,
    for the distribution (those events cost about 2 us per call on MI355X, so the per-call
    figures sit slightly above the bracketed mean)."""
    import torch

    stream = torch.cuda.current_stream()
    _precondition(call)
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        call()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    return ms, [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]


def time_calls(fa, w, dev, steps: int, warmup: int, out=None, mask=None, bounded=False):
    """Per-call GPU times (ms) with events on the stream the library launches on.  With `mask`
    (a ggml f16 KQ mask) the calls take the explicit-mask path instead of w.mask_mode;
    `bounded` sets FLAG_BOUNDED_WORKSPACE."""
    import torch

    import sixi_attn as sa

    if out is None:
        out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    mode = w.mask_mode if mask is None else sa.MASK_EXPLICIT

    def call():
        fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"],
           mask_mode=mode, mask=mask, stream=stream.cuda_stream, bounded_workspace=bounded)

    return _timed(call, steps, warmup)


def time_paged(fa, w, dev, steps: int, warmup: int, head_major: bool = False, out=None):
    """The workload's call with K and V in a page pool (include/sixi_attn.h page_table): each
    stream's 256-cell pages placed at shuffled pool pages (seeded), read through the table.
    head_major: each page holds its kv-heads one after the other ([Hkv][256 cells][D], the
    page pool's layout: a kv-head's cells of a page are one contiguous 64 KB run); otherwise
    token-major ([256 cells][Hkv][D], llama.cpp's cell rows).  Returns (ms, per-call ms, pages)."""
    import numpy as np
    import torch

    import sixi_attn as sa

    S, cap = dev["k"].shape[0], dev["k"].shape[1]
    per = cap // sa.PAGE_CELLS
    n_pages = S * per
    perm = np.random.default_rng(0x51A7).permutation(n_pages).astype(np.int32)
    table = torch.from_numpy(perm.reshape(S, per)).cuda()
    idx = table.reshape(-1).long()
    pools = []
    for name in ("k", "v"):
        c = dev[name]
        Hkv, X = c.shape[2], c.shape[3]
        if head_major:
            pool = torch.empty((n_pages, Hkv, sa.PAGE_CELLS, X), dtype=c.dtype, device="cuda").permute(0, 2, 1, 3)
        else:
            pool = torch.empty((n_pages, sa.PAGE_CELLS, Hkv, X), dtype=c.dtype, device="cuda")
        pool[idx] = c.reshape(n_pages, sa.PAGE_CELLS, Hkv, X)
        pools.append(pool)
    if out is None:
        out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    def call():
        fa(dev["q"], pools[0], pools[1], out, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=w.mask_mode,
           stream=stream.cuda_stream, page_table=table)

    ms, per_call = _timed(call, steps, warmup)
    del pools
    return ms, per_call, n_pages


def ws_bytes(fa, w, dev, mask=None, bounded=False) -> int:
    """sixi_attn_workspace_bytes of a call of workload w: the split-K partial slots; q8_0 prefill
    blocks add the f16 staging of K and V while it fits the 64 MiB cap (none with `bounded`);
    explicit llama masks add the pre-pass's row table."""
    import torch

    import sixi_attn as sa

    out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    p = fa.params(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"],
                  mask_mode=w.mask_mode if mask is None else sa.MASK_EXPLICIT, mask=mask, bounded_workspace=bounded)
    return int(fa.workspace_bytes(p))


def summarize(w, ms: float, per) -> dict:
    """`us` and the rates: the mean over the bracketed calls (the timed region); median and
    p10/p90 of the per-call times (a second pass with an event after each call)."""
    per_sorted = sorted(per)
    n = len(per_sorted)
    med = statistics.median(per_sorted)
    return {
        "us": round(ms * 1e3, 2),
        "us_median": round(med * 1e3, 2),
        "us_p10_p50_p90": [round(per_sorted[n // 10] * 1e3, 2), round(per_sorted[n // 2] * 1e3, 2),
                           round(per_sorted[(9 * n) // 10] * 1e3, 2)],
        "GBps": round(w.bytes() / (ms * 1e-3) / 1e9, 1),
        "TFLOPs": round(w.flops() / (ms * 1e-3) / 1e12, 2),
        "GBps_median": round(w.bytes() / (med * 1e-3) / 1e9, 1),
        "bytes": w.bytes(),
        "flops": w.flops(),
    }


def _cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as "Model name")."""
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(w, host, gpu_out=None, repeats: int = 5) -> dict:
    """The oracle on the host cores: the whole verify workload (all 32 streams) on every
    core of the process affinity, median of `repeats` runs after one warm-up, with the f16 V
    accumulator of ggml's CPU kernel (upstream) and, beside it, with an f32 accumulator; plus
    one stream on one thread.  With `gpu_out` (the GPU's output of the same workload,
    [S, n_q, H, D]) the distances of the GPU result from both CPU modes are reported over the
    valid rows (mean-abs, RMSE, KL, ... as compute_diff_metrics)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np

    import oracle

    threads = oracle.cpu_threads()
    oracle.attention_for_workload(host, w.kv_type, [0], v_acc_f16=True, n_threads=threads)

    def timed(acc16):
        runs, out = [], None
        for _ in range(repeats):
            t0 = time.perf_counter()
            out = oracle.attention_for_workload(host, w.kv_type, None, v_acc_f16=acc16, n_threads=threads)
            runs.append(time.perf_counter() - t0)
        return statistics.median(runs), out

    dt, ref16 = timed(True)
    dt32, ref32 = timed(False)
    # one stream near the mean length on one thread
    lens = [abs(x - sum(w.kv_len) / w.S) for x in w.kv_len]
    s1 = lens.index(min(lens))
    t0 = time.perf_counter()
    oracle.attention_for_workload(host, w.kv_type, [s1], v_acc_f16=True, n_threads=1)
    dt1 = time.perf_counter() - t0
    sub = type(w)(w.name, w.seed, 1, [w.kv_len[s1]], [w.q_len[s1]], H=w.H, Hkv=w.Hkv, D=w.D,
                  kv_type=w.kv_type, q_type=w.q_type)
    res = {
        "value": round(w.bytes() / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": _cpu_model(),
        "sample": f"the whole workload ({w.S} streams, {sum(w.kv_len)} cached cells, {sum(w.q_len)} rows), "
                  f"f16 V accumulator as ggml's CPU kernel, median of {repeats} runs: {dt * 1e3:.1f} ms/call",
        "us_per_call": round(dt * 1e6, 1),
        "f32_accumulator": {"value": round(w.bytes() / dt32 / 1e9, 3), "unit": "GB/s",
                            "us_per_call": round(dt32 * 1e6, 1),
                            "sample": f"same workload, f32 V accumulator, median of {repeats} runs"},
        "one_thread": {"value": round(sub.bytes() / dt1 / 1e9, 3), "unit": "GB/s",
                       "sample": f"stream {s1} ({w.kv_len[s1]} cached cells, {w.q_len[s1]} rows), "
                                 f"{dt1 * 1e3:.1f} ms"},
    }
    if gpu_out is not None:
        ql = host["q_len"]

        def rows(x):
            return np.concatenate([x[s, :ql[s]].ravel() for s in range(w.S)]).astype(np.float64)

        g = rows(gpu_out)
        res["gpu_vs_cpu"] = {}
        for name, ref in (("f16_accumulator_upstream", ref16), ("f32_accumulator", ref32)):
            m = oracle.diff_metrics(rows(ref), g)
            res["gpu_vs_cpu"][name] = {k: (float(f"{v:.4g}") if isinstance(v, float) else v) for k, v in m.items()}
    return res


def traffic_from_profile():
    """HBM bytes per verify call from the committed counter summary, if present."""
    if not TRAFFIC_PROFILE.exists():
        return None
    m = re.search(r"^traffic_bytes_per_call:\s*(\d+)", TRAFFIC_PROFILE.read_text(), re.M)
    return int(m.group(1)) if m else None


def copy_calibration(steps: int) -> int:
    import torch

    n = 1 << 28  # 1 GiB of f32
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(steps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"workload": "copy", "bytes_read_per_copy": n * 4, "bytes_written_per_copy": n * 4,
                      "copies": steps}), flush=True)
    return 0


def time_prefill(fa, steps: int, warmup: int, kv_type=None, head_dim=None, explicit_mask=False, bounded=False):
    """Both 2048-row chunks of the 4k causal prefill: (TFLOP/s, us for the two chunks).
    kv_type q8_0 runs the same chunks over a q8_0 cache (K and V staged as f16 per call under the
    64 MiB cap, at 128- and 256-dim heads);
    explicit_mask hands the causal mask over as a ggml f16 KQ mask (the ggml hook's path);
    bounded sets FLAG_BOUNDED_WORKSPACE (the q8_0 tiles converted in LDS, nothing staged)."""
    import dataclasses

    import torch

    from sixi_attn import workloads as wl

    pre = []
    for name in ("prefill_chunk0", "prefill_chunk1"):
        wp = wl.config(name)
        if kv_type is not None:
            wp = dataclasses.replace(wp, kv_type=kv_type)
        if head_dim is not None:
            wp = dataclasses.replace(wp, D=head_dim)
        dp = wl.to_device(wl.make_host(wp))
        mask = None
        if explicit_mask:
            mask = torch.from_numpy(wl.kq_mask(dp["k"].shape[1], wp.n_q, wp.kv_len, wp.q_len)).view(torch.float16).cuda()
        msp, _ = time_calls(fa, wp, dp, steps, warmup, mask=mask, bounded=bounded)
        pre.append((wp, msp, ws_bytes(fa, wp, dp, bounded=bounded)))
        del dp
    flops = sum(wp.flops() for wp, _, _ in pre)
    t = sum(msp for _, msp, _ in pre)
    return flops / (t * 1e-3) / 1e12, t * 1e3, max(b for _, _, b in pre)


def time_kv_store(w, dev, steps: int, warmup: int) -> dict:
    """The KV-cache store before the verify attention (include/sixi_kv.h): the block's K and V
    rows of every stream (f32, [S, q_len, Hkv, D]) written to cells kv_len .. kv_len+q_len-1,
    as f16 into the workload's own cache and as q8_0 into a q8_0 cache of the same cells.

    The two launches take a few microseconds of GPU time, less than the host needs to issue
    them from Python, so they are captured once in a HIP graph (8 K+V stores per graph) and
    the graph is replayed; the time is GPU time per K+V store."""
    import ctypes

    import torch

    import sixi_attn as sa

    lib = sa.load_library()
    res = {}
    src_k = torch.randn((w.S, w.n_q, w.Hkv, w.D), dtype=torch.float32, device="cuda")
    src_v = torch.randn_like(src_k)
    q8_k = torch.zeros((w.S, dev["k"].shape[1], w.Hkv, w.D // 32 * 34), dtype=torch.uint8, device="cuda")
    q8_v = torch.zeros_like(q8_k)
    rows = int(sum(w.q_len)) * w.Hkv
    per_graph = 8
    for name, ck, cv, row_bytes in (("f16", dev["k"], dev["v"], w.D * 2), ("q8_0", q8_k, q8_v, w.D // 32 * 34)):
        pk = sa.kv_write_params(src_k, ck, dev["kv_len"], dev["q_len"])
        pv = sa.kv_write_params(src_v, cv, dev["kv_len"], dev["q_len"])

        def store():
            st = torch.cuda.current_stream().cuda_stream
            pk.stream = pv.stream = st
            for p in (pk, pv):
                rc = lib.sixi_kv_write(ctypes.byref(p))
                if rc != sa.OK:
                    raise sa.SixiAttnError(rc, sa.strerror(rc))

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                store()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(per_graph):
                store()
        torch.cuda.synchronize()
        reps = max(1, steps // per_graph)
        _precondition(g.replay)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / (reps * per_graph) * 1e3
        nbytes = 2 * rows * (w.D * 4 + row_bytes)  # K and V: f32 rows read, cache rows written
        res[name] = {"us_k_and_v": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes}
        del g
    del q8_k, q8_v
    return res


def _graph_us(fn, steps: int, warmup: int, per_graph: int = 8) -> float:
    """GPU time per call of ``fn`` (a few short launches): warmed up on a side stream, captured
    ``per_graph`` times in one HIP graph, the graph replayed; microseconds per call."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    _precondition(g.replay)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * per_graph) * 1e3


def time_layer(steps: int, warmup: int) -> dict:
    """The work around the attention of one Qwen3.8 full-attention layer (include/sixi_layer.h)
    for the 256-dim verify batch (32 streams x 16 rows, 24 q-heads, 4 kv-heads): the prologue
    (Q/K RMS norm + RoPE on 64 dims, Q written, K and V stored in the f16 cache) and the output
    gate.  Algorithmic bytes: prologue 2*H*D*4 (Q half read, Q written) + 2*Hkv*D*4 (K, V read)
    + 2*Hkv*D*2 (cache rows written) per row; gate 3*H*D*4 per row (output and gate read,
    output written).  `layer`: the prologue, the attention and the gate as three calls, and as
    two with the gate fused into the attention's stores, also with the prologue's Q in f16 (GPU
    time per layer, graph replays)."""
    import ctypes

    import torch

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    lib = sa.load_library()
    w = wl.config("batched_verify_d256")
    S, R, H, Hkv, D = w.S, w.n_q, w.H, w.Hkv, w.D
    n_cells = max(a + b for a, b in zip(w.kv_len, w.q_len))
    qg = torch.randn((S, R, H, 2 * D), dtype=torch.float32, device="cuda")
    k = torch.randn((S, R, Hkv, D), dtype=torch.float32, device="cuda")
    v = torch.randn_like(k)
    wq = torch.rand(D, dtype=torch.float32, device="cuda") + 0.5
    wk = torch.rand_like(wq) + 0.5
    q_out = torch.empty((S, R, H, D), dtype=torch.float32, device="cuda")
    kc = torch.zeros((S, n_cells, Hkv, D), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    kl = torch.tensor(w.kv_len, dtype=torch.int32, device="cuda")
    ql = torch.tensor(w.q_len, dtype=torch.int32, device="cuda")
    out = torch.randn((S, R, H, D), dtype=torch.float32, device="cuda")
    pp = sa.qk_prologue_params(qg, k, v, wq, wk, q_out, kc, vc, kl, ql)
    pg = sa.SixiAttnGateParams()
    pg.out = sa.view_of(out, tokens_heads=False)
    pg.qg = sa.view_of(qg, tokens_heads=False)
    pg.q_len = ql.data_ptr()

    def call(fn, p):
        def run():
            p.stream = torch.cuda.current_stream().cuda_stream
            rc = fn(ctypes.byref(p))
            if rc != sa.OK:
                raise sa.SixiAttnError(rc, sa.strerror(rc))
        return run

    rows = int(sum(w.q_len))
    res = {"workload": f"{S} streams x {R} rows, {H} q-heads / {Hkv} kv-heads x {D}, 64 rotated dims, f16 cache"}
    for name, fn, p, per_row in (("prologue", lib.sixi_qk_prologue, pp, 2 * H * D * 4 + 2 * Hkv * D * 4 + 2 * Hkv * D * 2),
                                 ("gate", lib.sixi_attn_gate, pg, 3 * H * D * 4)):
        us = _graph_us(call(fn, p), steps, warmup)
        nbytes = rows * per_row
        res[name] = {"us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes,
                     "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    # the layer around the attention: prologue -> attention -> gate (three calls) against
    # prologue -> attention with the output gate fused into its stores (SIXI_ATTN_FLAG_GATE)
    fa = sa.FlashAttnExt()
    prologue, gate = call(lib.sixi_qk_prologue, pp), call(lib.sixi_attn_gate, pg)

    def three():
        prologue()
        fa(q_out, kc, vc, out, kv_len=kl, q_len=ql)
        gate()

    def two():
        prologue()
        fa(q_out, kc, vc, out, kv_len=kl, q_len=ql, gate=qg)

    q16 = torch.empty((S, R, H, D), dtype=torch.float16, device="cuda")
    pp16 = sa.qk_prologue_params(qg, k, v, wq, wk, q16, kc, vc, kl, ql)
    prologue16 = call(lib.sixi_qk_prologue, pp16)

    def two16():
        prologue16()
        fa(q16, kc, vc, out, kv_len=kl, q_len=ql, gate=qg)

    res["layer"] = {"prologue_attention_gate_us": round(_graph_us(three, steps, warmup), 2),
                    "prologue_attention_with_fused_gate_us": round(_graph_us(two, steps, warmup), 2),
                    "prologue_f16_q_attention_with_fused_gate_us": round(_graph_us(two16, steps, warmup), 2)}
    return res


def time_gdn(steps: int, warmup: int) -> dict:
    """The gated-delta-rule verify (include/sixi_gdn.h) of one linear-attention layer for the
    verify batch: 32 streams x 16 rows, 48 value heads of 128 with 128-dim keys (the model's
    ssm_time_step_rank / ssm_state_size).  Algorithmic bytes: the state read and written once
    (2 * 4 * 128 * 128 per group and stream) plus q, k, v, y (4 * 128 each per row and group) and
    alpha, beta; FLOPs: 3 * 2 * 128 * 128 per row and group (read, update, output)."""
    import ctypes

    import torch

    import sixi_attn as sa

    lib = sa.load_library()
    S, n, G, K, HD = 32, 16, 48, 128, 128
    q = torch.randn((S, n, G, K), device="cuda") / K ** 0.5
    k = torch.nn.functional.normalize(torch.randn((S, n, G, K), device="cuda"), dim=-1)
    v = torch.randn((S, n, G, HD), device="cuda")
    al = torch.rand((S, n, G), device="cuda") * 0.2 + 0.8
    be = torch.rand((S, n, G), device="cuda")
    y = torch.empty((S, n, G, HD), device="cuda")
    st = torch.randn((S, G, HD, K), device="cuda") * 0.5
    p = sa.gdn_verify_params(q, k, v, al, be, y, st)

    def run():
        p.stream = torch.cuda.current_stream().cuda_stream
        rc = lib.sixi_gdn_verify(ctypes.byref(p))
        if rc != sa.OK:
            raise sa.SixiAttnError(rc, sa.strerror(rc))

    us = _graph_us(run, steps, warmup)
    nbytes = S * G * (2 * 4 * HD * K + n * (4 * (2 * K + 2 * HD) + 8))
    flops = S * n * G * 6 * HD * K
    return {"workload": f"{S} streams x {n} rows, {G} groups, state {HD} x {K} f32, in place", "us": round(us, 2),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes,
            "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "TFLOPs": round(flops / (us * 1e-6) / 1e12, 2), "flops": flops,
            "frac_of_fp32_peak": round(flops / (us * 1e-6) / 1e12 / FP32_PEAK_TFLOPS, 4)}


def batched_verify_q8():
    """The headline verify workload over a q8_0 cache (same seeds, lengths and heads)."""
    import dataclasses

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    return dataclasses.replace(wl.config("batched_verify"), name="batched_verify_q8", kv_type=sa.TYPE_Q8_0)


def operating_point(q_len: int, q8: bool):
    """The verify batch the engine runs at 8 or more streams: 3 or 5 drafted tokens per stream
    (q_len 4 or 6; src/core/core_execution.cpp:3995-4003) on the model's 256-dim heads
    (configs/qwen3.8-27b-ud-q4-k-xl.sixi:35), the headline's 32 streams and cached lengths, an
    f16 or q8_0 cache."""
    import dataclasses

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    w = wl.config("batched_verify_d256")
    return dataclasses.replace(w, name=f"batched_verify_d256_q{q_len}" + ("_q8" if q8 else ""), q_len=[q_len] * w.S,
                               kv_type=sa.TYPE_Q8_0 if q8 else w.kv_type)


OPERATING_POINTS = tuple((ql, q8) for q8 in (False, True) for ql in (4, 6))


def headline_only(steps: int, warmup: int) -> int:
    """The headline call alone (the page pool with head-major pages), for the profiler."""
    import sixi_attn as sa
    from sixi_attn import workloads as wl

    fa = sa.FlashAttnExt()
    w = wl.config("batched_verify")
    dev = wl.to_device(wl.make_host(w))
    ms, per, n_pages = time_paged(fa, w, dev, max(1, steps), warmup, head_major=True)
    r = summarize(w, ms, per)
    _log(f"headline: {r}")
    print(json.dumps(r), flush=True)
    return 0


def verify_op_only(steps: int, warmup: int) -> int:
    """The four operating-point verify calls alone (32 streams, q_len 4 and 6, 256-dim heads,
    f16 and q8_0 caches): eager median and graph-replay time per call, GB/s of each."""
    import torch

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    fa = sa.FlashAttnExt()
    res = {}
    for ql, q8 in OPERATING_POINTS:
        w = operating_point(ql, q8)
        dev = wl.to_device(wl.make_host(w))
        ms, per = time_calls(fa, w, dev, max(1, steps), warmup)
        r = summarize(w, ms, per)
        out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
        usg = _graph_us(lambda: fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"],
                                   mask_mode=w.mask_mode), max(40, steps), 3)
        r["us_graph"] = round(usg, 2)
        r["GBps_graph"] = round(w.bytes() / (usg * 1e-6) / 1e9, 1)
        res[w.name] = r
        _log(f"{w.name}: {r}")
        del dev
    print(json.dumps(res), flush=True)
    return 0


def q8_variant(name: str):
    """A config over a q8_0 cache (same seeds, lengths and heads)."""
    import dataclasses

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    return dataclasses.replace(wl.config(name), name=name + "_q8", kv_type=sa.TYPE_Q8_0)


def verify_q8_only(steps: int, warmup: int, head_dim: int = 128, q8: bool = True) -> int:
    """The 32 x 16 batched verify alone: a q8_0 cache at 128-dim heads, or 256-dim heads over
    an f16 or q8_0 cache."""
    import dataclasses

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    fa = sa.FlashAttnExt()
    w = batched_verify_q8() if head_dim == 128 else wl.config("batched_verify_d256")
    if q8:
        w = dataclasses.replace(w, kv_type=sa.TYPE_Q8_0)
    dev = wl.to_device(wl.make_host(w))
    ms, per = time_calls(fa, w, dev, max(1, steps), warmup)
    print(json.dumps({"workload": f"batched verify, {w.D}-dim heads, {'q8_0' if q8 else 'f16'} cache",
                      **summarize(w, ms, per)}), flush=True)
    return 0


def long_q8_only(steps: int, warmup: int) -> int:
    """The long-context q8_0 configurations alone: 8 streams x 64k cells of q8_0 KV, a decode
    (q_len 1) and an 8-row verify, one after the other, for the profiler."""
    import sixi_attn as sa
    from sixi_attn import workloads as wl

    fa = sa.FlashAttnExt()
    res = {}
    for name in ("long_q8_decode", "long_q8_verify"):
        w = wl.config(name)
        dev = wl.to_device(wl.make_host(w))
        ms, per = time_calls(fa, w, dev, max(1, steps), warmup)
        res[name] = summarize(w, ms, per)
    print(json.dumps({"workload": "8 streams x 65536 cells, q8_0 KV, 24 q-heads / 4 kv-heads x 128: q_len 1 and 8",
                      **res}), flush=True)
    return 0


def verify_mask_only(steps: int, warmup: int) -> int:
    """The 32 x 16 batched verify over the contiguous f16 cache with its block-causal mask handed
    over as llama.cpp's explicit f16 KQ mask (the ggml hook's call)."""
    import torch

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    fa = sa.FlashAttnExt()
    w = wl.config("batched_verify")
    dev = wl.to_device(wl.make_host(w))
    mask = torch.from_numpy(wl.kq_mask(dev["k"].shape[1], w.n_q, w.kv_len, w.q_len)).view(torch.float16).cuda()
    # the lengths-only call first, for comparison in the same trace
    ms0, per0 = time_calls(fa, w, dev, max(1, steps), warmup)
    ms, per = time_calls(fa, w, dev, max(1, steps), warmup, mask=mask)
    print(json.dumps({"workload": "batched verify, explicit llama mask, contiguous f16 cache",
                      **summarize(w, ms, per), "lengths_only": summarize(w, ms0, per0)}), flush=True)
    return 0


def prefill_only(steps: int, warmup: int, q8: bool = False, head_dim=None, bounded: bool = False,
                 explicit_mask: bool = False) -> int:
    import sixi_attn as sa

    fa = sa.FlashAttnExt()
    extra = {}
    if explicit_mask:
        # the lengths-only call first, for comparison in the same trace
        tf0, us0, _ = time_prefill(fa, max(1, steps), warmup)
        extra = {"lengths_only": {"us_two_chunks": round(us0, 2), "TFLOPs": round(tf0, 2)}}
    tf, us, wsb = time_prefill(fa, max(1, steps), warmup, kv_type=sa.TYPE_Q8_0 if q8 else None, head_dim=head_dim,
                               bounded=bounded, explicit_mask=explicit_mask)
    print(json.dumps({"workload": "prefill 4096 rows in two 2048-row chunks" + (" over a q8_0 cache" if q8 else "") +
                      (f", {head_dim}-dim heads" if head_dim else "") + (", bounded workspace" if bounded else "") +
                      (", explicit llama mask" if explicit_mask else ""),
                      "us_two_chunks": round(us, 2), "TFLOPs": round(tf, 2), "workspace_bytes": wsb, **extra}),
          flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="verify", choices=["verify", "copy", "prefill", "prefill_q8", "prefill_q8_bounded",
                                                               "prefill_d256_q8", "prefill_d256_q8_bounded", "layer",
                                                               "gdn", "verify_q8", "verify_d256", "verify_d256_q8", "verify_op",
                                                               "headline", "verify_mask", "prefill_mask", "long_q8"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="time only the headline workload")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs on a single MI355X (streams would shard "
              "across GPUs with no exchange, so N GPUs = N independent copies); run with --gpus 1",
              file=sys.stderr)
        return 2

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.workload == "copy":
        return copy_calibration(max(1, args.steps))
    if args.workload == "prefill_mask":
        return prefill_only(args.steps, args.warmup, explicit_mask=True)
    if args.workload == "verify_mask":
        return verify_mask_only(args.steps, args.warmup)
    if args.workload.startswith("prefill"):
        return prefill_only(args.steps, args.warmup, q8=args.workload != "prefill",
                            head_dim=256 if "d256" in args.workload else None,
                            bounded=args.workload.endswith("_bounded"))
    if args.workload == "layer":
        print(json.dumps(time_layer(max(8, args.steps), args.warmup)), flush=True)
        return 0
    if args.workload == "gdn":
        print(json.dumps(time_gdn(max(8, args.steps), args.warmup)), flush=True)
        return 0
    if args.workload == "verify_q8":
        return verify_q8_only(args.steps, args.warmup)
    if args.workload == "verify_op":
        return verify_op_only(args.steps, args.warmup)
    if args.workload == "headline":
        return headline_only(args.steps, args.warmup)
    if args.workload == "long_q8":
        return long_q8_only(args.steps, args.warmup)
    if args.workload.startswith("verify_d256"):
        return verify_q8_only(args.steps, args.warmup, head_dim=256, q8=args.workload.endswith("_q8"))

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    fa = sa.FlashAttnExt()
    props = torch.cuda.get_device_properties(0)
    _log(f"device {props.name} CUs={props.multi_processor_count}")

    w = wl.config("batched_verify")
    _log("generating batched_verify inputs")
    host = wl.make_host(w)
    dev = wl.to_device(host)
    _log(f"timing {args.steps} steps after {args.warmup} warm-up")
    out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    # the headline: the cache in the page pool's own layout (shuffled 256-cell pages, each page
    # head-major), read through the page table
    ms, per, n_pages = time_paged(fa, w, dev, args.steps, args.warmup, head_major=True, out=out)
    head = summarize(w, ms, per)
    gbs = head["GBps"]
    _log(f"verify: median {head['us_median']} us/call (mean {head['us']}), {gbs} GB/s, {head['TFLOPs']} TFLOP/s")
    gpu_out = out.cpu().numpy()

    traffic = traffic_from_profile()
    result = {
        "metric": METRIC,
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (PCG32 seed 0x51A70003, N(0,1))",
        "config": {
            "workload": "batched speculative verify: 32 streams x 16 rows, block-causal, cached lengths "
                        "U[512,16384] (seeded), 24 q-heads / 4 kv-heads x 128, f32 Q, f16 KV in the page pool: "
                        "256-cell pages at shuffled pool positions, read through the page table, each page "
                        "head-major ([kv-head][256 cells][128]); llama.cpp's token-major cells beside it "
                        "(verify_token_major_pages, verify_contiguous)",
            "streams": w.S, "rows_per_stream": 16, "mean_cached_len": round(sum(w.kv_len) / w.S, 1),
            "bytes_per_call": w.bytes(), "flops_per_call": w.flops(), "pool_pages": n_pages,
            "page_layout": "head-major",
        },
        "value_stat": "algorithmic bytes / the mean time of the steps bracketed by synchronisation "
                      "(ms_per_step); the per-call median and p10/p90 come from a second pass with an event "
                      "after every call (those events add ~2 us per call); before the warm-up steps the call "
                      f"runs untimed for {PRECONDITION_S * 1e3:.0f} ms so that the timed steps see the GPU's "
                      "settled clocks, not the power-management dip of calls ~11-100 after an idle period",
        "us_per_layer": head["us"],
        "us_per_layer_median": head["us_median"],
        "us_per_layer_p10_p50_p90": head["us_p10_p50_p90"],
        "workspace_bytes": ws_bytes(fa, w, dev),
        "verify_tflops": head["TFLOPs"],
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_wide<3,2,0,128> + decode_merge_rows<128> (one sixi_attn_forward call; "
                      "achieved = algorithmic bytes / call time)",
            "achieved": gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": f"{TRAFFIC_PROFILE.relative_to(ROOT)} (FETCH_SIZE + WRITE_SIZE of a separate "
                              "rocprofv3 --pmc run of this command, scaled by the copy calibration)",
        },
    }

    # the same verify with llama.cpp's token-major cell rows: in the page pool, and as one
    # contiguous cache per stream (the ggml hook's layout)
    msp, perp, _ = time_paged(fa, w, dev, max(20, args.steps // 2), max(5, args.warmup // 2), head_major=False)
    result["verify_token_major_pages"] = summarize(w, msp, perp)
    _log(f"verify, token-major pages: {result['verify_token_major_pages']}")
    msc, perc = time_calls(fa, w, dev, max(20, args.steps // 2), max(5, args.warmup // 2))
    result["verify_contiguous"] = summarize(w, msc, perc)
    _log(f"verify, contiguous token-major cache: {result['verify_contiguous']}")

    # the same verify with the block-causal mask handed over as an explicit ggml KQ mask (the
    # ggml FLASH_ATTN_EXT drop-in path)
    mask = torch.from_numpy(wl.kq_mask(dev["k"].shape[1], w.n_q, w.kv_len, w.q_len)).view(torch.float16).cuda()
    msm, perm = time_calls(fa, w, dev, max(20, args.steps // 2), max(5, args.warmup // 2), mask=mask)
    result["verify_explicit_mask"] = summarize(w, msm, perm)
    result["verify_explicit_mask"]["workspace_bytes"] = ws_bytes(fa, w, dev, mask=mask)
    _log(f"verify, explicit mask: {result['verify_explicit_mask']}")
    del mask

    if not args.no_extra:
        extra = {}
        op_names = {operating_point(ql, q8).name: (ql, q8) for ql, q8 in OPERATING_POINTS}
        for name in ("decode", "verify", "long_q8_decode", "long_q8_verify", "batched_verify_q8", "decode_d256",
                     "batched_verify_d256", "decode_d256_q8", "batched_verify_d256_q8", *op_names):
            try:
                if name in op_names:
                    we = operating_point(*op_names[name])
                elif name == "batched_verify_q8":
                    we = batched_verify_q8()
                elif name.endswith("_q8"):
                    we = q8_variant(name[:-3])
                else:
                    we = wl.config(name)
                he = wl.make_host(we)
                de = wl.to_device(he)
                mse, pere = time_calls(fa, we, de, max(20, args.steps // 2), max(5, args.warmup // 2))
                extra[name] = summarize(we, mse, pere)
                extra[name]["workspace_bytes"] = ws_bytes(fa, we, de)
                # the eager figure includes the host's issue time when a call is shorter than it
                # (decode); GPU time per call from HIP-graph replays of the same call
                oute = torch.empty((we.S, we.n_q, we.H, we.D), dtype=torch.float32, device="cuda")
                usg = _graph_us(lambda: fa(de["q"], de["k"], de["v"], oute, kv_len=de["kv_len"], q_len=de["q_len"],
                                           mask_mode=we.mask_mode), max(40, args.steps // 2), 3)
                extra[name]["us_graph"] = round(usg, 2)
                extra[name]["GBps_graph"] = round(we.bytes() / (usg * 1e-6) / 1e9, 1)
                # the same call with its block-causal mask as llama.cpp's explicit f16 KQ mask
                # (the ggml hook's call: the mask pre-pass, then the kernels it chooses between)
                me = torch.from_numpy(wl.kq_mask(de["k"].shape[1], we.n_q, we.kv_len, we.q_len)).view(
                    torch.float16).cuda()
                usm = _graph_us(lambda: fa(de["q"], de["k"], de["v"], oute, kv_len=de["kv_len"], q_len=de["q_len"],
                                           mask_mode=sa.MASK_EXPLICIT, mask=me), max(40, args.steps // 2), 3)
                extra[name]["us_graph_explicit_mask"] = round(usm, 2)
                del de, me
            except sa.SixiAttnError as e:
                extra[name] = {"unavailable": str(e)}
            _log(f"{name}: {extra[name]}")
        result["configs"] = extra
        # the KV-cache store that precedes each verify call (block rows of all streams)
        try:
            result["kv_store"] = time_kv_store(w, dev, max(20, args.steps // 2), max(5, args.warmup // 2))
        except sa.SixiAttnError as e:
            result["kv_store"] = {"unavailable": str(e)}
        _log(f"kv_store: {result['kv_store']}")
        # the Q/K prologue with the KV store, and the output gate, of a 256-dim layer
        try:
            result["layer_prologue_gate"] = time_layer(max(40, args.steps // 2), max(5, args.warmup // 2))
        except sa.SixiAttnError as e:
            result["layer_prologue_gate"] = {"unavailable": str(e)}
        _log(f"layer prologue/gate: {result['layer_prologue_gate']}")
        # the gated-delta-rule verify of one linear-attention layer
        try:
            result["gdn_verify"] = time_gdn(max(40, args.steps // 2), max(5, args.warmup // 2))
        except sa.SixiAttnError as e:
            result["gdn_verify"] = {"unavailable": str(e)}
        _log(f"gdn verify: {result['gdn_verify']}")

        # chunked causal prefill (2 chunks of 2048 rows on a 2048-cell cache)
        try:
            tf, us, wsb = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4))
            result["prefill_workspace_bytes"] = wsb
            result["prefill_tflops"] = round(tf, 2)
            result["prefill_us_two_chunks"] = round(us, 2)
            result["prefill_roofline"] = {"bound": "mfma", "achieved": round(tf, 2), "peak": F16_PEAK_TFLOPS,
                                          "unit": "TFLOP/s", "frac": round(tf / F16_PEAK_TFLOPS, 4)}
            _log(f"prefill: {us:.1f} us for 2 chunks, {tf:.1f} TFLOP/s")
            tq, uq, wsq = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4), kv_type=sa.TYPE_Q8_0)
            result["configs"]["prefill_q8_0"] = {"us_two_chunks": round(uq, 2), "TFLOPs": round(tq, 2),
                                                 "workspace_bytes": wsq, "path": "f16 staging"}
            _log(f"prefill q8_0 KV: {uq:.1f} us for 2 chunks, {tq:.1f} TFLOP/s")
            tqb, uqb, wsqb = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4), kv_type=sa.TYPE_Q8_0,
                                          bounded=True)
            result["configs"]["prefill_q8_0_bounded"] = {"us_two_chunks": round(uqb, 2), "TFLOPs": round(tqb, 2),
                                                         "workspace_bytes": wsqb, "path": "q8_0 tiles converted in LDS"}
            _log(f"the same with a bounded workspace: {uqb:.1f} us for 2 chunks, {tqb:.1f} TFLOP/s")
            td, ud, wsd = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4), head_dim=256)
            result["configs"]["prefill_d256"] = {"us_two_chunks": round(ud, 2), "TFLOPs": round(td, 2),
                                                 "workspace_bytes": wsd}
            _log(f"prefill 256-dim heads: {ud:.1f} us for 2 chunks, {td:.1f} TFLOP/s")
            tdq, udq, wsdq = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4), kv_type=sa.TYPE_Q8_0,
                                          head_dim=256)
            result["configs"]["prefill_d256_q8_0"] = {"us_two_chunks": round(udq, 2), "TFLOPs": round(tdq, 2),
                                                      "workspace_bytes": wsdq, "path": "f16 staging"}
            _log(f"prefill 256-dim heads over q8_0 KV: {udq:.1f} us for 2 chunks, {tdq:.1f} TFLOP/s")
            tdb, udb, wsdb = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4), kv_type=sa.TYPE_Q8_0,
                                          head_dim=256, bounded=True)
            result["configs"]["prefill_d256_q8_0_bounded"] = {"us_two_chunks": round(udb, 2), "TFLOPs": round(tdb, 2),
                                                              "workspace_bytes": wsdb, "path": "q8_0 tiles converted in LDS"}
            _log(f"the same with a bounded workspace: {udb:.1f} us for 2 chunks, {tdb:.1f} TFLOP/s")
            tm, um, wsm = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4), explicit_mask=True)
            result["configs"]["prefill_explicit_mask"] = {"us_two_chunks": round(um, 2), "TFLOPs": round(tm, 2),
                                                          "workspace_bytes": wsm}
            _log(f"prefill with the causal mask as an explicit ggml mask: {um:.1f} us for 2 chunks, {tm:.1f} TFLOP/s")
            tmd, umd, wsmd = time_prefill(fa, max(10, args.steps // 4), max(3, args.warmup // 4), head_dim=256,
                                          explicit_mask=True)
            result["configs"]["prefill_d256_explicit_mask"] = {"us_two_chunks": round(umd, 2), "TFLOPs": round(tmd, 2),
                                                               "workspace_bytes": wsmd}
            _log(f"the same at 256-dim heads: {umd:.1f} us for 2 chunks, {tmd:.1f} TFLOP/s")
        except sa.SixiAttnError as e:
            result["prefill_tflops"] = None
            result["prefill_note"] = f"prefill kernel unavailable: {e}"
            _log(result["prefill_note"])

    if not args.no_cpu:
        _log("CPU baseline (oracle on host cores)")
        result["cpu_baseline"] = cpu_baseline(w, host, gpu_out)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
