"""Benchmark of the MI355X attention hot path (one GPU).

Workload (the headline): batched speculative verify -- 32 streams x 16 drafted rows,
block-causal, per-stream cached lengths drawn from [512, 16384] (mean ~8.4k), 24/4 heads x
128, f16 KV in per-stream 256-cell pages, f32 Q -- one attention layer per step.  The
chunked causal prefill (2 x 2048-row chunks over a 2048-cell cache, f16) is timed beside it
when its kernel is built.

Prints one JSON line: value = algorithmic HBM GB/s of the verify call (K/V of every attended
cell + Q + O, counted once) with inputs resident in HBM; roofline = that rate against the
8 TB/s HBM peak; cpu_baseline = the oracle (a restatement of ggml's CPU flash_attn_ext,
f16 V accumulator as upstream) on the host cores, same inputs.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "sixi-asi_amd"))

METRIC = "verify-attn µs/layer & HBM GB/s (32 streams×16 tok, 8k ctx); prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2500.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_calls(fa, w, dev, steps: int, warmup: int):
    """Per-call GPU time with events on the stream the library launches on."""
    import torch

    import sixi_attn as sa

    out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    def call():
        fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"],
           mask_mode=sa.MASK_BLOCK_CAUSAL, stream=stream.cuda_stream)

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        call()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    total = ev[0].elapsed_time(ev[steps])
    return total / steps, per


def cpu_baseline(w, host, budget_s: float = 15.0) -> dict:
    """The oracle on the host cores over a bounded sample of the same workload."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import numpy as np

    import oracle

    threads = oracle.cpu_threads()
    lens = np.array(w.kv_len)
    order = list(np.argsort(np.abs(lens - lens.mean())))  # streams nearest the mean first
    t0 = time.perf_counter()
    oracle.attention_for_workload(host, w.kv_type, order[:1], v_acc_f16=True, n_threads=threads)
    one = time.perf_counter() - t0
    n = int(max(1, min(w.S, budget_s / max(one, 1e-3))))
    sample = sorted(order[:n])
    t0 = time.perf_counter()
    oracle.attention_for_workload(host, w.kv_type, sample, v_acc_f16=True, n_threads=threads)
    dt = time.perf_counter() - t0
    sub = type(w)(w.name, w.seed, len(sample), [w.kv_len[i] for i in sample], [w.q_len[i] for i in sample],
                  H=w.H, Hkv=w.Hkv, D=w.D, kv_type=w.kv_type, q_type=w.q_type)
    return {
        "value": round(sub.bytes() / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(sample)} of {w.S} streams ({sum(sub.kv_len)} cached cells, {sum(sub.q_len)} rows),"
                  f" f16 V accumulator, {dt:.2f} s",
        "us_per_call_sample": round(dt * 1e6, 1),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the attention path has no multi-GPU mode "
              "(streams would shard across GPUs with no exchange); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import sixi_attn as sa
    from sixi_attn import workloads as wl

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    fa = sa.FlashAttnExt()
    props = torch.cuda.get_device_properties(0)
    _log(f"device {props.name} CUs={props.multi_processor_count}")

    w = wl.config("batched_verify")
    _log("generating batched_verify inputs")
    host = wl.make_host(w)
    dev = wl.to_device(host)
    _log(f"timing {args.steps} steps after {args.warmup} warm-up")
    ms, per = time_calls(fa, w, dev, args.steps, args.warmup)
    per_sorted = sorted(per)
    med = per_sorted[len(per) // 2]
    gbs = w.bytes() / (ms * 1e-3) / 1e9
    tflops = w.flops() / (ms * 1e-3) / 1e12
    _log(f"verify: {ms * 1e3:.1f} us/call, {gbs:.0f} GB/s, {tflops:.1f} TFLOP/s")

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
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
                        "U[512,16384] (seeded), 24 q-heads / 4 kv-heads x 128, f16 KV in 256-cell pages, f32 Q",
            "streams": w.S, "rows_per_stream": 16, "mean_cached_len": round(sum(w.kv_len) / w.S, 1),
            "bytes_per_call": w.bytes(), "flops_per_call": w.flops(),
        },
        "us_per_layer": round(ms * 1e3, 2),
        "us_per_layer_p10_p50_p90": [round(per_sorted[len(per) // 10] * 1e3, 2), round(med * 1e3, 2),
                                     round(per_sorted[(9 * len(per)) // 10] * 1e3, 2)],
        "verify_tflops": round(tflops, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "splitk_f16_d128 + splitk_merge_d128 (one verify call)",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
    }

    # chunked causal prefill (2 chunks of 2048 rows), when its kernel is available
    try:
        pre = []
        for name in ("prefill_chunk0", "prefill_chunk1"):
            wp = wl.config(name)
            hp = wl.make_host(wp)
            dp = wl.to_device(hp)
            msp, _ = time_calls(fa, wp, dp, max(10, args.steps // 4), max(3, args.warmup // 4))
            pre.append((wp, msp))
        flops = sum(wp.flops() for wp, _ in pre)
        t = sum(msp for _, msp in pre)
        tf = flops / (t * 1e-3) / 1e12
        result["prefill_tflops"] = round(tf, 2)
        result["prefill_us_two_chunks"] = round(t * 1e3, 2)
        result["prefill_roofline"] = {"bound": "mfma", "achieved": round(tf, 2), "peak": F16_PEAK_TFLOPS,
                                      "unit": "TFLOP/s", "frac": round(tf / F16_PEAK_TFLOPS, 4)}
        _log(f"prefill: {t * 1e3:.1f} us for 2 chunks, {tf:.1f} TFLOP/s")
    except sa.SixiAttnError as e:
        result["prefill_tflops"] = None
        result["prefill_note"] = f"prefill kernel unavailable: {e}"
        _log(result["prefill_note"])

    if not args.no_cpu:
        _log("CPU baseline (oracle on host cores)")
        result["cpu_baseline"] = cpu_baseline(w, host)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
