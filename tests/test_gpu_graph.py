"""The library's calls inside a captured HIP graph: the library issues kernel launches only (no memset,
no allocation), so a replayed graph must reproduce the eager result.  Each graph is replayed several
times with eager work and synchronisation between the replays, and every replay is compared bitwise
with the eager call (every kernel here is deterministic: fixed reduction orders, no atomics).
"""
import sys

import pytest
import torch

import sixi_attn as sa
from sixi_attn import workloads as wl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def lib():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    return sa.load_library()


def _replays(fn, outputs, reps=3):
    """Eager result of fn, then `reps` replays of its captured graph, each checked bitwise.  The
    outputs are cleared before every run, so rows a call leaves unwritten compare equal too."""
    for o in outputs:
        o.zero_()
    fn()
    torch.cuda.synchronize()
    want = [o.clone() for o in outputs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for r in range(reps):
        for o in outputs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outputs, want)):
            assert torch.equal(o, w), f"replay {r}: output {i} differs from the eager call"
        _ = torch.ones(1024, device="cuda").sum().item()   # eager work between replays


def test_verify_step_graph():
    """KV store -> attention, the verify batch's shapes (32 streams x 16 rows)."""
    w = wl.config("batched_verify")
    _say(f"graph: verify step S={w.S} rows={w.n_q}")
    host = wl.make_host(w)
    dev = wl.to_device(host)
    fa = sa.FlashAttnExt()
    src_k = torch.randn((w.S, w.n_q, w.Hkv, w.D), device="cuda")
    src_v = torch.randn_like(src_k)
    out = torch.empty((w.S, w.n_q, w.H, w.D), device="cuda")

    def step():
        sa.kv_write(src_k, dev["k"], dev["kv_len"], dev["q_len"])
        sa.kv_write(src_v, dev["v"], dev["kv_len"], dev["q_len"])
        fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"])

    _replays(step, [out])


def test_layer_graph():
    """Prologue -> attention -> gate at the Qwen geometry (256-dim heads), f16 and q8_0 caches."""
    S, R, H, Hkv, D, n_cells = 4, 16, 24, 4, 256, 1040
    kv_len = torch.tensor([1000, 3, 517, 64], dtype=torch.int32, device="cuda")
    q_len = torch.tensor([16, 16, 5, 1], dtype=torch.int32, device="cuda")
    qg = torch.randn((S, R, H, 2 * D), device="cuda")
    k = torch.randn((S, R, Hkv, D), device="cuda")
    v = torch.randn_like(k)
    wq = torch.rand(D, device="cuda") + 0.5
    wk = torch.rand(D, device="cuda") + 0.5
    q = torch.zeros((S, R, H, D), device="cuda")
    fa = sa.FlashAttnExt()
    for q8 in (False, True):
        _say(f"graph: layer prologue/attention/gate q8={q8}")
        if q8:
            kc = torch.zeros((S, n_cells, Hkv, D // 32 * 34), dtype=torch.uint8, device="cuda")
        else:
            kc = (torch.randn((S, n_cells, Hkv, D), device="cuda") * 0.5).half()
        vc = kc.clone()
        out = torch.empty((S, R, H, D), device="cuda")

        def layer():
            sa.qk_prologue(qg, k, v, wq, wk, q, kc, vc, kv_len, q_len)
            fa(q, kc, vc, out, kv_len=kv_len, q_len=q_len)
            sa.attn_gate(out, qg, q_len)

        fa(q, kc, vc, out, kv_len=kv_len, q_len=q_len)   # size the workspace before capture
        _replays(layer, [q, out])


def test_masked_calls_graph():
    """llama-mask calls (the ggml hook): the mask pre-pass and the dual kernels of a verify batch,
    the prefill pair, and single-stream decode (no pre-pass) replay the eager result."""
    fa = sa.FlashAttnExt()
    for name, kv_len, q_len in (("verify", [900, 5000, 37, 2000], [16, 16, 9, 16]),
                                ("prefill", [200, 700], [150, 260]),
                                ("decode", [4096], [1])):
        w = wl.Workload(f"graph mask {name}", 0x51A7_B000 + len(name), len(kv_len), kv_len, q_len)
        dev = wl.to_device(wl.make_host(w))
        mask = torch.from_numpy(wl.kq_mask(dev["k"].shape[1], w.n_q, w.kv_len, w.q_len)).view(torch.float16).cuda()
        out = torch.empty((w.S, w.n_q, w.H, w.D), device="cuda")
        _say(f"graph: {name} with the llama mask S={w.S} rows={w.n_q}")

        def call():
            fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"],
               mask_mode=sa.MASK_EXPLICIT, mask=mask)

        _replays(call, [out])


def test_layer_graph_fused_gate():
    """Prologue -> attention with the output gate fused (SIXI_ATTN_FLAG_GATE) replays the eager
    result, which equals the three-call layer bit for bit."""
    S, R, H, Hkv, D, n_cells = 4, 16, 24, 4, 256, 1040
    kv_len = torch.tensor([1000, 3, 517, 64], dtype=torch.int32, device="cuda")
    q_len = torch.tensor([16, 16, 5, 1], dtype=torch.int32, device="cuda")
    qg = torch.randn((S, R, H, 2 * D), device="cuda")
    k = torch.randn((S, R, Hkv, D), device="cuda")
    v = torch.randn_like(k)
    wq = torch.rand(D, device="cuda") + 0.5
    wk = torch.rand(D, device="cuda") + 0.5
    q = torch.zeros((S, R, H, D), device="cuda")
    kc = (torch.randn((S, n_cells, Hkv, D), device="cuda") * 0.5).half()
    vc = kc.clone()
    out = torch.empty((S, R, H, D), device="cuda")
    fa = sa.FlashAttnExt()
    _say("graph: layer prologue/attention with the fused gate")

    def layer():
        sa.qk_prologue(qg, k, v, wq, wk, q, kc, vc, kv_len, q_len)
        fa(q, kc, vc, out, kv_len=kv_len, q_len=q_len, gate=qg)

    fa(q, kc, vc, out, kv_len=kv_len, q_len=q_len, gate=qg)   # size the workspace before capture
    _replays(layer, [q, out])
    fused = out.clone()
    out.zero_()
    sa.qk_prologue(qg, k, v, wq, wk, q, kc, vc, kv_len, q_len)
    fa(q, kc, vc, out, kv_len=kv_len, q_len=q_len)
    sa.attn_gate(out, qg, q_len)
    torch.cuda.synchronize()
    assert torch.equal(out, fused)


def test_gdn_graph():
    """GDN verify out of place (the input state stays fixed, so every replay has the same input);
    16 streams x 48 groups = 1536 items, more than the work-groups that fit at once, so the
    captured launch runs several items per work-group."""
    S, n, G, K, HD = 16, 16, 48, 128, 128
    _say(f"graph: gdn S={S} n={n} G={G}")
    q = torch.randn((S, n, G, K), device="cuda") / K ** 0.5
    k = torch.nn.functional.normalize(torch.randn((S, n, G, K), device="cuda"), dim=-1)
    v = torch.randn((S, n, G, HD), device="cuda")
    al = torch.rand((S, n, G), device="cuda") * 0.2 + 0.8
    be = torch.rand((S, n, G), device="cuda")
    st_in = torch.randn((S, G, HD, K), device="cuda")
    st_out = torch.empty_like(st_in)
    y = torch.zeros((S, n, G, HD), device="cuda")
    q_len = torch.tensor([16, 9, 1, 16, 0, 4, 16, 12] * 2, dtype=torch.int32, device="cuda")
    snap = torch.tensor([16, 3, 1, 0, 0, 4, 8, 12] * 2, dtype=torch.int32, device="cuda")

    def run():
        sa.gdn_verify(q, k, v, al, be, y, st_in, st_out, q_len, snap)

    _replays(run, [st_out, y])
    assert torch.all(torch.isfinite(y[0])) and torch.all(y[4] == 0)   # stream 4 has no rows


def _noalloc_call(fa, dev, out, w, stream):
    import ctypes

    p = fa.params(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"],
                  mask_mode=w.mask_mode)
    p.stream = stream
    rc = fa.lib.sixi_attn_forward_noalloc(ctypes.byref(p))
    assert rc == sa.OK, sa.strerror(rc)


def test_noalloc_graph():
    """The no-allocation entry point captured and replayed: every replay bitwise equal to the
    eager sixi_attn_forward call (the scratch's device address is looked up once per device,
    outside any stream work, and the kernels take it as an argument)."""
    w = wl.Workload("graph noalloc", 0x51A7_C300, 5, [3000, 17, 900, 6000, 255], [16, 3, 16, 9, 1])
    _say(f"graph: no-allocation verify S={w.S}")
    dev = wl.to_device(wl.make_host(w))
    fa = sa.FlashAttnExt()
    out = torch.empty((w.S, w.n_q, w.H, w.D), device="cuda")
    ref = torch.empty_like(out)
    ref.zero_()
    fa(dev["q"], dev["k"], dev["v"], ref, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=w.mask_mode)
    torch.cuda.synchronize()
    _replays(lambda: _noalloc_call(fa, dev, out, w, torch.cuda.current_stream().cuda_stream), [out])
    out.zero_()
    _noalloc_call(fa, dev, out, w, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


_FIRST_CALL_CHILD = r'''
import ctypes, sys
sys.path[:0] = [sys.argv[1]]
import torch
import sixi_attn as sa
from sixi_attn import workloads as wl
w = wl.Workload("graph noalloc first", 0x51A7_C301, 3, [2500, 40, 700], [16, 5, 12])
dev = wl.to_device(wl.make_host(w))
fa = sa.FlashAttnExt()
out = torch.zeros((w.S, w.n_q, w.H, w.D), device="cuda")
ref = torch.zeros_like(out)
side = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=side):   # the process's first no-allocation call
    p = fa.params(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=w.mask_mode)
    p.stream = side.cuda_stream
    rc = fa.lib.sixi_attn_forward_noalloc(ctypes.byref(p))
assert rc == sa.OK, sa.strerror(rc)
fa(dev["q"], dev["k"], dev["v"], ref, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=w.mask_mode)
torch.cuda.synchronize()
for r in range(3):
    out.zero_()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"replay {r}"
    _ = torch.ones(1024, device="cuda").sum().item()
print("first-call capture ok", flush=True)
'''


def test_noalloc_first_call_under_capture_in_a_fresh_process():
    """In a fresh process, the first no-allocation call (which looks up the scratch's device
    address) is made under graph capture; its replays equal the eager call bitwise."""
    import pathlib
    import subprocess

    _say("graph: first no-allocation call captured, child process")
    pkg = str(pathlib.Path(sa.__file__).resolve().parent.parent)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CHILD, pkg], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "first-call capture ok" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-4000:])
