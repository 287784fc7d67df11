"""sixi_attn_forward_noalloc against sixi_attn_forward, through the C ABI.

The no-allocation entry point runs the same kernels on the library's fixed device scratch
instead of a caller workspace.  Two calls in a row, the second with a smaller input (so the
scratch still holds the first call's partials), each bitwise equal to sixi_attn_forward on
the same inputs and within the oracle bar; a description whose scratch exceeds the fixed size
is rejected before any launch and leaves the output untouched.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

import oracle
import sixi_attn as sa
from sixi_attn import workloads as wl

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
REL_L2 = 1e-3


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def fa():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    sa.load_library()
    return sa.FlashAttnExt()


def _both(fa, w, host):
    dev = wl.to_device(host)
    outs = []
    for noalloc in (False, True):
        out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
        p = fa.params(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"])
        p.stream = torch.cuda.current_stream().cuda_stream
        if noalloc:
            rc = fa.lib.sixi_attn_forward_noalloc(ctypes.byref(p))
        else:
            ws = torch.empty(fa.workspace_bytes(p), dtype=torch.uint8, device="cuda")
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
            rc = fa.lib.sixi_attn_forward(ctypes.byref(p))
        assert rc == sa.OK, sa.strerror(rc)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    return outs


def _against_oracle(w, host, got):
    want = oracle.attention_for_workload(host, w.kv_type)
    for s in range(w.S):
        ql = w.q_len[s]
        m = oracle.diff_metrics(want[s, :ql], got[s, :ql])
        assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (s, m)


def test_noalloc_matches_forward_on_two_calls():
    fa = sa.FlashAttnExt()
    # first: the 32-stream x 16-row verify (96 rows per group on the 32-cell kernel)
    w1 = wl.config("batched_verify")
    _say("no-alloc call 1: batched verify, 32 streams x 16 rows")
    h1 = wl.make_host(w1, poison=True)
    ref1, got1 = _both(fa, w1, h1)
    assert np.array_equal(ref1, got1, equal_nan=True)
    _against_oracle(w1, h1, got1)
    # second, smaller: 3 streams of 256-dim heads, 48 rows per group (64-row slots)
    w2 = wl.Workload("noalloc small", 0x51A7_C000, 3, [900, 40, 3000], [8, 3, 6], D=256)
    _say("no-alloc call 2: 3 streams, 256-dim heads, up to 48 rows")
    h2 = wl.make_host(w2, poison=True)
    ref2, got2 = _both(fa, w2, h2)
    assert np.array_equal(ref2, got2, equal_nan=True)
    _against_oracle(w2, h2, got2)


def test_noalloc_q8_0_96_rows():
    """q8_0 at 96 rows per group: one launch of the 32-cell q8_0 kernel and its merge on the
    scratch (every head of a group rides along with each tile)."""
    fa = sa.FlashAttnExt()
    w = wl.Workload("noalloc q8", 0x51A7_C100, 4, [5000, 12, 800, 2000], [16, 16, 5, 9], kv_type=sa.TYPE_Q8_0)
    _say("no-alloc: q8_0, 96 rows per group")
    h = wl.make_host(w, poison=True)
    ref, got = _both(fa, w, h)
    assert np.array_equal(ref, got, equal_nan=True)
    _against_oracle(w, h, got)


def test_noalloc_q8_0_prefill_at_256_dims_converts_in_lds():
    """A 256-dim q8_0 prefill whose f16 staging (2 streams x 7000 cells: 57 MB) would not fit
    the fixed scratch: the no-allocation call converts the q8_0 tiles in LDS instead, while
    sixi_attn_forward stages them (under its cap); the two give the same operands, so the
    outputs agree bitwise."""
    fa = sa.FlashAttnExt()
    w = wl.Workload("noalloc q8 d256 prefill", 0x51A7_C200, 2, [6800, 5000], [200, 130], D=256,
                    kv_type=sa.TYPE_Q8_0)
    _say("no-alloc: q8_0 prefill, 256-dim heads, staging beyond the scratch")
    h = wl.make_host(w, poison=True)
    ref, got = _both(fa, w, h)
    for s in range(w.S):
        assert np.array_equal(ref[s, :w.q_len[s]], got[s, :w.q_len[s]]), s
    _against_oracle(w, h, got)


def test_noalloc_rejects_a_scratch_beyond_the_fixed_size():
    """512 streams of 256-dim heads at 96 rows per group need (2048 + groups) slots of 49920 B,
    more than the fixed scratch: rejected before any launch, output untouched."""
    fa = sa.FlashAttnExt()
    S, n_q, H, Hkv, D, n_kv = 512, 16, 24, 4, 256, 32
    q = torch.zeros((S, n_q, H, D), dtype=torch.float16, device="cuda")
    k = torch.zeros((S, n_kv, Hkv, D), dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    kl = torch.full((S,), n_kv - n_q, dtype=torch.int32, device="cuda")
    out = torch.full((S, n_q, H, D), 7.0, dtype=torch.float32, device="cuda")
    _say("no-alloc: oversize description")
    rc = fa(q, k, v, out, kv_len=kl, noalloc=True, check=False)
    assert rc == sa.E_OUT_OF_BOUNDS
    torch.cuda.synchronize()
    assert bool(torch.all(out == 7.0))
