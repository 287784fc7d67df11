"""Edge shapes of the split-K path against the oracle, through the C ABI: a stream with no rows,
the largest stream count the library takes (512), and a 64k-cell f16 context."""
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


def _run(fa, w, dev):
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"])
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(w, host, got, streams, label):
    sub = {k: (v[streams] if k in ("q", "k", "v", "kv_len", "q_len") else v) for k, v in host.items()}
    want = oracle.attention_for_workload(sub, w.kv_type)
    ql = host["q_len"]
    g = np.concatenate([got[s, :ql[s]].ravel() for s in streams])
    r = np.concatenate([want[i, :ql[s]].ravel() for i, s in enumerate(streams)])
    m = oracle.diff_metrics(r, g)
    _say(f"{label}: max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(g))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m


@pytest.mark.parametrize("q_len", [[16, 0, 5, 0], [1, 0, 1, 1], [0, 8, 0, 0]])
def test_streams_without_rows_are_left_untouched(fa, q_len):
    w = wl.Workload("no rows", 0x51A7_A000 + sum(q_len), 4, [300, 1200, 0, 77], q_len)
    _say(f"streams without rows: q_len {q_len}")
    host = wl.make_host(w, poison=True)
    got = _run(fa, w, wl.to_device(host))
    assert np.all(np.isnan(got[[s for s in range(w.S) if q_len[s] == 0]]))
    _check(w, host, got, [s for s in range(w.S) if q_len[s] > 0], f"q_len {q_len}")


def test_largest_stream_count(fa):
    S = 512  # the library's stream bound (LDS extents table)
    rng = np.random.default_rng(7)
    kv_len = [int(x) for x in rng.integers(0, 300, S)]
    q_len = [int(x) for x in rng.integers(1, 17, S)]
    w = wl.Workload("512 streams", 0x51A7_A100, S, kv_len, q_len)
    _say(f"{S} streams, kv_len <= 300, q_len 1..16")
    host = wl.make_host(w, poison=True)
    got = _run(fa, w, wl.to_device(host))
    picks = [0, 1, 77, 255, 256, 400, 510, 511]
    _check(w, host, got, picks, "512 streams (8 checked)")
    ql = host["q_len"]
    assert all(np.all(np.isfinite(got[s, :ql[s]])) for s in range(S))


def test_64k_cell_context(fa):
    w = wl.Workload("64k", 0x51A7_A200, 2, [65536 - 16, 40000], [16, 9])
    _say("64k-cell f16 context, 96 and 54 rows")
    host = wl.make_host(w, poison=True)
    got = _run(fa, w, wl.to_device(host))
    _check(w, host, got, [0, 1], "64k context")
