"""Workspace contents and non-finite inputs.

* The workspace needs no initialisation (include/sixi_attn.h): a call whose workspace is
  filled with NaN bit patterns gives bitwise the output of a call with a zeroed one, on every
  kernel path (16-cell and 32-cell split-K with either merge, 256-dim heads, the 16-cell and
  32-cell q8_0 split-K kernels, the q8_0 staging, the prefill kernel), and two calls in a row
  agree.
* Non-finite inputs give the oracle's result.  ggml's CPU kernel propagates a NaN score or V
  value through its online softmax: a row whose Q holds NaN or Inf is NaN in every dim; NaN in
  the K of a cell a row sees makes that row NaN; NaN in dim d of the V of a cell a row sees
  makes dim d of that row NaN.  Every other output keeps its bits.
"""
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


def _call(fa, w, dev, ws, q=None, k=None, v=None):
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    fa(dev["q"] if q is None else q, dev["k"] if k is None else k, dev["v"] if v is None else v, out,
       kv_len=dev["kv_len"], q_len=dev["q_len"], workspace=ws)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _ws_bytes(fa, w, dev):
    out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    return fa.workspace_bytes(fa.params(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"]))


@pytest.mark.parametrize("label,kv_len,q_len,H,Hkv,D,kv_type", [
    ("16-cell split-K, row merge", [700, 3000, 41], [5, 8, 1], 24, 4, 128, sa.TYPE_F16),
    ("16-cell split-K, piece merge", [30000], [3], 24, 4, 128, sa.TYPE_F16),
    ("32-cell split-K, 96 rows", [5000, 900, 12000], [16, 9, 16], 24, 4, 128, sa.TYPE_F16),
    ("32-cell split-K, piece merge", [40000], [16], 24, 4, 128, sa.TYPE_F16),
    ("256-dim heads, 48 rows", [6000, 333], [8, 6], 24, 4, 256, sa.TYPE_F16),
    ("q8_0 split-K", [4000, 64], [8, 3], 24, 4, 128, sa.TYPE_Q8_0),
    ("q8_0 96 rows, 32-cell kernel", [4000, 900], [16, 12], 24, 4, 128, sa.TYPE_Q8_0),
    ("q8_0 prefill", [300, 1000], [200, 130], 24, 4, 128, sa.TYPE_Q8_0),
    ("q8_0 prefill, 256-dim heads", [300, 1000], [200, 130], 24, 4, 256, sa.TYPE_Q8_0),
    ("prefill kernel", [100, 1500], [300, 129], 24, 4, 128, sa.TYPE_F16),
])
def test_nan_filled_workspace_changes_nothing(fa, label, kv_len, q_len, H, Hkv, D, kv_type):
    w = wl.Workload("ws", 0x51A7_B000 + sum(kv_len) + D, len(kv_len), kv_len, q_len, H=H, Hkv=Hkv, D=D,
                    kv_type=kv_type)
    _say(f"workspace poison: {label}")
    dev = wl.to_device(wl.make_host(w, poison=True))
    n = _ws_bytes(fa, w, dev)
    ws_zero = torch.zeros(n, dtype=torch.uint8, device="cuda")
    ws_nan = torch.full((n,), 0xFF, dtype=torch.uint8, device="cuda")  # NaN as f16 and as f32
    clean = _call(fa, w, dev, ws_zero)
    poisoned = _call(fa, w, dev, ws_nan)
    assert np.array_equal(clean, poisoned, equal_nan=True)
    again = _call(fa, w, dev, ws_nan)  # the workspace now holds the previous call's partials
    assert np.array_equal(clean, again, equal_nan=True)
    for s in range(w.S):
        assert np.all(np.isfinite(clean[s, :w.q_len[s]]))


def _nonfinite_case():
    w = wl.Workload("nonfinite", 0x51A7_B100, 3, [300, 2000, 45], [16, 7, 12])
    host = wl.make_host(w, poison=True)
    return w, host


def _compare_with_oracle(w, host, got, label):
    want = oracle.attention_for_workload(host, w.kv_type)
    for s in range(w.S):
        ql = w.q_len[s]
        g, r = got[s, :ql], want[s, :ql]
        assert np.array_equal(np.isnan(g), np.isnan(r)), (label, s)
        fin = np.isfinite(r)
        assert np.all(np.isfinite(g[fin]))
        if fin.any():
            m = oracle.diff_metrics(r[fin], g[fin])
            assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (label, s, m)
    return want


def test_non_finite_queries(fa):
    w, host = _nonfinite_case()
    dev = wl.to_device(host)
    n = _ws_bytes(fa, w, dev)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    base = _call(fa, w, dev, ws)
    bad = [(0, 3, 7, np.nan), (1, 0, 20, np.inf), (2, 11, 0, -np.inf)]  # (stream, row, head, value)
    h2 = dict(host)
    h2["q"] = host["q"].copy()
    for s, j, h, x in bad:
        h2["q"][s, j, h, 5] = x
    _say("NaN / Inf in Q")
    got = _call(fa, w, dev, ws, q=torch.from_numpy(h2["q"]).cuda())
    _compare_with_oracle(w, h2, got, "non-finite Q")
    for s, j, h, _ in bad:
        assert np.all(np.isnan(got[s, j, h]))
    keep = np.ones(got.shape, dtype=bool)
    for s, j, h, _ in bad:
        keep[s, j, h] = False
    assert np.array_equal(got[keep], base[keep], equal_nan=True)


def test_nan_in_cached_key_and_value(fa):
    """Cached cells (below kv_len) are seen by every row of the stream."""
    w, host = _nonfinite_case()
    dev = wl.to_device(host)
    n = _ws_bytes(fa, w, dev)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    base = _call(fa, w, dev, ws)
    h2 = dict(host)
    h2["k"] = host["k"].copy()
    h2["v"] = host["v"].copy()
    h2["k"][1, 1500, 2, 9] = 0x7E00   # stream 1, kv-head 2: heads 12..17 NaN in every dim
    h2["v"][0, 17, 0, 5] = 0x7E00     # stream 0, kv-head 0: dim 5 of heads 0..5 NaN
    _say("NaN in a cached K and a cached V cell")
    got = _call(fa, w, dev, ws, k=torch.from_numpy(h2["k"]).view(torch.float16).cuda(),
                v=torch.from_numpy(h2["v"]).view(torch.float16).cuda())
    _compare_with_oracle(w, h2, got, "NaN cached K/V")
    assert np.all(np.isnan(got[1, :7, 12:18]))
    assert np.all(np.isnan(got[0, :16, 0:6, 5]))
    keep = np.ones(got.shape, dtype=bool)
    keep[1, :, 12:18] = False
    keep[0, :, 0:6, 5] = False
    assert np.array_equal(got[keep], base[keep], equal_nan=True)


def test_nan_in_a_block_key(fa):
    """The K of block cell kv_len + j0 is seen by rows j >= j0 only: those rows of the kv-head
    group turn NaN, the rows before it keep their bits."""
    w, host = _nonfinite_case()
    dev = wl.to_device(host)
    n = _ws_bytes(fa, w, dev)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    base = _call(fa, w, dev, ws)
    j0 = 9
    h2 = dict(host)
    h2["k"] = host["k"].copy()
    h2["k"][0, w.kv_len[0] + j0, 1, 40] = 0x7E00
    _say("NaN in the K of a block cell")
    got = _call(fa, w, dev, ws, k=torch.from_numpy(h2["k"]).view(torch.float16).cuda())
    _compare_with_oracle(w, h2, got, "NaN block K")
    assert np.all(np.isnan(got[0, j0:16, 6:12]))
    keep = np.ones(got.shape, dtype=bool)
    keep[0, j0:, 6:12] = False
    assert np.array_equal(got[keep], base[keep], equal_nan=True)
