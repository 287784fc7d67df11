"""GPU parity of q8_0 KV decode/verify against the oracle, through the C ABI.

The oracle follows ggml: Q is quantised to q8_0 (per 32-dim block, d = amax/127, q rounded
half away from zero), every block dot is an exact integer sum scaled by d_k * d_q, and V is
dequantised to f32.  The GPU computes the same quantised values with one f16 rounding of
q * d per operand.  Bar: max-abs <= 2e-3 and rel-L2 <= 1e-3 on the f32 output.
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


def _run(fa, w, dev, mask_mode=sa.MASK_BLOCK_CAUSAL, mask=None, k=None, v=None, bounded_workspace=False):
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    fa(dev["q"], dev["k"] if k is None else k, dev["v"] if v is None else v, out, kv_len=dev["kv_len"],
       q_len=dev["q_len"], mask_mode=mask_mode, mask=mask, bounded_workspace=bounded_workspace)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(w, host, got, streams, label):
    want = oracle.attention_for_workload(host, w.kv_type, streams)
    ql = host["q_len"]
    rows_g = np.concatenate([got[s, :ql[s]].ravel() for s in streams])
    rows_w = np.concatenate([want[i, :ql[s]].ravel() for i, s in enumerate(streams)])
    m = oracle.diff_metrics(rows_w, rows_g)
    _say(f"{label} max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(rows_g))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m


@pytest.mark.parametrize("name", ["long_q8_decode", "long_q8_verify"])
def test_long_q8_configs(fa, name):
    _say(f"config {name} (all 8 streams against the oracle)")
    w = wl.config(name)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    got = _run(fa, w, dev)
    want = oracle.attention_for_workload(host, w.kv_type)
    rows = w.q_len[0]  # uniform
    m = oracle.diff_metrics(want[:, :rows], got[:, :rows])
    _say(f"{name} all streams max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(got[:, :rows]))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m
    for s in range(w.S):
        m = oracle.diff_metrics(want[s, :w.q_len[s]], got[s, :w.q_len[s]])
        assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (s, m)


@pytest.mark.parametrize("kv_len,q_len,H,Hkv", [
    ([0, 5, 100, 1531], [1, 3, 8, 7], 24, 4),   # empty cache, ragged rows up to 48 per group
    ([300, 33], [2, 2], 8, 8),                  # no GQA
    ([4000], [3], 32, 2),                       # 16 q-heads per kv-head, 48 rows
])
def test_q8_ragged(fa, kv_len, q_len, H, Hkv):
    _say(f"q8 ragged kv_len={kv_len} q_len={q_len} H={H} Hkv={Hkv}")
    w = wl.Workload("q8_ragged", 0x51A7_5000 + sum(kv_len), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv,
                    kv_type=sa.TYPE_Q8_0)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    _check(w, host, _run(fa, w, dev), list(range(w.S)), "q8 ragged")


def test_q8_explicit_mask_and_invariance(fa):
    _say("q8 explicit mask, and rows ignore cells past their position")
    w = wl.Workload("q8_small", 0x51A7_6000, 3, [130, 700, 41], [8, 8, 8], kv_type=sa.TYPE_Q8_0)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    base = _run(fa, w, dev)
    _check(w, host, base, list(range(w.S)), "q8 block-causal")
    n_kv = dev["k"].shape[1]
    mask = torch.from_numpy(oracle.build_kq_mask(n_kv, w.n_q, w.kv_len, w.q_len, True)).view(torch.float16).cuda()
    ex = _run(fa, w, dev, mask_mode=sa.MASK_EXPLICIT, mask=mask)
    _check(w, host, ex, list(range(w.S)), "q8 explicit mask")
    j = 3
    k2 = dev["k"].clone()
    v2 = dev["v"].clone()
    for s in range(w.S):
        k2[s, w.kv_len[s] + j + 1:] = 0x55
        v2[s, w.kv_len[s] + j + 1:] = 0x33
    alt = _run(fa, w, dev, k=k2, v=v2)
    assert np.array_equal(base[:, :j + 1], alt[:, :j + 1])
    for _ in range(5):
        assert np.array_equal(base, _run(fa, w, dev), equal_nan=True)


@pytest.mark.parametrize("kv_len,q_len,H,Hkv", [
    ([2000, 0, 513], [16, 16, 9], 24, 4),        # 16-token verify at GQA 6:1: 96 rows
    ([700, 4100], [12, 5], 20, 4),               # GQA 5:1, 60 rows (run as 64)
    ([30000], [16], 24, 4),                      # one long stream: many pieces per segment
])
def test_q8_more_than_48_rows(fa, kv_len, q_len, H, Hkv):
    """49..96 rows per kv-head group: the 32-cell q8_0 kernel, one launch reading the KV once."""
    _say(f"q8 49..96 rows kv_len={kv_len} q_len={q_len} H={H} Hkv={Hkv}")
    w = wl.Workload("q8_parts", 0x51A7_7000 + sum(kv_len), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv,
                    kv_type=sa.TYPE_Q8_0)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    _check(w, host, _run(fa, w, dev), list(range(w.S)), "q8 49..96 rows")


@pytest.mark.parametrize("name,kv_len,q_len,H,Hkv,q_type", [
    ("q8 64 rows, one stream", [100], [64], 24, 4, sa.TYPE_F32),          # 384 rows per group: prefill
    ("q8 prefill-sized, ragged", [300, 1000], [200, 130], 24, 4, sa.TYPE_F32),
    ("q8 prefill, f16 Q", [300, 1000], [200, 130], 24, 4, sa.TYPE_F16),
    ("q8 prefill, one-tile and empty streams", [0, 10, 333], [130, 40, 0], 8, 8, sa.TYPE_F32),
    ("q8 prefill, long stream", [5000], [300], 8, 2, sa.TYPE_F32),          # 83 tiles through the stages
    ("q8 64 rows of one head", [700, 90], [64, 49], 4, 4, sa.TYPE_F32),     # G = 1: 32-cell q8_0 kernel
])
def test_q8_prefill_blocks(fa, name, kv_len, q_len, H, Hkv, q_type):
    """Blocks beyond the q8_0 split-K kernels: K, V and Q staged as f16 in the workspace (a
    small cache), and with FLAG_BOUNDED_WORKSPACE the prefill kernel that moves each tile's
    q8_0 rows into LDS and converts them to f16 there -- the same operands, so the two agree
    bitwise."""
    _say(f"{name}: kv_len {kv_len} q_len {q_len} H {H} Hkv {Hkv} q_type {q_type}")
    w = wl.Workload("q8_prefill", 0x51A7_7100 + sum(q_len), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv,
                    kv_type=sa.TYPE_Q8_0, q_type=q_type)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    streams = [s for s in range(w.S) if q_len[s] > 0]
    got = _run(fa, w, dev)
    _check(w, host, got, streams, name)
    in_lds = _run(fa, w, dev, bounded_workspace=True)
    for s in streams:
        assert np.array_equal(got[s, :q_len[s]], in_lds[s, :q_len[s]]), (name, s)


def test_q8_prefill_explicit_mask(fa):
    """A plain explicit mask: the prefill kernel's LDS-staged mask mode over q8_0 tiles."""
    w = wl.Workload("q8_prefill_mask", 0x51A7_7180, 2, [500, 64], [160, 100], kv_type=sa.TYPE_Q8_0)
    host = wl.make_host(w)
    dev = wl.to_device(host)
    n_kv = dev["k"].shape[1]
    mask = oracle.build_kq_mask(n_kv, w.n_q, host["kv_len"], host["q_len"])
    dmask = torch.from_numpy(mask.view(np.float16)).cuda()
    _say("q8 prefill, explicit mask")
    got = _run(fa, w, dev, mask_mode=sa.MASK_EXPLICIT, mask=dmask)
    _check(w, host, got, list(range(w.S)), "q8 prefill explicit mask")
    in_lds = _run(fa, w, dev, mask_mode=sa.MASK_EXPLICIT, mask=dmask, bounded_workspace=True)
    for s in range(w.S):
        assert np.array_equal(got[s, :w.q_len[s]], in_lds[s, :w.q_len[s]]), s


def _shifted(t, nbytes):
    """The same q8_0 cache bytes at a base `nbytes` past a 256-byte aligned allocation."""
    buf = torch.empty(t.numel() + 256, dtype=torch.uint8, device="cuda")
    view = buf[nbytes:nbytes + t.numel()].view(t.shape)
    view.copy_(t)
    return view


def test_q8_more_than_48_rows_any_row_alignment(fa):
    """The 32-cell q8_0 kernel moves 136-byte rows with dword loads, so the rows' alignment does not
    matter: a cache moved by 4, 8 or 12 bytes (every head row's position within 16 bytes changes)
    gives the aligned cache's output bit for bit."""
    kv_len, q_len = [2000, 37, 513, 4097], [16, 16, 9, 11]
    w = wl.Workload("q8_align", 0x51A7_7100, len(kv_len), kv_len, q_len, H=24, Hkv=4, kv_type=sa.TYPE_Q8_0)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    base = _run(fa, w, dev)
    _check(w, host, base, list(range(w.S)), "q8 96 rows, aligned")
    for shift in (4, 8, 12):
        _say(f"q8 96 rows, cache moved by {shift} bytes")
        got = _run(fa, w, dev, k=_shifted(dev["k"], shift), v=_shifted(dev["v"], shift))
        assert np.array_equal(got, base, equal_nan=True), f"{shift}-byte shift changed the output"
