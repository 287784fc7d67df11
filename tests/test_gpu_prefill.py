"""GPU parity of the chunked-prefill path (blocks of more than 96 rows per GQA group)
against the oracle, through the C ABI.

Bar: max-abs <= 2e-3 and rel-L2 <= 1e-3 on the f32 output against the oracle's
f32-accumulator restatement of ggml's CPU flash_attn_ext.  At full chunk size the oracle
checks row slices: rows [a, b) of a chunk over kv_len cached cells are exactly a block of
b - a rows over kv_len + a cached cells (same cells, same causal rule).
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


def _run(fa, w, dev, mask_mode=sa.MASK_BLOCK_CAUSAL, q=None, mask=None):
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    fa(dev["q"] if q is None else q, dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"],
       mask_mode=mask_mode, mask=mask)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(want, got, label):
    m = oracle.diff_metrics(want, got)
    _say(f"{label} max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(got))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m


def _slice_host(host, s, a, b):
    """rows [a, b) of stream s as a one-stream block with kv_len + a cached cells."""
    kl = int(host["kv_len"][s])
    q = host["q"][s:s + 1, a:b]
    if q.dtype == np.float16:
        q = q.astype(np.float32)
    return {"q": np.ascontiguousarray(q), "k": host["k"][s:s + 1], "v": host["v"][s:s + 1],
            "kv_len": np.array([kl + a], np.int32), "q_len": np.array([b - a], np.int32)}


@pytest.mark.parametrize("name", ["prefill_chunk0", "prefill_chunk1"])
def test_prefill_chunks_parity_every_row(fa, name):
    """All 2048 rows of the chunk against the oracle, on the whole and per 128-row block (the
    prefill kernel's work-group), so a fault in one row block cannot hide in the aggregate."""
    _say(f"config {name} (every row)")
    w = wl.config(name)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    got = _run(fa, w, dev)
    want = oracle.attention_for_workload(host, w.kv_type)
    _check(want[0], got[0], f"{name} rows [0,{w.q_len[0]})")
    for a in range(0, w.q_len[0], 128):
        m = oracle.diff_metrics(want[0, a:a + 128], got[0, a:a + 128])
        assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (a, m)
    # a row slice is the same block over a longer cache: the slice's oracle agrees
    a, b = 1000, 1100
    sl = oracle.attention_for_workload(_slice_host(host, 0, a, b), w.kv_type)
    _check(sl[0], got[0, a:b], f"{name} rows [{a},{b}) as their own block")


@pytest.mark.parametrize("kv_len,q_len,H,Hkv", [
    ([0, 100, 1000], [130, 257, 17], 24, 4),   # ragged rows, empty cache, a stream under one row block
    ([64, 3], [200, 129], 8, 8),               # no GQA
    ([777, 5], [7, 300], 32, 2),               # 16 q-heads per kv-head
])
def test_ragged_prefill(fa, kv_len, q_len, H, Hkv):
    _say(f"ragged prefill kv_len={kv_len} q_len={q_len} H={H} Hkv={Hkv}")
    w = wl.Workload("ragged_prefill", 0x51A7_3000 + sum(q_len), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    got = _run(fa, w, dev)
    want = oracle.attention_for_workload(host, w.kv_type)
    rows_g = np.concatenate([got[s, :q_len[s]].ravel() for s in range(w.S)])
    rows_w = np.concatenate([want[s, :q_len[s]].ravel() for s in range(w.S)])
    _check(rows_w, rows_g, "ragged prefill")


def _small_prefill():
    w = wl.Workload("small_prefill", 0x51A7_4000, 2, [300, 50], [200, 160])
    host = wl.make_host(w, poison=True)
    return w, host, wl.to_device(host)


def test_prefill_mask_none(fa):
    _say("prefill, mask NONE over kv_len + q_len cells")
    w, host, dev = _small_prefill()
    got = _run(fa, w, dev, mask_mode=sa.MASK_NONE)
    want = oracle.attention_for_workload(host, w.kv_type, causal=False)
    for s in range(w.S):
        _check(want[s, :w.q_len[s]], got[s, :w.q_len[s]], f"mask NONE stream {s}")


def test_prefill_explicit_mask_matches_causal(fa):
    _say("prefill, explicit llama mask vs block-causal")
    w, host, dev = _small_prefill()
    a = _run(fa, w, dev)
    n_kv = dev["k"].shape[1]
    mask = torch.from_numpy(oracle.build_kq_mask(n_kv, w.n_q, w.kv_len, w.q_len, True)).view(torch.float16).cuda()
    b = _run(fa, w, dev, mask_mode=sa.MASK_EXPLICIT, mask=mask)
    want = oracle.attention_for_workload(host, w.kv_type)
    for s in range(w.S):
        _check(want[s, :w.q_len[s]], b[s, :w.q_len[s]], f"explicit mask stream {s}")
        assert np.max(np.abs(a[s, :w.q_len[s]] - b[s, :w.q_len[s]])) <= 1e-3


def test_prefill_row_ignores_later_cells_bitwise(fa):
    _say("prefill row j independent of cells > kv_len + j")
    w, host, dev = _small_prefill()
    base = _run(fa, w, dev)
    j = 150
    k2 = dev["k"].clone()
    v2 = dev["v"].clone()
    for s in range(w.S):
        k2[s, w.kv_len[s] + j + 1:] = -3.0
        v2[s, w.kv_len[s] + j + 1:] = 7.0
    alt = _run(fa, w, dict(dev, k=k2, v=v2))
    assert np.array_equal(base[:, :j + 1], alt[:, :j + 1])


def test_prefill_repeatable_bitwise(fa):
    _say("prefill 10 launches, bitwise")
    w, host, dev = _small_prefill()
    first = _run(fa, w, dev)
    for _ in range(9):
        assert np.array_equal(first, _run(fa, w, dev), equal_nan=True)


def test_prefill_f16_queries(fa):
    _say("prefill f16 Q")
    w, host, dev = _small_prefill()
    q16 = dev["q"].to(torch.float16)
    got = _run(fa, w, dev, q=q16)
    ref_host = dict(host)
    ref_host["q"] = q16.float().cpu().numpy()
    want = oracle.attention_for_workload(ref_host, w.kv_type)
    for s in range(w.S):
        _check(want[s, :w.q_len[s]], got[s, :w.q_len[s]], f"f16 Q stream {s}")
