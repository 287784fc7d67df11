"""GPU parity of the split-K decode/verify path against the oracle, through the C ABI.

Bar (fp32 output): max-abs <= 2e-3 and rel-L2 <= 1e-3 against the oracle's f32-accumulator
restatement of ggml's CPU flash_attn_ext on the same seeded inputs.  Masking and per-stream
lengths are checked bit-exactly through invariances: changing anything a row must not see
leaves that row's bits unchanged.
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
    sa.load_library()  # no fallback: a missing library fails here
    return sa.FlashAttnExt()


def _run(fa, w, dev, mask_mode=sa.MASK_BLOCK_CAUSAL, q=None, k=None, v=None, kv_len="dev", mask=None):
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    kl = dev["kv_len"] if kv_len == "dev" else kv_len
    fa(dev["q"] if q is None else q, dev["k"] if k is None else k, dev["v"] if v is None else v, out,
       kv_len=kl, q_len=dev["q_len"], mask_mode=mask_mode, mask=mask)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check(w, host, got, streams=None, label=""):
    idx = list(range(w.S)) if streams is None else list(streams)
    want = oracle.attention_for_workload(host, w.kv_type, idx)
    ql = host["q_len"][idx]
    g = got[idx]
    rows_g = np.concatenate([g[i, :ql[i]].ravel() for i in range(len(idx))])
    rows_w = np.concatenate([want[i, :ql[i]].ravel() for i in range(len(idx))])
    m = oracle.diff_metrics(rows_w, rows_g)
    _say(f"{label} max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(rows_g))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m
    return m


@pytest.mark.parametrize("name", ["decode", "verify"])
def test_config_parity(fa, name):
    _say(f"config {name}")
    w = wl.config(name)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    _check(w, host, _run(fa, w, dev), label=name)


def test_batched_verify_parity(fa):
    """Every row of all 32 streams against the oracle, and each stream on its own bar, so a
    fault confined to one split piece, segment or XCD cannot hide in the aggregate."""
    _say("config batched_verify (all 32 streams against the oracle)")
    w = wl.config("batched_verify")
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    got = _run(fa, w, dev)
    want = oracle.attention_for_workload(host, w.kv_type)
    m = oracle.diff_metrics(want[:, :16], got[:, :16])  # every stream has 16 rows
    _say(f"batched_verify, all streams max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(got[:, :16]))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m
    for s in range(w.S):
        m = oracle.diff_metrics(want[s, :16], got[s, :16])
        assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (s, m)


@pytest.mark.parametrize("kv_len,q_len,H,Hkv", [
    ([0, 5, 100, 31], [1, 3, 16, 7], 24, 4),     # empty cache, ragged rows, 96 rows max
    ([64, 1000, 2], [7, 7, 7], 24, 4),           # 42 rows: 3 row tiles
    ([3000, 45, 0, 511], [16, 13, 4, 16], 32, 8),  # GQA 4:1, 64 rows: 4 row tiles
    ([129, 2048], [16, 11], 40, 8),              # GQA 5:1, 80 rows: 5 row tiles run as 6
    ([700, 3000], [16, 10], 12, 2),              # 96 rows, two kv-heads: head groups of 2
    ([2000, 50, 900], [10, 16, 1], 6, 1),        # 96 rows, one kv-head: head groups of 1
    ([1500, 400], [16, 3], 36, 6),               # 96 rows, six kv-heads: three groups of 2
    ([300, 33], [2, 2], 8, 8),                   # no GQA
    ([4096, 77], [5, 9], 32, 2),                 # GQA 16:1, 144 > 96 rows -> not split-K
])
def test_ragged_shapes(fa, kv_len, q_len, H, Hkv):
    _say(f"ragged kv_len={kv_len} q_len={q_len} H={H} Hkv={Hkv}")
    w = wl.Workload("ragged", 0x51A7_1000 + sum(kv_len), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv)
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    if (H // Hkv) * w.n_q > 96:
        out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
        rc = fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"], check=False)
        assert rc in (sa.OK, sa.E_UNSUPPORTED)
        if rc == sa.OK:
            torch.cuda.synchronize()
            _check(w, host, out.cpu().numpy(), label="ragged (prefill kernel)")
        return
    _check(w, host, _run(fa, w, dev), label="ragged")


def _small(seed=0x51A7_2000, S=3, kv_len=(130, 700, 41), q_len=16):
    w = wl.Workload("small", seed, S, list(kv_len), [q_len] * S)
    host = wl.make_host(w, poison=True)
    return w, host, wl.to_device(host)


def test_mask_none_matches_ggml_without_mask(fa):
    _say("mask NONE, kv_len NULL (every cell of the view)")
    w, host, dev = _small()
    n_kv = 512
    k = dev["k"][:, :n_kv].contiguous()
    v = dev["v"][:, :n_kv].contiguous()
    # fill every cell so the whole view is valid data
    kh = np.ascontiguousarray(host["k"][:, :n_kv]); vh = np.ascontiguousarray(host["v"][:, :n_kv])
    rng = np.random.default_rng(9)
    kh[:] = rng.standard_normal(kh.shape).astype(np.float16).view(np.uint16)
    vh[:] = rng.standard_normal(vh.shape).astype(np.float16).view(np.uint16)
    k.copy_(torch.from_numpy(kh).view(torch.float16)); v.copy_(torch.from_numpy(vh).view(torch.float16))
    out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    fa(dev["q"], k, v, out, kv_len=None, q_len=None, mask_mode=sa.MASK_NONE)
    torch.cuda.synchronize()
    want = oracle.flash_attn_ext(host["q"], kh, vh, oracle.F16, None)
    m = oracle.diff_metrics(want, out.cpu().numpy())
    _say(f"mask NONE max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2


def test_explicit_llama_mask_matches_block_causal(fa):
    """The ggml-style explicit mask (general path: logits in log2 units, per-cell mask
    reads) and the block-causal lengths (fast path) select the same cells: both agree with
    the oracle and with each other far inside the parity bar."""
    _say("explicit llama mask vs block-causal")
    w, host, dev = _small()
    a = _run(fa, w, dev)
    n_kv = dev["k"].shape[1]
    mask = torch.from_numpy(oracle.build_kq_mask(n_kv, w.n_q, w.kv_len, w.q_len, True)).view(torch.float16).cuda()
    b = _run(fa, w, dev, mask_mode=sa.MASK_EXPLICIT, mask=mask)
    _check(w, host, b, label="explicit mask")
    assert np.max(np.abs(a - b)) <= 1e-3


def test_repeatable_bitwise_over_20_launches(fa):
    _say("20 launches, bitwise")
    w, host, dev = _small()
    first = _run(fa, w, dev)
    for _ in range(19):
        assert np.array_equal(first, _run(fa, w, dev), equal_nan=True)


def test_row_ignores_later_rows_and_cells(fa):
    _say("row j independent of rows > j and cells > kv_len + j")
    w, host, dev = _small()
    base = _run(fa, w, dev)
    j = 6
    q2 = dev["q"].clone(); k2 = dev["k"].clone(); v2 = dev["v"].clone()
    q2[:, j + 1:] = 3.0
    for s in range(w.S):
        k2[s, w.kv_len[s] + j + 1:] = -7.0
        v2[s, w.kv_len[s] + j + 1:] = 5.0
    alt = _run(fa, w, dev, q=q2, k=k2, v=v2)
    assert np.array_equal(base[:, :j + 1], alt[:, :j + 1])
    assert not np.array_equal(base[:, j + 1:], alt[:, j + 1:])


def test_stream_ignores_other_streams_data(fa):
    _say("stream 0 independent of other streams' data")
    w, host, dev = _small()
    base = _run(fa, w, dev)
    q2 = dev["q"].clone(); k2 = dev["k"].clone(); v2 = dev["v"].clone()
    q2[1:] *= -1.0
    k2[1:] = 0.25
    v2[1:] = -1.5
    alt = _run(fa, w, dev, q=q2, k=k2, v=v2)
    assert np.array_equal(base[0], alt[0])


def test_gqa_heads_with_equal_queries_agree_bitwise(fa):
    _say("GQA group heads with identical Q")
    w, host, dev = _small()
    q2 = dev["q"].clone()
    for g in range(w.Hkv):
        q2[:, :, g * 6:(g + 1) * 6] = q2[:, :, g * 6:g * 6 + 1]
    out = _run(fa, w, dev, q=q2)
    for g in range(w.Hkv):
        for h in range(g * 6 + 1, (g + 1) * 6):
            assert np.array_equal(out[:, :, g * 6], out[:, :, h])


def test_f16_queries(fa):
    _say("f16 Q")
    w, host, dev = _small()
    q16 = dev["q"].to(torch.float16)
    got = _run(fa, w, dev, q=q16)
    ref_host = dict(host)
    ref_host["q"] = q16.float().cpu().numpy()
    _check(w, ref_host, got, label="f16 Q")


def test_workspace_too_small_is_rejected(fa):
    _say("workspace too small")
    w, host, dev = _small()
    out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    p = fa.params(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"])
    need = fa.workspace_bytes(p)
    ws = torch.empty(need // 2, dtype=torch.uint8, device="cuda")
    p.workspace = ws.data_ptr()
    p.workspace_bytes = ws.numel()
    import ctypes
    assert fa.lib.sixi_attn_forward(ctypes.byref(p)) == sa.E_OUT_OF_BOUNDS
