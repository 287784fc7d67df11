"""The fused output gate (SIXI_ATTN_FLAG_GATE): out = attention * sigmoid(gate), the gate being
the second half of each head of the layer prologue's qg (include/sixi_layer.h; the Qwen3.8
full-attention layer, configs/qwen3.8-27b-ud-q4-k-xl.sixi:35,46-47).

Bar: a gated call equals the ungated call followed by sixi_attn_gate bit for bit on every row
it writes, for every kind of writer of the output -- rows the split kernels write whole (the
merge then gates them in place), both merges (few and many pieces per segment), the prefill
kernel, the llama-mask dual kernels -- and rows past a stream's q_len stay untouched."""
import sys

import numpy as np
import pytest
import torch

import oracle
import sixi_attn as sa
from sixi_attn import workloads as wl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def fa():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    sa.load_library()
    return sa.FlashAttnExt()


# label, kv_type, D, kv_len, q_len, H, Hkv, explicit llama mask
CASES = [
    ("decode, 16-cell kernel, many pieces", sa.TYPE_F16, 128, [4096], [1], 24, 4, False),
    ("decode batch with a short stream (whole-segment rows)", sa.TYPE_F16, 128, [20, 3000, 700], [1, 1, 1], 24, 4, False),
    ("verify 96 rows, 32-cell kernel", sa.TYPE_F16, 128, [900, 5000, 37, 2000], [16, 16, 9, 16], 24, 4, False),
    ("verify 96 rows, q8_0", sa.TYPE_Q8_0, 128, [900, 3000, 37], [16, 11, 16], 24, 4, False),
    ("verify q_len 4, q8_0, 256-dim", sa.TYPE_Q8_0, 256, [1500, 300, 4000], [4, 4, 3], 24, 4, False),
    ("verify q_len 6, f16, 256-dim", sa.TYPE_F16, 256, [1500, 300, 4000], [6, 6, 2], 24, 4, False),
    ("verify q_len 6, q8_0, 256-dim", sa.TYPE_Q8_0, 256, [1500, 300, 4000], [6, 6, 2], 24, 4, False),
    ("decode f16 256-dim", sa.TYPE_F16, 256, [4100], [1], 24, 4, False),
    ("prefill", sa.TYPE_F16, 128, [200, 700], [150, 260], 24, 4, False),
    ("prefill 256-dim", sa.TYPE_F16, 256, [300], [130], 24, 4, False),
    ("verify with the llama mask", sa.TYPE_F16, 128, [900, 5000, 37], [16, 16, 9], 24, 4, True),
    ("decode with the llama mask", sa.TYPE_F16, 128, [4096], [1], 24, 4, True),
    ("prefill with the llama mask", sa.TYPE_F16, 128, [200, 700], [150, 260], 24, 4, True),
]


@pytest.mark.parametrize("label,kv_type,D,kv_len,q_len,H,Hkv,masked", CASES, ids=[c[0] for c in CASES])
def test_gated_call_equals_attention_then_gate(fa, label, kv_type, D, kv_len, q_len, H, Hkv, masked):
    w = wl.Workload(label, 0x51A7_A000 + len(label), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv, D=D, kv_type=kv_type)
    host = wl.make_host(w)
    dev = wl.to_device(host)
    gen = torch.Generator(device="cuda").manual_seed(0x51A7 + len(label))
    qg = torch.randn((w.S, w.n_q, H, 2 * D), generator=gen, device="cuda", dtype=torch.float32) * 3.0
    mask = None
    mode = sa.MASK_BLOCK_CAUSAL
    if masked:
        bits = oracle.build_kq_mask(dev["k"].shape[1], w.n_q, w.kv_len, w.q_len, True)
        mask = torch.from_numpy(bits).cuda().view(torch.float16)
        mode = sa.MASK_EXPLICIT
    _say(f"{label}: S={w.S} kv_len={kv_len} q_len={q_len} H={H}/{Hkv} D={D} type={kv_type} mask={masked}")
    ref = torch.full((w.S, w.n_q, H, D), float("nan"), device="cuda")
    fa(dev["q"], dev["k"], dev["v"], ref, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=mode, mask=mask)
    sa.attn_gate(ref, qg, q_len=dev["q_len"])
    got = torch.full_like(ref, float("nan"))
    fa(dev["q"], dev["k"], dev["v"], got, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=mode, mask=mask, gate=qg)
    torch.cuda.synchronize()
    r, g = ref.cpu().numpy(), got.cpu().numpy()
    for s in range(w.S):
        assert np.array_equal(g[s, :q_len[s]], r[s, :q_len[s]]), (label, s)
        assert np.all(np.isnan(g[s, q_len[s]:])), (label, s, "rows past q_len written")
    # and the gated output is the gate applied to the oracle's attention, within the parity bar
    want = oracle.attention_for_workload(host, kv_type, list(range(w.S)))
    gate = qg.cpu().numpy()[..., D:]
    want = want * (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32)
    rows_g = np.concatenate([g[s, :q_len[s]].ravel() for s in range(w.S)])
    rows_w = np.concatenate([want[s, :q_len[s]].ravel() for s in range(w.S)])
    met = oracle.diff_metrics(rows_w, rows_g)
    _say(f"{label}: vs oracle max_abs={met['max_abs']:.3e} rel_l2={met['rel_l2']:.3e}")
    assert met["max_abs"] <= 2e-3 and met["rel_l2"] <= 1e-3, met


def test_gated_noalloc_equals_gated_forward(fa):
    w = wl.Workload("gated noalloc", 0x51A7_A100, 4, [900, 5000, 37, 2000], [16, 16, 9, 16])
    dev = wl.to_device(wl.make_host(w))
    qg = torch.randn((w.S, w.n_q, w.H, 2 * w.D), device="cuda", dtype=torch.float32)
    a = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), device="cuda")
    b = torch.full_like(a, float("nan"))
    fa(dev["q"], dev["k"], dev["v"], a, kv_len=dev["kv_len"], q_len=dev["q_len"], gate=qg)
    fa(dev["q"], dev["k"], dev["v"], b, kv_len=dev["kv_len"], q_len=dev["q_len"], gate=qg, noalloc=True)
    torch.cuda.synchronize()
    assert torch.equal(torch.nan_to_num(a, nan=7.0), torch.nan_to_num(b, nan=7.0))
