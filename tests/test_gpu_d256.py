"""256-dim heads (the real model's key/value length, configs/qwen3.8-27b-ud-q4-k-xl.sixi) on the
32-cell split-K kernel, against the oracle through the C ABI: decode, speculative verify (96 rows
per group as one lane of three row groups), ragged streams, an explicit mask and f16 Q; the
prefill kernel for 256-dim heads; q8_0 caches on the 16-cell kernel (up to 48 rows, lengths
only: q8_0 dequantised in registers), on the 32-cell q8_0 kernel (explicit masks, more rows: one
lane, up to three row groups of two row tiles) and, for prefill-sized blocks, on the prefill
kernel over q8_0 tiles
converted in LDS (rows that are not 16-byte aligned: through the f16 staging).  Bar: max-abs <=
2e-3 and rel-L2 <= 1e-3 on the f32 output."""
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


def _unaligned_rows(t):
    """The same q8_0 cache [S, cells, Hkv, 272] with 4 spare bytes after every cell, so that no
    cell row starts 16-byte aligned (cell stride Hkv * 272 + 4)."""
    S, cells, Hkv, row = t.shape
    buf = torch.zeros((S, cells, Hkv * row + 4), dtype=torch.uint8, device=t.device)
    buf[:, :, :Hkv * row] = t.reshape(S, cells, Hkv * row)
    return buf[:, :, :Hkv * row].unflatten(2, (Hkv, row))


def _run_check(fa, w, label, mask_mode=sa.MASK_BLOCK_CAUSAL, explicit=False, unaligned=False, both=False):
    """Against the oracle; ``both``: also with FLAG_BOUNDED_WORKSPACE, whose q8_0 prefill
    converts the q8_0 tiles in LDS instead of staging them as f16 -- the same operands, so the
    outputs must agree bitwise."""
    host = wl.make_host(w, poison=not explicit)
    dev = wl.to_device(host)
    if unaligned:
        dev["k"], dev["v"] = _unaligned_rows(dev["k"]), _unaligned_rows(dev["v"])
        assert dev["k"].stride(1) % 16 == 4
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    mask = None
    if explicit:
        m = oracle.build_kq_mask(dev["k"].shape[1], w.n_q, host["kv_len"], host["q_len"])
        mask = torch.from_numpy(m.view(np.float16)).cuda()
        mask_mode = sa.MASK_EXPLICIT
    _say(f"{label}: S={w.S} kv_len={w.kv_len} q_len={w.q_len} H={w.H} Hkv={w.Hkv} D={w.D}")
    fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=mask_mode, mask=mask)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    if both:
        out2 = torch.full_like(out, float("nan"))
        fa(dev["q"], dev["k"], dev["v"], out2, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=mask_mode,
           mask=mask, bounded_workspace=True)
        torch.cuda.synchronize()
        got2 = out2.cpu().numpy()
        for s in range(w.S):
            assert np.array_equal(got[s, :w.q_len[s]], got2[s, :w.q_len[s]]), f"{label}: stream {s}"
    want = oracle.attention_for_workload(host, w.kv_type, causal=mask_mode != sa.MASK_NONE)
    ql = host["q_len"]
    g = np.concatenate([got[s, :ql[s]].ravel() for s in range(w.S)])
    r = np.concatenate([want[s, :ql[s]].ravel() for s in range(w.S)])
    m = oracle.diff_metrics(r, g)
    _say(f"{label}: max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(g))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m


@pytest.mark.parametrize("label,kv_len,q_len,H,Hkv", [
    ("decode", [4096], [1], 24, 4),                       # 6 rows per group
    ("decode ragged", [700, 3000, 5], [1, 1, 1], 24, 4),
    ("verify", [2000, 8192], [16, 16], 24, 4),            # 96 rows: one lane of three row groups
    ("verify ragged", [1500, 300, 900], [16, 3, 9], 24, 4),
    ("32 rows", [1200], [8], 16, 4),
    ("64 rows, one launch", [999], [8], 32, 4),
    ("MHA", [1000, 64], [16, 5], 4, 4),                    # G = 1
])
def test_d256_against_oracle(fa, label, kv_len, q_len, H, Hkv):
    w = wl.Workload("d256", 0x51A7_9100 + sum(kv_len), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv, D=256)
    _run_check(fa, w, label)


def test_d256_explicit_mask(fa):
    w = wl.Workload("d256 mask", 0x51A7_9200, 2, [600, 77], [16, 4], D=256)
    _run_check(fa, w, "explicit mask", explicit=True)


def test_d256_f16_q(fa):
    w = wl.Workload("d256 f16 q", 0x51A7_9300, 2, [1300, 50], [12, 1], D=256, q_type=sa.TYPE_F16)
    _run_check(fa, w, "f16 Q")


@pytest.mark.parametrize("label,kv_len,q_len", [
    ("prefill chunk", [500], [300]),                # 1800 rows per group: the prefill kernel
    ("prefill ragged", [64, 1000], [200, 129]),
])
def test_d256_prefill(fa, label, kv_len, q_len):
    w = wl.Workload("d256 prefill", 0x51A7_9500 + sum(q_len), len(kv_len), kv_len, q_len, D=256, q_type=sa.TYPE_F16,
                    mul=0.5)
    _run_check(fa, w, label)


def test_d256_prefill_explicit_mask(fa):
    w = wl.Workload("d256 prefill mask", 0x51A7_9600, 1, [300], [150], D=256)
    _run_check(fa, w, "prefill explicit mask", explicit=True)


@pytest.mark.parametrize("label,kv_len,q_len,explicit", [
    ("q8_0 decode", [3000, 70], [1, 1], False),                 # 6 rows: the 16-cell kernel, one tile
    ("q8_0 24 rows", [1800, 640], [4, 3], False),               # 16-cell kernel, two row tiles
    ("q8_0 36 rows", [2300, 17, 5000], [6, 6, 2], False),       # 16-cell kernel, three row tiles
    ("q8_0 48 rows", [2500, 90], [8, 8], False),                # 16-cell kernel, three row tiles
    ("q8_0 24 rows, one long stream", [30000], [4], False),     # 16-cell kernel, many pieces
    ("q8_0 ragged batch", [700, 12000, 3, 255, 4096, 1, 9000, 513], [4, 6, 6, 1, 5, 6, 3, 4], False),
    ("q8_0 24 rows, explicit mask", [1800, 640], [4, 3], True),  # the 32-cell q8_0 kernel
    ("q8_0 verify", [1200, 400], [16, 7], False),               # 96 rows: three row groups
    ("q8_0 verify, one long stream", [20000], [16], False),     # many pieces
    ("q8_0 verify, explicit mask", [1500, 333], [16, 5], True),
    ("q8_0 decode, explicit mask", [4000], [1], True),
    ("q8_0 prefill", [200], [150], False),
    ("q8_0 prefill ragged", [3000, 0, 700], [300, 129, 200], False),
    ("q8_0 prefill, long stream", [5000], [260], False),    # 83 tiles, 20 pages
    ("q8_0 prefill, explicit mask", [300, 40], [150, 260], True),
])
def test_d256_q8_0(fa, label, kv_len, q_len, explicit):
    """q8_0 caches of 256-dim heads: split-K calls of up to 48 rows with lengths only run the
    16-cell kernel (q8_0 dequantised in registers), the others the 32-cell q8_0 kernel on one lane;
    prefill-sized blocks stage K, V and Q as f16 (a small cache) or, with
    FLAG_BOUNDED_WORKSPACE, run the prefill kernel that converts each tile's q8_0 rows in LDS:
    both against the oracle, and bitwise against each other."""
    w = wl.Workload("d256 q8", 0x51A7_9700 + sum(q_len), len(kv_len), kv_len, q_len, D=256, kv_type=sa.TYPE_Q8_0)
    _run_check(fa, w, label, explicit=explicit, both=True)


def test_d256_q8_0_prefill_f16_q_and_no_mask(fa):
    w = wl.Workload("d256 q8 f16q", 0x51A7_9750, 2, [900, 64], [200, 150], D=256, kv_type=sa.TYPE_Q8_0,
                    q_type=sa.TYPE_F16)
    _run_check(fa, w, "q8_0 prefill, f16 Q", both=True)
    w = wl.Workload("d256 q8 none", 0x51A7_9760, 2, [900, 64], [200, 150], D=256, kv_type=sa.TYPE_Q8_0)
    _run_check(fa, w, "q8_0 prefill, no mask", mask_mode=sa.MASK_NONE, both=True)


def test_d256_q8_0_prefill_beyond_the_staging_cap(fa):
    """A cache whose f16 staging would exceed STAGE_CAP_BYTES (4 streams x 9000 cells: 147 MB)
    runs the in-LDS conversion by default: a token workspace, output against the oracle."""
    w = wl.Workload("d256 q8 long", 0x51A7_9770, 4, [9000, 8800, 100, 4000], [130, 200, 150, 160], D=256,
                    kv_type=sa.TYPE_Q8_0)
    host = wl.make_host(w)
    dev = wl.to_device(host)
    out = torch.empty((w.S, w.n_q, w.H, w.D), dtype=torch.float32, device="cuda")
    p = fa.params(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"])
    assert fa.workspace_bytes(p) <= 4096
    _run_check(fa, w, "q8_0 prefill beyond the staging cap")


@pytest.mark.parametrize("label,kv_len,q_len", [
    ("q8_0 prefill, rows not 16-byte aligned (staged)", [200, 900], [150, 130]),
    ("q8_0 verify, rows not 16-byte aligned (staged)", [1200, 400], [16, 7]),
])
def test_d256_q8_0_unaligned_rows_are_staged(fa, label, kv_len, q_len):
    """256-dim q8_0 rows that do not start 16-byte aligned cannot come in by 16-byte LDS-DMA
    loads: such calls stage K, V and Q as f16 operands in the workspace and run the f16
    kernels."""
    w = wl.Workload("d256 q8 unaligned", 0x51A7_9780 + sum(q_len), len(kv_len), kv_len, q_len, D=256,
                    kv_type=sa.TYPE_Q8_0)
    _run_check(fa, w, label, unaligned=True)
