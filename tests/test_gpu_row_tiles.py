"""Every row count the split-K launcher maps, at both head dims, against the oracle.

The launcher runs G * q_len rows per kv-head group as 16-row tiles: 1, 2 or 3 tiles on the
16-cell kernel (128-dim heads), 4 and 6 tiles (5 runs as 6) on the 32-cell kernel, and at
256-dim heads 1, 2, 4 (3 runs as 4) and 6 tiles.  Each row count runs twice: as one long
stream, whose segments split into many pieces (the piece-parallel merge), and as a ragged batch
of short streams (the row-block merge).  q8_0 caches cover the 16-cell q8_0 kernel (<= 48 rows)
and the 32-cell q8_0 kernel (more rows; every row count at 256-dim heads).  Every row of every
stream is compared.  Bar: max-abs <= 2e-3 and rel-L2 <= 1e-3 on the f32 output.
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


# q_len at GQA 6:1 -> rows per group: 2 -> 12, 5 -> 30, 6 -> 36, 8 -> 48, 10 -> 60, 13 -> 78, 16 -> 96
Q_LENS = (2, 5, 6, 8, 10, 13, 16)
SHAPES = {"long": ([20000], None), "ragged": ([700, 3, 2500, 129, 64], [1, 0, 2, 3])}


def _workload(D, kv_type, q_len, shape):
    kv_len, cut = SHAPES[shape]
    # the ragged batch gives some streams fewer rows (cut[i] fewer), one stream none
    ql = [q_len] * len(kv_len) if cut is None else [max(0, q_len - c) for c in cut] + [q_len]
    if shape == "ragged":
        ql[1] = 0
    seed = 0x51A7_A000 + 97 * q_len + D + (1 if kv_type == sa.TYPE_Q8_0 else 0) + (7 if shape == "long" else 0)
    return wl.Workload(f"rows {shape}", seed, len(kv_len), kv_len, ql, D=D, kv_type=kv_type)


@pytest.mark.parametrize("shape", sorted(SHAPES))
@pytest.mark.parametrize("q_len", Q_LENS)
@pytest.mark.parametrize("D,kv_type", [(128, sa.TYPE_F16), (256, sa.TYPE_F16), (128, sa.TYPE_Q8_0),
                                       (256, sa.TYPE_Q8_0)])
def test_row_count(fa, D, kv_type, q_len, shape):
    w = _workload(D, kv_type, q_len, shape)
    _say(f"D={D} kv={'q8_0' if kv_type == sa.TYPE_Q8_0 else 'f16'} {shape}: kv_len={w.kv_len} q_len={w.q_len} "
         f"({6 * max(w.q_len)} rows per group)")
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = oracle.attention_for_workload(host, w.kv_type)
    for s in range(w.S):
        ql = w.q_len[s]
        if ql == 0:
            assert np.all(np.isnan(got[s])), "a stream without rows is left untouched"
            continue
        m = oracle.diff_metrics(want[s, :ql], got[s, :ql])
        assert np.all(np.isfinite(got[s, :ql])), s
        assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (s, m)
        assert np.all(np.isnan(got[s, ql:])), "rows past q_len are left untouched"
