"""The per-cell attention modes against the oracle: ggml explicit masks with finite values
(ALiBi-style distance terms), ALiBi slopes (max_bias), logit softcap, and masks that cannot
be staged through LDS (rows not 16-byte aligned, more than 32 rows), at every decode shape
that takes them -- f16 at 6, 24 and 48 rows per GQA group (32-cell kernel, one row group per
lane), 64 and 96 rows, q8_0 (16-cell kernel up to 48 rows, the 32-cell q8_0 kernel beyond),
256-dim heads -- and the prefill kernel over f16 and q8_0 tiles (its LDS-staged mask mode for a
plain explicit mask, the generic mode otherwise).
Bar: max-abs <= 2e-3 and rel-L2 <= 1e-3 on the f32 output, as for the other parity tests."""
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


def _mask(n_kv, n_q, kv_len, q_len, slope_term, pad_cells=0):
    """f16 mask [S, 1, n_q, n_kv + pad_cells]: causal visibility; visible cells hold
    -slope_term * distance (0 when slope_term is 0), the rest -inf."""
    S = len(kv_len)
    width = n_kv + pad_cells
    m = np.full((S, 1, n_q, width), -np.inf, dtype=np.float32)
    for s in range(S):
        for j in range(q_len[s]):
            last = kv_len[s] + j
            cells = np.arange(last + 1)
            m[s, 0, j, :last + 1] = -slope_term * (last - cells)
    return m.astype(np.float16)


CASES = [
    # label, kv_type, D, kv_len, q_len, H, Hkv, slope_term, max_bias, softcap, pad_cells
    ("f16 6 rows, softcap", sa.TYPE_F16, 128, [900, 37, 4000], [1, 1, 1], 24, 4, 0.0, 0.0, 30.0, 0),
    ("f16 24 rows, alibi", sa.TYPE_F16, 128, [600, 1500], [4, 3], 24, 4, 0.05, 8.0, 0.0, 0),
    ("f16 48 rows, distance mask", sa.TYPE_F16, 128, [700, 1800], [8, 5], 24, 4, 0.02, 0.0, 0.0, 0),
    ("f16 48 rows, unaligned mask rows", sa.TYPE_F16, 128, [700, 1800], [8, 5], 24, 4, 0.0, 0.0, 0.0, 3),
    ("f16 40 rows of one head (mask not staged)", sa.TYPE_F16, 128, [500, 77], [40, 21], 4, 4, 0.01, 0.0, 0.0, 0),
    ("f16 96 rows, alibi + softcap", sa.TYPE_F16, 128, [900, 300, 2500], [16, 9, 16], 24, 4, 0.03, 4.0, 20.0, 0),
    ("f16 64 rows, softcap", sa.TYPE_F16, 128, [1200], [8], 32, 4, 0.0, 0.0, 50.0, 0),
    ("q8_0 48 rows, alibi", sa.TYPE_Q8_0, 128, [1000, 200], [8, 8], 24, 4, 0.05, 8.0, 0.0, 0),
    ("q8_0 12 rows, softcap", sa.TYPE_Q8_0, 128, [1500], [2], 24, 4, 0.0, 0.0, 30.0, 0),
    ("q8_0 96 rows, distance mask", sa.TYPE_Q8_0, 128, [900, 2000], [16, 11], 24, 4, 0.02, 0.0, 0.0, 0),
    ("q8_0 72 rows, alibi + softcap", sa.TYPE_Q8_0, 128, [1300, 40], [12, 12], 24, 4, 0.03, 8.0, 20.0, 0),
    ("256-dim 96 rows, alibi", sa.TYPE_F16, 256, [600, 1100], [16, 4], 24, 4, 0.03, 8.0, 0.0, 0),
    ("256-dim 6 rows, softcap", sa.TYPE_F16, 256, [2000], [1], 24, 4, 0.0, 0.0, 30.0, 0),
    ("q8_0 256-dim 96 rows, alibi + softcap", sa.TYPE_Q8_0, 256, [900, 1300], [16, 11], 24, 4, 0.02, 8.0, 20.0, 0),
    ("q8_0 256-dim 6 rows, distance mask", sa.TYPE_Q8_0, 256, [2500], [1], 24, 4, 0.03, 0.0, 0.0, 0),
    ("prefill rows, alibi + softcap", sa.TYPE_F16, 128, [200], [150], 24, 4, 0.02, 8.0, 25.0, 0),
    # an explicit mask alone: the prefill kernel's LDS-staged mask mode (dead tiles skipped)
    ("prefill rows, distance mask", sa.TYPE_F16, 128, [200, 700], [150, 260], 24, 4, 0.02, 0.0, 0.0, 0),
    ("prefill rows, causal mask, empty stream", sa.TYPE_F16, 128, [0, 333, 90], [130, 0, 300], 24, 4, 0.0, 0.0, 0.0, 0),
    ("256-dim prefill rows, distance mask", sa.TYPE_F16, 256, [300], [130], 24, 4, 0.01, 0.0, 0.0, 0),
    ("prefill rows, unaligned mask rows", sa.TYPE_F16, 128, [200], [150], 24, 4, 0.02, 0.0, 0.0, 3),
    ("q8_0 prefill rows, alibi + softcap", sa.TYPE_Q8_0, 128, [200], [150], 24, 4, 0.02, 8.0, 25.0, 0),
    ("q8_0 prefill rows, distance mask", sa.TYPE_Q8_0, 128, [200, 700], [150, 260], 24, 4, 0.02, 0.0, 0.0, 0),
    ("q8_0 prefill rows, unaligned mask rows", sa.TYPE_Q8_0, 128, [200], [150], 24, 4, 0.02, 0.0, 0.0, 3),
]


@pytest.mark.parametrize("label,kv_type,D,kv_len,q_len,H,Hkv,slope_term,max_bias,softcap,pad",
                         CASES, ids=[c[0] for c in CASES])
def test_generic_modes_against_the_oracle(fa, label, kv_type, D, kv_len, q_len, H, Hkv, slope_term, max_bias,
                                          softcap, pad):
    w = wl.Workload(label, 0x51A7_9400 + len(label), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv, D=D, kv_type=kv_type)
    host = wl.make_host(w)
    dev = wl.to_device(host)
    cap = dev["k"].shape[1]
    m = _mask(cap, w.n_q, w.kv_len, w.q_len, slope_term, pad)
    # the view covers the first cap cells of each (padded) mask row
    mask_dev = torch.from_numpy(m.view(np.uint16)).cuda().view(torch.float16)[..., :cap]
    _say(f"{label}: S={w.S} kv_len={kv_len} q_len={q_len} H={H} D={D} type={kv_type} "
         f"max_bias={max_bias} softcap={softcap} mask row bytes={m.shape[-1] * 2}")
    out = torch.full((w.S, w.n_q, H, D), float("nan"), device="cuda")
    fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=sa.MASK_EXPLICIT,
       mask=mask_dev, max_bias=max_bias, logit_softcap=softcap)
    torch.cuda.synchronize()
    q = host["q"].astype(np.float32)
    want = oracle.flash_attn_ext(q, host["k"], host["v"], kv_type,
                                 np.ascontiguousarray(m[..., :cap]).view(np.uint16), max_bias=max_bias,
                                 logit_softcap=softcap)
    got = out.cpu().numpy()
    g = np.concatenate([got[s, :q_len[s]].ravel() for s in range(w.S)])
    r = np.concatenate([want[s, :q_len[s]].ravel() for s in range(w.S)])
    assert np.all(np.isfinite(g))
    met = oracle.diff_metrics(r, g)
    _say(f"{label}: max_abs={met['max_abs']:.3e} rel_l2={met['rel_l2']:.3e}")
    assert met["max_abs"] <= MAX_ABS and met["rel_l2"] <= REL_L2, met
    if kv_type == sa.TYPE_Q8_0:
        # the q8_0 tiles converted in LDS instead of a staged f16 copy (prefill-sized blocks):
        # the same operands, the same output bit for bit
        out2 = torch.full_like(out, float("nan"))
        fa(dev["q"], dev["k"], dev["v"], out2, kv_len=dev["kv_len"], q_len=dev["q_len"],
           mask_mode=sa.MASK_EXPLICIT, mask=mask_dev, max_bias=max_bias, logit_softcap=softcap,
           bounded_workspace=True)
        torch.cuda.synchronize()
        got2 = out2.cpu().numpy()
        for s in range(w.S):
            assert np.array_equal(got[s, :q_len[s]], got2[s, :q_len[s]]), (label, s)
