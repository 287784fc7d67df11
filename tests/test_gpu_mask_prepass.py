"""The explicit-mask pre-pass (fa_mask.hip) and the kernels that follow it.

llama.cpp builds the KQ mask of a verify block or a prefill chunk from the batch positions
(src/core/core_execution.cpp:2047-2062): row j of stream s sees cells [0, N_s + j].  The
pre-pass reduces each mask row to the kv offset it implies; when every row of every stream is
such a block-causal prefix, the attention runs the lengths-only body with those offsets, and
otherwise the staged-mask body, chosen on the device.

Bars:
  * a llama mask gives the block-causal lengths call's output bit for bit (the same body on the
    same offsets, in the same split), and meets the oracle's parity bar (max-abs <= 2e-3,
    rel-L2 <= 1e-3);
  * a prefix mask whose offsets are not the call's kv_len gives the lengths call with those
    offsets bit for bit;
  * masks that are not block-causal prefixes (a hole, a fully masked row, a finite bias, one
    span shared by every row) meet the oracle's bar through the mask body (the staged mask of
    the 32-cell kernels and of prefill, the per-cell mode of the 16-cell kernel, one row tile
    at a time);
  * -0.0 counts as a visible cell, exactly as +0.0.
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
F16_NEG_INF = 0xFC00
F16_NEG_ZERO = 0x8000


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def fa():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    sa.load_library()
    return sa.FlashAttnExt()


# label, kv_type, D, kv_len, q_len, H, Hkv, bitwise (the lengths call runs the same kernel)
CASES = [
    ("f16 64 rows", sa.TYPE_F16, 128, [900, 3000, 37], [16, 16, 9], 32, 8, True),
    ("f16 96 rows", sa.TYPE_F16, 128, [1500, 260], [16, 11], 24, 4, True),
    ("f16 256-dim 6 rows", sa.TYPE_F16, 256, [2100, 70], [1, 1], 24, 4, True),
    ("f16 256-dim 24 rows", sa.TYPE_F16, 256, [1300, 400], [4, 3], 24, 4, True),
    ("f16 256-dim 48 rows", sa.TYPE_F16, 256, [800], [8], 24, 4, True),
    ("f16 256-dim 96 rows", sa.TYPE_F16, 256, [1000, 33], [16, 16], 24, 4, True),
    ("q8_0 6 rows", sa.TYPE_Q8_0, 128, [2500, 100, 7], [1, 1, 1], 24, 4, True),
    ("q8_0 16 rows", sa.TYPE_Q8_0, 128, [1200], [4], 32, 8, True),
    ("q8_0 64 rows", sa.TYPE_Q8_0, 128, [1800, 500], [16, 12], 32, 8, True),
    ("q8_0 96 rows", sa.TYPE_Q8_0, 128, [700, 1900], [16, 16], 24, 4, True),
    ("q8_0 256-dim 64 rows", sa.TYPE_Q8_0, 256, [1500, 90], [16, 16], 32, 8, True),
    ("q8_0 256-dim 96 rows", sa.TYPE_Q8_0, 256, [600], [16], 24, 4, True),
    ("q8_0 256-dim 36 rows", sa.TYPE_Q8_0, 256, [900, 300], [6, 6], 24, 4, True),
    ("q8_0 256-dim 6 rows", sa.TYPE_Q8_0, 256, [3000, 5], [1, 1], 24, 4, True),
    ("f16 6 rows", sa.TYPE_F16, 128, [4000, 900, 1], [1, 1, 1], 24, 4, True),
    ("f16 24 rows", sa.TYPE_F16, 128, [2000, 150], [4, 4], 24, 4, True),
    ("f16 48 rows", sa.TYPE_F16, 128, [700, 1800], [8, 5], 24, 4, True),
    ("q8_0 24 rows", sa.TYPE_Q8_0, 128, [2200, 40], [4, 3], 24, 4, True),
    ("q8_0 48 rows", sa.TYPE_Q8_0, 128, [1600], [12], 16, 4, True),
    ("prefill f16", sa.TYPE_F16, 128, [200, 700], [150, 260], 24, 4, True),
    ("prefill f16 with an empty stream", sa.TYPE_F16, 128, [0, 333, 90], [130, 0, 300], 24, 4, True),
    ("prefill f16 256-dim", sa.TYPE_F16, 256, [300], [130], 24, 4, True),
    ("prefill q8_0", sa.TYPE_Q8_0, 128, [200, 700], [150, 260], 24, 4, True),
]


def _setup(label, kv_type, D, kv_len, q_len, H, Hkv):
    w = wl.Workload(label, 0x51A7_9800 + len(label), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv, D=D,
                    kv_type=kv_type)
    host = wl.make_host(w)
    return w, host, wl.to_device(host)


def _mask_host(w, n_kv, kv_len, pad_rows=0):
    """llama-style mask bits [S, 1, n_q + pad_rows, n_kv] (uint16) for offsets kv_len."""
    return oracle.build_kq_mask(n_kv, w.n_q + pad_rows, kv_len, w.q_len, True)


def _call(fa, w, dev, mask_bits=None, kv_len=None, bounded=False):
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), device="cuda")
    kl = dev["kv_len"] if kv_len is None else torch.tensor(kv_len, dtype=torch.int32, device="cuda")
    if mask_bits is None:
        fa(dev["q"], dev["k"], dev["v"], out, kv_len=kl, q_len=dev["q_len"], mask_mode=sa.MASK_BLOCK_CAUSAL,
           bounded_workspace=bounded)
    else:
        mask = torch.from_numpy(np.ascontiguousarray(mask_bits)).cuda().view(torch.float16)
        fa(dev["q"], dev["k"], dev["v"], out, kv_len=kl, q_len=dev["q_len"], mask_mode=sa.MASK_EXPLICIT,
           mask=mask, bounded_workspace=bounded)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _rows(w, a):
    return [a[s, :w.q_len[s]] for s in range(w.S)]


def _oracle_check(w, host, got, mask_bits, label):
    cap = mask_bits.shape[-1]
    want = oracle.flash_attn_ext(host["q"].astype(np.float32), host["k"], host["v"], w.kv_type,
                                 np.ascontiguousarray(mask_bits[:, :, :w.n_q, :cap]))
    g = np.concatenate([x.ravel() for x in _rows(w, got)])
    r = np.concatenate([x.ravel() for x in _rows(w, want)])
    assert np.all(np.isfinite(g)), label
    met = oracle.diff_metrics(r, g)
    _say(f"{label}: max_abs={met['max_abs']:.3e} rel_l2={met['rel_l2']:.3e}")
    assert met["max_abs"] <= MAX_ABS and met["rel_l2"] <= REL_L2, (label, met)


@pytest.mark.parametrize("label,kv_type,D,kv_len,q_len,H,Hkv,bitwise", CASES, ids=[c[0] for c in CASES])
def test_llama_mask_is_the_lengths_call(fa, label, kv_type, D, kv_len, q_len, H, Hkv, bitwise):
    w, host, dev = _setup(label, kv_type, D, kv_len, q_len, H, Hkv)
    cap = dev["k"].shape[1]
    bits = _mask_host(w, cap, w.kv_len, pad_rows=3)
    _say(f"{label}: S={w.S} kv_len={kv_len} q_len={q_len} H={H}/{Hkv} D={D} type={kv_type}")
    got = _call(fa, w, dev, bits)
    _oracle_check(w, host, got, bits, label)
    if bitwise:
        ref = _call(fa, w, dev)
        for s, (x, y) in enumerate(zip(_rows(w, got), _rows(w, ref))):
            assert np.array_equal(x, y), (label, s)
    if kv_type == sa.TYPE_Q8_0 and w.n_q > 96 // (H // Hkv):
        # prefill over q8_0 tiles converted in LDS (no staged copy): the same operands
        got2 = _call(fa, w, dev, bits, bounded=True)
        ref2 = _call(fa, w, dev, bounded=True)
        for s, (x, y) in enumerate(zip(_rows(w, got2), _rows(w, ref2))):
            assert np.array_equal(x, y), (label, "bounded", s)


@pytest.mark.parametrize("label,kv_type,D,kv_len,q_len,H,Hkv,bitwise",
                         [c for c in CASES if c[7] and min(c[3]) >= 8], ids=[c[0] for c in CASES if c[7] and min(c[3]) >= 8])
def test_prefix_offsets_other_than_kv_len(fa, label, kv_type, D, kv_len, q_len, H, Hkv, bitwise):
    """A block-causal mask built for shorter streams than the call's kv_len: the call attends
    to what the mask shows, i.e. the lengths call at the mask's offsets."""
    w, host, dev = _setup(label, kv_type, D, kv_len, q_len, H, Hkv)
    cap = dev["k"].shape[1]
    shorter = [k - 1 - (k // 7) for k in w.kv_len]
    bits = _mask_host(w, cap, shorter)
    _say(f"{label}: mask offsets {shorter} under kv_len {list(w.kv_len)}")
    got = _call(fa, w, dev, bits)
    ref = _call(fa, w, dev, kv_len=shorter)
    for s, (x, y) in enumerate(zip(_rows(w, got), _rows(w, ref))):
        assert np.array_equal(x, y), (label, s)


def _edit(bits, w, kind):
    """A llama mask changed so that it is not a block-causal prefix (or, for "neg_zero", still is)."""
    b = bits.copy()
    s = w.S - 1 if w.q_len[-1] > 0 else 0
    j = min(w.q_len[s] - 1, 2)
    last = w.kv_len[s] + j  # row j's last visible cell
    if kind == "hole":
        b[s, 0, j, last // 2] = F16_NEG_INF
    elif kind == "masked_row":
        b[s, 0, j, :] = F16_NEG_INF
    elif kind == "bias":
        b[s, 0, j, 0] = np.float16(-0.5).view(np.uint16)
    elif kind == "shared_span":
        # every row of stream s sees the first row's cells: one span, not causal
        for jj in range(w.q_len[s]):
            b[s, 0, jj, :] = b[s, 0, 0, :]
    elif kind == "neg_zero":
        b[s, 0, j, : last + 1 : 3] = F16_NEG_ZERO
    return b


FALLBACK = ["hole", "masked_row", "bias", "shared_span"]
EDIT_CASES = [c for c in CASES if c[0] in ("f16 64 rows", "f16 256-dim 24 rows", "q8_0 6 rows", "q8_0 96 rows",
                                           "q8_0 256-dim 64 rows", "f16 48 rows", "q8_0 24 rows",
                                           "q8_0 256-dim 36 rows", "prefill f16", "prefill q8_0")]


@pytest.mark.parametrize("kind", FALLBACK + ["neg_zero"])
@pytest.mark.parametrize("label,kv_type,D,kv_len,q_len,H,Hkv,bitwise", EDIT_CASES, ids=[c[0] for c in EDIT_CASES])
def test_masks_that_are_not_prefixes(fa, label, kv_type, D, kv_len, q_len, H, Hkv, bitwise, kind):
    w, host, dev = _setup(label, kv_type, D, kv_len, q_len, H, Hkv)
    cap = dev["k"].shape[1]
    bits = _edit(_mask_host(w, cap, w.kv_len), w, kind)
    _say(f"{label}: {kind}")
    got = _call(fa, w, dev, bits)
    if kind == "masked_row":
        # ggml: a row without visible cells has S = 0 and writes zeros; the rest meets the bar
        s = w.S - 1 if w.q_len[-1] > 0 else 0
        j = min(w.q_len[s] - 1, 2)
        assert np.all(got[s, j] == 0.0), label
        got[s, j] = 0.0
    _oracle_check(w, host, got, bits, f"{label} {kind}")
    if kind == "neg_zero":
        ref = _call(fa, w, dev)
        for s, (x, y) in enumerate(zip(_rows(w, got), _rows(w, ref))):
            assert np.array_equal(x, y), (label, s)


def test_llama_mask_without_q_len(fa):
    """The hook's usual call: no q_len array (every stream has n_q rows), mask rows padded."""
    w, host, dev = _setup("no q_len", sa.TYPE_F16, 128, [1000, 2000, 50, 700], [16, 16, 16, 16], 32, 8)
    cap = dev["k"].shape[1]
    bits = _mask_host(w, cap, w.kv_len, pad_rows=48)
    mask = torch.from_numpy(bits).cuda().view(torch.float16)
    out = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), device="cuda")
    fa(dev["q"], dev["k"], dev["v"], out, kv_len=dev["kv_len"], q_len=None, mask_mode=sa.MASK_EXPLICIT, mask=mask)
    ref = torch.full_like(out, float("nan"))
    fa(dev["q"], dev["k"], dev["v"], ref, kv_len=dev["kv_len"], q_len=None, mask_mode=sa.MASK_BLOCK_CAUSAL)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


# Single-stream decode (one row): the dual kernels read the mask row themselves (no pre-pass).
# label, kv_type, D, kv_len, H, Hkv
DECODE_CASES = [
    ("f16 decode", sa.TYPE_F16, 128, 4096, 24, 4),
    ("q8_0 decode", sa.TYPE_Q8_0, 128, 3000, 24, 4),
    ("f16 256-dim decode", sa.TYPE_F16, 256, 4100, 24, 4),
    ("q8_0 256-dim decode", sa.TYPE_Q8_0, 256, 2500, 24, 4),
    ("f16 decode, 48 rows", sa.TYPE_F16, 128, 777, 48, 1),
]


@pytest.mark.parametrize("kind", ["llama", "hole", "hidden_last", "neg_zero"])
@pytest.mark.parametrize("label,kv_type,D,kv_len,H,Hkv", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_single_stream_decode_mask(fa, label, kv_type, D, kv_len, H, Hkv, kind):
    w, host, dev = _setup(label, kv_type, D, [kv_len], [1], H, Hkv)
    cap = dev["k"].shape[1]
    bits = _mask_host(w, cap, w.kv_len)
    last = kv_len  # the row's last visible cell
    if kind == "hole":
        bits[0, 0, 0, last // 3] = F16_NEG_INF
    elif kind == "hidden_last":
        bits[0, 0, 0, last] = F16_NEG_INF
    elif kind == "neg_zero":
        bits[0, 0, 0, : last + 1 : 5] = F16_NEG_ZERO
    _say(f"{label}: {kind}, kv_len {kv_len}")
    got = _call(fa, w, dev, bits)
    _oracle_check(w, host, got, bits, f"{label} {kind}")
    if kind in ("llama", "neg_zero"):
        ref = _call(fa, w, dev)
        assert np.array_equal(got[0, :1], ref[0, :1]), label
    if kind == "hidden_last":
        # the same as the lengths call one cell shorter
        ref = _call(fa, w, dev, kv_len=[kv_len - 1])
        met = oracle.diff_metrics(ref[0, :1].ravel(), got[0, :1].ravel())
        assert met["max_abs"] <= MAX_ABS, met


def test_single_stream_decode_mask_tight_view(fa):
    """The mask row ends one cell past the call's cells, not on a 16-byte piece: its last cells
    are read one by one."""
    w, host, dev = _setup("tight", sa.TYPE_F16, 128, [1000], [1], 24, 4)
    n_kv = 1005
    k = dev["k"][:, :n_kv]
    v = dev["v"][:, :n_kv]
    bits = _mask_host(w, 1024, w.kv_len)
    for kind in ("llama", "hidden_last"):
        b = bits.copy()
        if kind == "hidden_last":
            b[0, 0, 0, 1000] = F16_NEG_INF
        mask = torch.from_numpy(b).cuda().view(torch.float16)[..., :n_kv]
        out = torch.full((1, 1, 24, 128), float("nan"), device="cuda")
        fa(dev["q"], k, v, out, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=sa.MASK_EXPLICIT, mask=mask)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want = oracle.flash_attn_ext(host["q"].astype(np.float32), np.ascontiguousarray(host["k"][:, :n_kv]),
                                     np.ascontiguousarray(host["v"][:, :n_kv]), w.kv_type,
                                     np.ascontiguousarray(b[:, :, :1, :n_kv]))
        met = oracle.diff_metrics(want[0, :1].ravel(), got[0, :1].ravel())
        _say(f"tight view {kind}: max_abs={met['max_abs']:.3e}")
        assert met["max_abs"] <= MAX_ABS and met["rel_l2"] <= REL_L2, (kind, met)


def test_noalloc_with_the_pre_pass_table(fa):
    """The no-allocation entry point holds the pre-pass's table in its scratch: the same output as
    sixi_attn_forward, for a verify batch and a prefill block, twice in a row (the second smaller)."""
    for name, kv_len, q_len in (("verify", [900, 5000, 37, 2000], [16, 16, 9, 16]), ("verify small", [300, 40], [4, 2]),
                                ("prefill", [200, 700], [150, 260]), ("prefill small", [90], [120])):
        w, host, dev = _setup(f"noalloc {name}", sa.TYPE_F16, 128, kv_len, q_len, 24, 4)
        bits = _mask_host(w, dev["k"].shape[1], w.kv_len)
        mask = torch.from_numpy(bits).cuda().view(torch.float16)
        a = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), device="cuda")
        b = torch.full_like(a, float("nan"))
        fa(dev["q"], dev["k"], dev["v"], a, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=sa.MASK_EXPLICIT,
           mask=mask)
        fa(dev["q"], dev["k"], dev["v"], b, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=sa.MASK_EXPLICIT,
           mask=mask, noalloc=True)
        torch.cuda.synchronize()
        _say(f"noalloc {name}")
        assert torch.equal(torch.nan_to_num(a, nan=7.0), torch.nan_to_num(b, nan=7.0)), name
