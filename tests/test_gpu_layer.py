"""GPU layer prologue (sixi_qk_prologue) and output gate (sixi_attn_gate) against the oracle,
through the C ABI, and the three calls of a Qwen3.8 full-attention layer's core in a row.

Floating-point work in f32: Q after norm and RoPE within max-abs 5e-5 and rel-L2 1e-6 of the
oracle (the angles are the same f32 products on both sides; cos/sin, the sum of squares and
fused multiply-adds round differently by a few ulp).  The stores: V bit-exact (no arithmetic
before the codec); K within one f16 ulp (f16 cache) or one quant step with 99% of the blocks
bit-identical (q8_0), since the f32 value entering the codec may differ in its last bits.
Cells that are not written keep their poisoned bytes.  The gate within rel 1e-6.  The layer
core (prologue, attention, gate) within the attention's bar (max-abs 2e-3, rel-L2 1e-3).
"""
import sys

import numpy as np
import pytest
import torch

import oracle
import sixi_attn as sa

pytestmark = pytest.mark.gpu

Q_MAX_ABS, Q_REL_L2 = 5e-5, 1e-6
MAX_ABS, REL_L2 = 2e-3, 1e-3


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def lib():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    return sa.load_library()


def _inputs(S, R, H, Hkv, D, seed):
    rng = np.random.default_rng(seed)
    qg = (rng.standard_normal((S, R, H, 2 * D)) * 2).astype(np.float32)
    k = (rng.standard_normal((S, R, Hkv, D)) * 3).astype(np.float32)
    v = rng.standard_normal((S, R, Hkv, D)).astype(np.float32)
    wq = rng.uniform(0.3, 1.7, D).astype(np.float32)
    wk = rng.uniform(0.3, 1.7, D).astype(np.float32)
    return qg, k, v, wq, wk


def _poisoned(S, n_cells, Hkv, D, q8, seed):
    rng = np.random.default_rng(seed)
    if q8:
        return rng.integers(0, 256, size=(S, n_cells, Hkv, D // 32 * 34), dtype=np.uint8)
    return rng.integers(0, 1 << 16, size=(S, n_cells, Hkv, D), dtype=np.uint16)


def _dev_cache(c):
    return torch.from_numpy(c.copy()).cuda() if c.dtype == np.uint8 else torch.from_numpy(c.view(np.float16).copy()).cuda()


def _host_cache(t, like):
    a = t.cpu().numpy()
    return a if like.dtype == np.uint8 else a.view(np.uint16)


def _written(S, R, n_cells, kv_len, q_len):
    """(s, cell) pairs the prologue stores."""
    out = []
    for s in range(S):
        ql = R if q_len is None else min(q_len[s], R)
        for j in range(ql):
            c = (0 if kv_len is None else kv_len[s]) + j
            if 0 <= c < n_cells:
                out.append((s, c))
    return out


def _check_k(got, want, cells, q8, D, label):
    mask = np.zeros(got.shape[:2], dtype=bool)
    for s, c in cells:
        mask[s, c] = True
    # untouched cells: bytes unchanged
    assert np.array_equal(got[~mask], want[~mask]), f"{label}: K cells outside the block changed"
    g, w = got[mask], want[mask]
    if not q8:
        gf = oracle.fp16_bits_to_fp32(g).astype(np.float64)
        wf = oracle.fp16_bits_to_fp32(w).astype(np.float64)
        ulp = np.spacing(np.abs(wf).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(gf - wf) <= ulp), f"{label}: K beyond one f16 ulp"
        return
    nb = D // 32
    gb = g.reshape(-1, nb, 34)
    wb = w.reshape(-1, nb, 34)
    same = np.all(gb == wb, axis=-1)
    assert same.mean() >= 0.99, f"{label}: only {same.mean():.4f} of the K blocks identical"
    gd = oracle.dequantize_q8_0(g.ravel(), g.size // 34 * 32).reshape(-1, 32)
    wd = oracle.dequantize_q8_0(w.ravel(), w.size // 34 * 32).reshape(-1, 32)
    dg = oracle.fp16_bits_to_fp32(gb[..., :2].copy().view(np.uint16)).reshape(-1, 1)
    dw = oracle.fp16_bits_to_fp32(wb[..., :2].copy().view(np.uint16)).reshape(-1, 1)
    step = np.maximum(np.abs(dg), np.abs(dw)).astype(np.float64) * 1.01
    assert np.all(np.abs(gd.astype(np.float64) - wd) <= step), f"{label}: K beyond one q8_0 step"


def _run_prologue(S, R, H, Hkv, D, n_cells, kv_len, q_len, q8, n_rot, seed, label, rope_base=1e7, eps=1e-6):
    _say(f"prologue {label}: S={S} R={R} H={H} Hkv={Hkv} D={D} n_cells={n_cells} kv_len={kv_len} "
         f"q_len={q_len} q8={q8} n_rot={n_rot}")
    qg, k, v, wq, wk = _inputs(S, R, H, Hkv, D, seed)
    kc = _poisoned(S, n_cells, Hkv, D, q8, seed + 1)
    vc = _poisoned(S, n_cells, Hkv, D, q8, seed + 2)
    d = {n: torch.from_numpy(a).cuda() for n, a in (("qg", qg), ("k", k), ("v", v), ("wq", wq), ("wk", wk))}
    dkc, dvc = _dev_cache(kc), _dev_cache(vc)
    q_out = torch.full((S, R, H, D), float("nan"), dtype=torch.float32, device="cuda")
    kl = torch.tensor(kv_len, dtype=torch.int32, device="cuda") if kv_len is not None else None
    ql = torch.tensor(q_len, dtype=torch.int32, device="cuda") if q_len is not None else None
    sa.qk_prologue(d["qg"], d["k"], d["v"], d["wq"], d["wk"], q_out, dkc, dvc, kl, ql, eps=eps, rope_base=rope_base,
                   n_rot=n_rot)
    torch.cuda.synchronize()
    want_q, _, want_kc, want_vc = oracle.qk_prologue(qg, k, v, wq, wk, kc, vc, kv_len, q_len, eps, rope_base, n_rot)
    got_q = q_out.cpu().numpy()
    valid = ~np.isnan(want_q)
    assert np.array_equal(np.isnan(got_q), ~valid), f"{label}: rows past q_len written, or rows missing"
    m = oracle.diff_metrics(want_q[valid], got_q[valid])
    _say(f"prologue {label}: q max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert m["max_abs"] <= Q_MAX_ABS and m["rel_l2"] <= Q_REL_L2, m
    got_vc = _host_cache(dvc, vc)
    bad = np.argwhere(got_vc != want_vc)
    assert bad.size == 0, f"{label}: {len(bad)} V bytes differ, first at {bad[:4].tolist()}"
    _check_k(_host_cache(dkc, kc), want_kc, _written(S, R, n_cells, kv_len, q_len), q8, D, label)


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("label,S,R,kv_len,q_len,n_cells", [
    ("decode", 1, 1, [4096], None, 4097),
    ("verify", 4, 16, [0, 100, 5000, 1200], [16, 9, 1, 16], 5100),
    ("far position", 1, 16, [70000], None, 70016),          # angles of positions 70000..70015
    ("past the cache", 2, 8, [60, -3], [8, 8], 64),          # cells >= 64 and < 0 are skipped
    ("prefill chunk", 1, 96, [512], None, 608),
])
def test_prologue_qwen_geometry(q8, label, S, R, kv_len, q_len, n_cells):
    # heads of 256, 24 q-heads, 4 kv-heads, 64 rotated dims, base 1e7, eps 1e-6
    _run_prologue(S, R, 24, 4, 256, n_cells, kv_len, q_len, q8, 64, 11, label)


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("n_rot,rope_base", [(128, 1e4), (0, 1e4), (32, 5e5), (4, 1e6)])
def test_prologue_d128(q8, n_rot, rope_base):
    _run_prologue(3, 5, 8, 2, 128, 300, [0, 37, 290], [5, 2, 5], q8, n_rot, 21 + n_rot, f"D=128 n_rot={n_rot}",
                  rope_base=rope_base)


def test_prologue_without_lengths():
    _run_prologue(2, 4, 4, 2, 256, 8, None, None, False, 256, 31, "no lengths, full rotation")


@pytest.mark.parametrize("q8", [False, True])
def test_prologue_zero_rows(q8, monkeypatch):
    # rows of zeros (pad rows of a ragged block): the norm divides by sqrt(eps) and gives zeros
    real = _inputs

    def zeroed(S, R, H, Hkv, D, seed):
        qg, k, v, wq, wk = real(S, R, H, Hkv, D, seed)
        qg[:, 1::2] = 0.0
        k[:, 1::2] = 0.0
        v[:, 1::2] = 0.0
        return qg, k, v, wq, wk

    monkeypatch.setattr(sys.modules[__name__], "_inputs", zeroed)
    _run_prologue(2, 6, 24, 4, 256, 64, [10, 40], [6, 4], q8, 64, 61, "zero rows")


@pytest.mark.parametrize("D", [128, 256])
def test_gate(D):
    rng = np.random.default_rng(41 + D)
    S, R, H = 3, 7, 6
    out = rng.standard_normal((S, R, H, D)).astype(np.float32)
    qg = (rng.standard_normal((S, R, H, 2 * D)) * 6).astype(np.float32)
    qg[0, 0, 0, D:D + 4] = [0.0, 200.0, -200.0, -90.0]
    q_len = [7, 0, 3]
    _say(f"gate D={D}: S={S} R={R} H={H} q_len={q_len}")
    d_out = torch.from_numpy(out).cuda()
    sa.attn_gate(d_out, torch.from_numpy(qg).cuda(), torch.tensor(q_len, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    got = d_out.cpu().numpy()
    want = oracle.attn_gate(out, qg, q_len)
    assert np.array_equal(got[1], out[1]) and np.array_equal(got[2, 3:], out[2, 3:])
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("kv_type", [sa.TYPE_F16, sa.TYPE_Q8_0])
def test_layer_core(kv_type):
    """prologue -> attention over the updated cache -> gate, against the oracle's three steps."""
    S, R, H, Hkv, D, n_cells = 3, 16, 24, 4, 256, 2304
    kv_len, q_len = [2000, 17, 700], [16, 16, 5]
    q8 = kv_type == sa.TYPE_Q8_0
    _say(f"layer core: kv_type={kv_type} S={S} kv_len={kv_len} q_len={q_len}")
    qg, k, v, wq, wk = _inputs(S, R, H, Hkv, D, 51)
    rng = np.random.default_rng(52)
    zero = np.zeros((S, n_cells, Hkv, D // 32 * 34), np.uint8) if q8 else np.zeros((S, n_cells, Hkv, D), np.uint16)
    # history: cells before kv_len hold earlier tokens' K (unit-RMS rows, as after the norm) and V
    hk = rng.standard_normal((S, n_cells, Hkv, D)).astype(np.float32)
    hv = rng.standard_normal((S, n_cells, Hkv, D)).astype(np.float32)
    kc = oracle.kv_write(hk, zero, None, None)
    vc = oracle.kv_write(hv, zero, None, None)
    dkc, dvc = _dev_cache(kc), _dev_cache(vc)
    d_qg = torch.from_numpy(qg).cuda()
    q_out = torch.zeros((S, R, H, D), dtype=torch.float32, device="cuda")
    kl = torch.tensor(kv_len, dtype=torch.int32, device="cuda")
    ql = torch.tensor(q_len, dtype=torch.int32, device="cuda")
    sa.qk_prologue(d_qg, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), torch.from_numpy(wq).cuda(),
                   torch.from_numpy(wk).cuda(), q_out, dkc, dvc, kl, ql)
    out = torch.full((S, R, H, D), float("nan"), dtype=torch.float32, device="cuda")
    fa = sa.FlashAttnExt()
    fa(q_out, dkc, dvc, out, kv_len=kl, q_len=ql)
    sa.attn_gate(out, d_qg, ql)
    torch.cuda.synchronize()
    got = out.cpu().numpy()

    wq_out, _, wkc, wvc = oracle.qk_prologue(qg, k, v, wq, wk, kc, vc, kv_len, q_len)
    n_kv = max(a + b for a, b in zip(kv_len, q_len))
    mask = oracle.build_kq_mask(n_kv, R, np.array(kv_len), np.array(q_len), True)
    att = oracle.flash_attn_ext(np.nan_to_num(wq_out), np.ascontiguousarray(wkc[:, :n_kv]),
                                np.ascontiguousarray(wvc[:, :n_kv]), kv_type, mask)
    want = oracle.attn_gate(att, qg, q_len)
    g = np.concatenate([got[s, :q_len[s]].ravel() for s in range(S)])
    r = np.concatenate([want[s, :q_len[s]].ravel() for s in range(S)])
    m = oracle.diff_metrics(r, g)
    _say(f"layer core kv_type={kv_type}: max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert np.all(np.isfinite(g))
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m


@pytest.mark.parametrize("kv_type", [sa.TYPE_F16, sa.TYPE_Q8_0])
def test_layer_core_f16_q_and_fused_gate(kv_type):
    """The same layer with the gate fused into the attention and, over an f16 cache, the
    prologue's Q written in f16 (the f32 Q rounded to nearest even, bit for bit): the output
    equals the f32-Q, three-call layer bit for bit (the attention rounds Q to f16 itself).  Over
    a q8_0 cache, whose Q conversion starts from the f32 values, the prologue refuses an f16 Q
    and the f32-Q layer with the fused gate meets the oracle's bar."""
    S, R, H, Hkv, D, n_cells = 3, 16, 24, 4, 256, 2304
    kv_len, q_len = [2000, 17, 700], [16, 16, 5]
    q8 = kv_type == sa.TYPE_Q8_0
    _say(f"layer f16 Q + fused gate: kv_type={kv_type}")
    qg, k, v, wq, wk = _inputs(S, R, H, Hkv, D, 53)
    rng = np.random.default_rng(54)
    zero = np.zeros((S, n_cells, Hkv, D // 32 * 34), np.uint8) if q8 else np.zeros((S, n_cells, Hkv, D), np.uint16)
    hk = rng.standard_normal((S, n_cells, Hkv, D)).astype(np.float32)
    hv = rng.standard_normal((S, n_cells, Hkv, D)).astype(np.float32)
    kc = oracle.kv_write(hk, zero, None, None)
    vc = oracle.kv_write(hv, zero, None, None)
    dkc, dvc = _dev_cache(kc), _dev_cache(vc)
    d_qg, dk, dv = torch.from_numpy(qg).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    dwq, dwk = torch.from_numpy(wq).cuda(), torch.from_numpy(wk).cuda()
    kl = torch.tensor(kv_len, dtype=torch.int32, device="cuda")
    ql = torch.tensor(q_len, dtype=torch.int32, device="cuda")
    fa = sa.FlashAttnExt()
    q32 = torch.zeros((S, R, H, D), dtype=torch.float32, device="cuda")
    sa.qk_prologue(d_qg, dk, dv, dwq, dwk, q32, dkc, dvc, kl, ql)
    ref = torch.full((S, R, H, D), float("nan"), dtype=torch.float32, device="cuda")
    fa(q32, dkc, dvc, ref, kv_len=kl, q_len=ql)
    sa.attn_gate(ref, d_qg, ql)
    q16 = torch.zeros((S, R, H, D), dtype=torch.float16, device="cuda")
    got = torch.full_like(ref, float("nan"))
    if q8:
        assert sa.qk_prologue(d_qg, dk, dv, dwq, dwk, q16, dkc, dvc, kl, ql, check=False) == sa.E_INVALID_ARGUMENT
        fa(q32, dkc, dvc, got, kv_len=kl, q_len=ql, gate=d_qg)
    else:
        sa.qk_prologue(d_qg, dk, dv, dwq, dwk, q16, dkc, dvc, kl, ql)
        fa(q16, dkc, dvc, got, kv_len=kl, q_len=ql, gate=d_qg)
    torch.cuda.synchronize()
    r, g = ref.cpu().numpy(), got.cpu().numpy()
    for s in range(S):
        if not q8:
            assert torch.equal(q16[s, :q_len[s]], q32[s, :q_len[s]].half()), s
        assert np.array_equal(g[s, :q_len[s]], r[s, :q_len[s]]), s
    wq_out, _, wkc, wvc = oracle.qk_prologue(qg, k, v, wq, wk, kc, vc, kv_len, q_len)
    n_kv = max(a + b for a, b in zip(kv_len, q_len))
    mask = oracle.build_kq_mask(n_kv, R, np.array(kv_len), np.array(q_len), True)
    att = oracle.flash_attn_ext(np.nan_to_num(wq_out), np.ascontiguousarray(wkc[:, :n_kv]),
                                np.ascontiguousarray(wvc[:, :n_kv]), kv_type, mask)
    want = oracle.attn_gate(att, qg, q_len)
    gg = np.concatenate([g[s, :q_len[s]].ravel() for s in range(S)])
    ww = np.concatenate([want[s, :q_len[s]].ravel() for s in range(S)])
    m = oracle.diff_metrics(ww, gg)
    _say(f"layer f16 Q kv_type={kv_type}: max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m
