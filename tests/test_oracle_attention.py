"""Pins of the oracle's attention (the ggml CPU flash_attn_ext restatement).

Nothing here retypes the oracle's formula: each check is an independent float64 brute
force, a case that reduces to a textbook result, an invariance, or an equivalence between
two different code paths of the oracle (explicit mask vs. truncated views).
"""
import numpy as np
import pytest

import oracle

RNG = np.random.default_rng(1234)


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16)


def brute_f16(q, k16, v16, kv_len, q_len, causal=True, scale=None):
    """float64 softmax attention on Q rounded to f16 (ggml converts Q to K's dot type)."""
    S, nq, H, D = q.shape
    Hkv = k16.shape[2]
    G = H // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    q16 = _f16(q).astype(np.float64)
    out = np.zeros((S, nq, H, D))
    for s in range(S):
        for j in range(q_len[s]):
            n = kv_len[s] + (j + 1 if causal else q_len[s])
            for h in range(H):
                g = h // G
                K = k16[s, :n, g].astype(np.float64)
                V = v16[s, :n, g].astype(np.float64)
                sc = K @ q16[s, j, h] * scale
                p = np.exp(sc - sc.max())
                out[s, j, h] = p @ V / p.sum()
    return out


def _case(S=2, nq=5, H=6, Hkv=2, D=128, n_kv=40, kv_len=(20, 31)):
    q = RNG.standard_normal((S, nq, H, D)).astype(np.float32)
    k = _f16(RNG.standard_normal((S, n_kv, Hkv, D)))
    v = _f16(RNG.standard_normal((S, n_kv, Hkv, D)))
    return q, k, v, list(kv_len), [nq] * S


def _run(q, k, v, kv_len, q_len, causal=True, **kw):
    mask = oracle.build_kq_mask(k.shape[1], q.shape[1], kv_len, q_len, causal)
    return oracle.flash_attn_ext(q, k.view(np.uint16), v.view(np.uint16), oracle.F16, mask, **kw)


@pytest.mark.parametrize("D,H,Hkv", [(128, 6, 2), (128, 24, 4), (256, 8, 1), (64, 4, 4)])
def test_f16_kv_matches_float64_brute_force(D, H, Hkv):
    q, k, v, kl, ql = _case(H=H, Hkv=Hkv, D=D)
    got = _run(q, k, v, kl, ql)
    want = brute_f16(q, k, v, kl, ql)
    assert np.max(np.abs(got - want)) < 2e-5


def test_q8_0_kv_matches_float64_brute_force():
    S, nq, H, Hkv, D, n_kv = 2, 3, 6, 2, 128, 33
    q = RNG.standard_normal((S, nq, H, D)).astype(np.float32)
    kf = RNG.standard_normal((S, n_kv, Hkv, D)).astype(np.float32)
    vf = RNG.standard_normal((S, n_kv, Hkv, D)).astype(np.float32)
    kb = oracle.quantize_q8_0(kf).reshape(S, n_kv, Hkv, D // 32 * 34)
    vb = oracle.quantize_q8_0(vf).reshape(S, n_kv, Hkv, D // 32 * 34)
    kl, ql = [10, 30], [nq] * S
    mask = oracle.build_kq_mask(n_kv, nq, kl, ql, True)
    got = oracle.flash_attn_ext(q, kb, vb, oracle.Q8_0, mask)
    # float64: Q is quantized to q8_0 exactly as ggml does, then every product is exact
    kd = oracle.dequantize_q8_0(kb, kf.size).reshape(kf.shape).astype(np.float64)
    vd = oracle.dequantize_q8_0(vb, vf.size).reshape(vf.shape).astype(np.float64)
    qd = oracle.dequantize_q8_0(oracle.quantize_q8_0(q), q.size).reshape(q.shape).astype(np.float64)
    G = H // Hkv
    for s in range(S):
        for j in range(nq):
            n = kl[s] + j + 1
            for h in range(H):
                sc = kd[s, :n, h // G] @ qd[s, j, h] / np.sqrt(D)
                p = np.exp(sc - sc.max())
                want = p @ vd[s, :n, h // G] / p.sum()
                assert np.max(np.abs(got[s, j, h] - want)) < 2e-5


def test_single_cell_returns_that_value_row():
    q, k, v, _, _ = _case(S=1, nq=1, n_kv=8)
    got = _run(q, k, v, [0], [1])
    assert np.array_equal(got[0, 0], v[0, 0, np.arange(6) // 3].astype(np.float32))


def test_equal_scores_give_mean_of_visible_values():
    q, k, v, kl, ql = _case()
    q[:] = 0.0
    got = _run(q, k, v, kl, ql)
    G = 3
    for s in range(2):
        for j in range(5):
            n = kl[s] + j + 1
            want = v[s, :n].astype(np.float64).mean(axis=0)[np.arange(6) // G]
            assert np.max(np.abs(got[s, j] - want)) < 1e-5


def test_dominant_key_selects_its_value_row():
    q, k, v, kl, ql = _case(S=1, nq=1, kv_len=(17,))
    k[0, 7, :, :] = _f16(8.0 * np.sign(q[0, 0, 0]))  # kv-head 0: key 7 aligned with q-head 0
    got = _run(q, k, v, kl, ql)
    assert np.max(np.abs(got[0, 0, 0] - v[0, 7, 0].astype(np.float32))) < 1e-4


def test_key_permutation_invariance():
    q, k, v, kl, ql = _case(S=1, nq=1, n_kv=64, kv_len=(63,))
    perm = RNG.permutation(64)
    a = _run(q, k, v, kl, ql)
    b = _run(q, k[:, perm].copy(), v[:, perm].copy(), kl, ql)
    assert np.max(np.abs(a - b)) < 1e-6


def test_q_scale_reciprocity_is_exact_for_powers_of_two():
    q, k, v, kl, ql = _case()
    a = _run(q, k, v, kl, ql)
    b = _run(q * 2.0, k, v, kl, ql, scale=1.0 / np.sqrt(128) / 2.0)
    assert np.array_equal(a, b)


def test_explicit_mask_equals_truncated_views_bitwise():
    """Masked cells are skipped, so a row over the full view with the llama mask equals the
    same row over a view truncated to its visible cells, bit for bit."""
    q, k, v, kl, ql = _case()
    full = _run(q, k, v, kl, ql)
    for s in range(2):
        for j in range(5):
            n = kl[s] + j + 1
            row = oracle.flash_attn_ext(np.ascontiguousarray(q[s:s + 1, j:j + 1]),
                                        np.ascontiguousarray(k[s:s + 1, :n]).view(np.uint16),
                                        np.ascontiguousarray(v[s:s + 1, :n]).view(np.uint16), oracle.F16, None)
            assert np.array_equal(full[s, j], row[0, 0])


def test_mask_builder_semantics():
    m = oracle.build_kq_mask(12, 4, [3, 0], [2, 4], True).view(np.float16).astype(np.float32)
    vis = np.isfinite(m)
    assert vis[0, 0, 0].tolist() == [True] * 4 + [False] * 8      # row 0 of stream 0 sees cells 0..3
    assert vis[0, 0, 1].tolist() == [True] * 5 + [False] * 7
    assert not vis[0, 0, 2:].any()                                 # rows past q_len see nothing
    assert vis[1, 0, 3].tolist() == [True] * 4 + [False] * 8
    nc = oracle.build_kq_mask(12, 4, [3, 0], [2, 4], False).view(np.float16).astype(np.float32)
    assert np.isfinite(nc[0, 0, 0]).sum() == 5 and np.isfinite(nc[0, 0, 1]).sum() == 5


def test_workload_mask_builder_matches_the_oracle():
    """The package's numpy mask (used by bench.py's explicit-mask timing) equals the oracle's,
    bit for bit, on ragged streams, empty blocks and both mask kinds."""
    from sixi_attn import workloads as wl

    for kl, ql, n_kv, n_q in (([3, 0], [2, 4], 12, 4), ([700, 5, 0, 31], [16, 1, 0, 16], 768, 16), ([0], [1], 1, 1)):
        for causal in (True, False):
            want = oracle.build_kq_mask(n_kv, n_q, kl, ql, causal)
            got = wl.kq_mask(n_kv, n_q, kl, ql, causal)
            assert got.shape == want.shape and got.dtype == np.uint16
            assert np.array_equal(got, want)
    with pytest.raises(ValueError):
        wl.kq_mask(10, 4, [8], [3])


def test_poisoned_cells_past_the_length_are_never_used():
    q, k, v, kl, ql = _case()
    a = _run(q, k, v, kl, ql)
    k2, v2 = k.copy(), v.copy()
    for s in range(2):
        k2[s, kl[s] + ql[s]:] = np.float16(np.nan)
        v2[s, kl[s] + ql[s]:] = np.float16(np.nan)
    assert np.array_equal(a, _run(q, k2, v2, kl, ql))


def test_simd_and_scalar_paths_are_bitwise_identical():
    lib = oracle.load()
    if not lib.oracle_have_simd():
        pytest.skip("oracle built without AVX2/F16C/FMA")
    q, k, v, kl, ql = _case(nq=6, n_kv=70, kv_len=(50, 64))
    outs = []
    for simd in (1, 0):
        lib.oracle_set_simd(simd)
        outs.append([_run(q, k, v, kl, ql), _run(q, k, v, kl, ql, v_acc_f16=True)])
    lib.oracle_set_simd(1)
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_f16_accumulator_is_the_upstream_one_row_kernel():
    """With V accumulated in f16 (ggml's one-row kernel) the error grows with the length;
    with f32 it stays at f32 rounding.  Both are within the documented bounds of float64."""
    q, k, v, kl, ql = _case(S=1, nq=2, n_kv=2048, kv_len=(2046,))
    want = brute_f16(q, k, v, kl, ql)
    e32 = oracle.diff_metrics(want, _run(q, k, v, kl, ql))
    e16 = oracle.diff_metrics(want, _run(q, k, v, kl, ql, v_acc_f16=True))
    assert e32["rel_l2"] < 2e-5
    assert 1e-4 < e16["rel_l2"] < 5e-2
