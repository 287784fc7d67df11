"""Pins of the oracle's layer prologue / epilogue (oracle.rms_norm, rope_neox, qk_prologue,
attn_gate) by closed forms and invariants.

The ops are upstream llama.cpp's (pinned at a691b234, scripts/build_llamacpp.sh:12; not in the
reference tree, which holds no vectors for them), applied to the qwen35 layers of
configs/qwen3.8-27b-ud-q4-k-xl.sixi.  Each check is chosen so that a plausible slip fails it:
eps outside the root, a missing weight, the interleaved (GPT-J) pairing instead of NEOX, a sign
flip in either half of the rotation, a wrong frequency exponent, per-pair positions, a gate
taken from the query half.
"""
import numpy as np
import pytest

import oracle as O

BASE, N_ROT, EPS = 1e7, 64, 1e-6


def _theta64(p, i, base=BASE, n_rot=N_ROT):
    return p * base ** (-2.0 * i / n_rot)


def test_theta_scale_is_f32_power():
    ts = O.rope_theta_scale(BASE, N_ROT)
    exact = BASE ** (-2.0 / N_ROT)
    assert ts.dtype == np.float32
    assert abs(float(ts) - exact) <= np.spacing(np.float32(exact))
    assert O.rope_theta_scale(BASE, 0) == np.float32(1.0)


def test_rms_norm_constant_row_closed_form():
    # a row of constant c: y = c / sqrt(c^2 + eps) * w -- eps sits under the root, added to the mean
    D = 256
    w = np.linspace(0.5, 1.5, D).astype(np.float32)
    for c, eps in ((1e-3, 1e-6), (2.0, 1e-6), (-3.0, 0.5)):
        y = O.rms_norm(np.full((1, D), c, np.float32), w, eps)
        ref = c / np.sqrt(c * c + eps) * w.astype(np.float64)
        np.testing.assert_allclose(y[0], ref, rtol=2e-6)


def test_rms_norm_unit_rms_and_direction():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 128)).astype(np.float32) * 3
    w = rng.uniform(0.5, 2.0, 128).astype(np.float32)
    y = O.rms_norm(x, w, 0.0).astype(np.float64) / w
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, rtol=1e-6)
    # the same direction as x
    cos = np.sum(y * x, -1) / np.linalg.norm(y, axis=-1) / np.linalg.norm(x, axis=-1)
    np.testing.assert_allclose(cos, 1.0, rtol=1e-6)


def test_rope_position_zero_is_identity_and_tail_untouched():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 3, 4, 256)).astype(np.float32)
    pos = np.array([[0, 0, 0], [5, 600, 70000]])
    y = O.rope_neox(x, pos, N_ROT, O.rope_theta_scale(BASE, N_ROT))
    assert np.array_equal(y[0], x[0])
    assert np.array_equal(y[..., N_ROT:], x[..., N_ROT:])
    assert not np.array_equal(y[1, :, :, :N_ROT], x[1, :, :, :N_ROT])


@pytest.mark.parametrize("p", [1, 7, 33])
def test_rope_unit_vectors_neox_pairs(p):
    # e_i -> (cos t_i) e_i + (sin t_i) e_{i+h};  e_{i+h} -> -(sin t_i) e_i + (cos t_i) e_{i+h}
    D, half = 256, N_ROT // 2
    ts = O.rope_theta_scale(BASE, N_ROT)
    eye = np.eye(D, dtype=np.float32)[None, None]                  # [1, 1, D, D]: head d is e_d
    y = O.rope_neox(eye, np.array([[p]]), N_ROT, ts)[0, 0].astype(np.float64)
    for i in (0, 1, 5, half - 1):
        t = _theta64(p, i)
        row = y[i]
        assert abs(row[i] - np.cos(t)) < 2e-6 and abs(row[i + half] - np.sin(t)) < 2e-6
        others = np.delete(row, [i, i + half])
        assert np.all(others == 0)
        row2 = y[i + half]
        assert abs(row2[i] + np.sin(t)) < 2e-6 and abs(row2[i + half] - np.cos(t)) < 2e-6


def test_rope_first_pair_exact_angle_at_large_position():
    # t_0 is the position itself (no product), so even at 70000 the first pair is cos/sin(p)
    x = np.zeros((1, 1, 1, 256), np.float32)
    x[..., 0] = 1.0
    y = O.rope_neox(x, np.array([[70000]]), N_ROT, O.rope_theta_scale(BASE, N_ROT))
    assert abs(y[0, 0, 0, 0] - np.cos(70000.0)) < 1e-6
    assert abs(y[0, 0, 0, N_ROT // 2] - np.sin(70000.0)) < 1e-6


def test_rope_preserves_pair_norms_and_relative_positions():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 1, 1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 1, 1, 128)).astype(np.float32)
    ts = O.rope_theta_scale(1e4, 128)
    half = 64
    yq = O.rope_neox(q, np.array([[11]]), 128, ts)
    n_in = q[..., :half] ** 2 + q[..., half:] ** 2
    n_out = yq[..., :half] ** 2 + yq[..., half:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)

    def score(pq, pk):
        a = O.rope_neox(q, np.array([[pq]]), 128, ts).astype(np.float64)
        b = O.rope_neox(k, np.array([[pk]]), 128, ts).astype(np.float64)
        return float(np.sum(a * b))

    # <rope(q, p), rope(k, p')> depends on p - p' only (every pair uses the same position)
    s0 = score(9, 4)
    for shift in (1, 3, 20):
        assert abs(score(9 + shift, 4 + shift) - s0) < 1e-4


def test_gate_closed_forms():
    rng = np.random.default_rng(4)
    out = rng.standard_normal((2, 3, 4, 128)).astype(np.float32)
    qg = rng.standard_normal((2, 3, 4, 256)).astype(np.float32)
    qg[..., 128:] = 0.0                                            # sigmoid(0) = 1/2 exactly
    assert np.array_equal(O.attn_gate(out, qg), out * np.float32(0.5))
    qg[..., 128:] = 100.0                                          # sigmoid -> 1
    assert np.array_equal(O.attn_gate(out, qg), out)
    qg[..., 128:] = -200.0                                         # sigmoid -> 0 (e^200 overflows f32)
    assert np.all(O.attn_gate(out, qg) == 0)
    # interior points: sigmoid(ln 3) = 3/4 and sigmoid(-ln 3) = 1/4 (a slip such as
    # sigmoid(g/2) gives 0.634 and 0.366)
    ones = np.ones_like(out)
    qg[..., 128:] = np.float32(np.log(3.0))
    np.testing.assert_allclose(O.attn_gate(ones, qg), 0.75, rtol=2e-7)
    qg[..., 128:] = np.float32(-np.log(3.0))
    np.testing.assert_allclose(O.attn_gate(ones, qg), 0.25, rtol=5e-7)
    qg[..., :128] = 1e9                                            # the query half plays no part
    qg[..., 128:] = 0.0
    assert np.array_equal(O.attn_gate(out, qg, q_len=[3, 1])[1, 1:], out[1, 1:])


def test_qk_prologue_positions_follow_kv_len():
    # row j of a stream with kv_len = N is the row 0 of a stream with kv_len = N + j
    rng = np.random.default_rng(5)
    S, R, H, Hkv, D = 2, 4, 2, 1, 128
    qg = rng.standard_normal((S, R, H, 2 * D)).astype(np.float32)
    k = rng.standard_normal((S, R, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((S, R, Hkv, D)).astype(np.float32)
    wq = rng.uniform(0.5, 1.5, D).astype(np.float32)
    wk = rng.uniform(0.5, 1.5, D).astype(np.float32)
    kc = np.zeros((S, 16, Hkv, D), np.uint16)
    q, kr, kc2, vc2 = O.qk_prologue(qg, k, v, wq, wk, kc, kc.copy(), kv_len=[3, 9], q_len=[4, 2], n_rot=D)
    for j in range(2):
        q1, kr1, _, _ = O.qk_prologue(qg[:1, j:j + 1], k[:1, j:j + 1], v[:1, j:j + 1], wq, wk, kc[:1], kc[:1],
                                      kv_len=[3 + j], n_rot=D)
        assert np.array_equal(q1[0, 0], q[0, j]) and np.array_equal(kr1[0, 0], kr[0, j])
    assert np.all(np.isnan(q[1, 2:]))
    # V is stored unnormalised in cells kv_len .. kv_len + q_len - 1, nothing else changes
    assert np.array_equal(O.fp16_bits_to_fp32(vc2[0, 3:7]), v[0].astype(np.float16).astype(np.float32))
    assert np.all(vc2[0, :3] == 0) and np.all(vc2[0, 7:] == 0) and np.all(vc2[1, 11:] == 0)
