"""Pins of the oracle's gated-delta-rule verify (oracle.gdn_verify, fa_oracle.c), a restatement
of the reference's GdnOperator::step_token (src/core/core_execution.cpp:254-335) run row by row.

The reference keeps no expected values for the step (its test, tests/test_cuda_kernels.cpp:259-341,
compares its CPU and CUDA forms with each other), so the restatement is pinned by what the delta
rule fixes in closed form.  Each check fails for a plausible slip: the decay applied to the read
(or not), the outer product transposed, y read before the update, beta outside the difference,
a snapshot taken at the wrong row.
"""
import numpy as np
import pytest

import oracle as O


def _orthonormal(n, K, seed):
    rng = np.random.default_rng(seed)
    m, _ = np.linalg.qr(rng.standard_normal((K, K)))
    return m[:, :n].T.astype(np.float32)            # n orthonormal keys of length K


def _one_stream(rows):
    """(q, k, v, alpha, beta) lists of per-row vectors -> arrays [1, n, 1, ...]."""
    q, k, v, a, b = zip(*rows)
    return (np.array(q)[None, :, None], np.array(k)[None, :, None], np.array(v)[None, :, None],
            np.array(a, np.float32)[None, :, None], np.array(b, np.float32)[None, :, None])


def test_delta_rule_stores_values_at_orthonormal_keys():
    # alpha 1, beta 1: after writing v1 at k1 and v2 at k2, S k1 = v1 and S k2 = v2, and the
    # step's y = S q reads the state after the update
    K, HD = 64, 128
    k1, k2 = _orthonormal(2, K, 1)
    rng = np.random.default_rng(2)
    v1, v2 = rng.standard_normal((2, HD)).astype(np.float32)
    rows = [(k2, k1, v1, 1.0, 1.0), (k1, k2, v2, 1.0, 1.0), (k1, k1, v1, 1.0, 1.0)]
    y, st = O.gdn_verify(*_one_stream(rows), np.zeros((1, 1, HD, K), np.float32))
    S = st[0, 0].astype(np.float64)
    np.testing.assert_allclose(S @ k1, v1, atol=2e-6)
    np.testing.assert_allclose(S @ k2, v2, atol=2e-6)
    np.testing.assert_allclose(y[0, 0, 0], 0.0, atol=1e-6)            # row 0 reads k2 after writing k1
    np.testing.assert_allclose(y[0, 1, 0], v1, atol=2e-6)             # row 1 reads k1 after writing k2
    np.testing.assert_allclose(y[0, 2, 0], v1, atol=2e-6)             # rewriting v1 at k1 changes nothing


def test_beta_scales_the_correction_and_alpha_the_old_state():
    K, HD = 64, 64
    (k1,) = _orthonormal(1, K, 3)
    rng = np.random.default_rng(4)
    S0 = rng.standard_normal((HD, K)).astype(np.float32)
    v = rng.standard_normal(HD).astype(np.float32)
    a, b = 0.75, 0.25
    _, st = O.gdn_verify(*_one_stream([(k1, k1, v, a, b)]), S0[None, None])
    sk = S0.astype(np.float64) @ k1
    want = a * S0 + np.outer(b * (v - sk), k1)                         # the reference's form (:318-325)
    np.testing.assert_allclose(st[0, 0], want, atol=2e-6)
    # read back at k1: a Sk + b (v - Sk) -- the decay does not act on the read
    np.testing.assert_allclose(st[0, 0] @ k1, a * sk + b * (v - sk), atol=2e-6)


def test_decay_first_writes_the_value_exactly_and_the_reference_form_does_not():
    K, HD = 64, 64
    (k1,) = _orthonormal(1, K, 5)
    rng = np.random.default_rng(6)
    S0 = rng.standard_normal((HD, K)).astype(np.float32)
    v = rng.standard_normal(HD).astype(np.float32)
    rows = _one_stream([(k1, k1, v, 0.5, 1.0)])
    _, st_ref = O.gdn_verify(*rows, S0[None, None])
    _, st_df = O.gdn_verify(*rows, S0[None, None], decay_first=True)
    sk = S0.astype(np.float64) @ k1
    np.testing.assert_allclose(st_df[0, 0] @ k1, v, atol=2e-6)                       # aS + (v - aSk) k
    np.testing.assert_allclose(st_ref[0, 0] @ k1, v - 0.5 * sk, atol=2e-6)            # aS + (v - Sk) k
    # with alpha 1 the two forms are the same computation
    rows1 = _one_stream([(k1, k1, v, 1.0, 0.3)])
    a1 = O.gdn_verify(*rows1, S0[None, None])
    b1 = O.gdn_verify(*rows1, S0[None, None], decay_first=True)
    assert np.array_equal(a1[0], b1[0]) and np.array_equal(a1[1], b1[1])


def test_pure_decay_is_exact_powers():
    K, HD, n = 64, 64, 5
    rng = np.random.default_rng(7)
    S0 = rng.standard_normal((1, 2, HD, K)).astype(np.float32)
    q = rng.standard_normal((1, n, 2, K)).astype(np.float32)
    k = rng.standard_normal((1, n, 2, K)).astype(np.float32)
    v = rng.standard_normal((1, n, 2, HD)).astype(np.float32)
    y, st = O.gdn_verify(q, k, v, np.full((1, n, 2), 0.5, np.float32), np.zeros((1, n, 2), np.float32), S0)
    assert np.array_equal(st, S0 * np.float32(0.5 ** n))               # beta 0: S_n = 0.5^n S_0, exactly
    np.testing.assert_allclose(y[0, 2, 1], (S0[0, 1].astype(np.float64) * 0.125) @ q[0, 2, 1], rtol=1e-5, atol=1e-6)


def test_snapshot_row_and_ragged_lengths():
    rng = np.random.default_rng(8)
    S, n, G, K, HD = 3, 6, 2, 64, 64
    q = rng.standard_normal((S, n, G, K)).astype(np.float32) / 8
    k = rng.standard_normal((S, n, G, K)).astype(np.float32) / 8
    v = rng.standard_normal((S, n, G, HD)).astype(np.float32)
    al = rng.uniform(0.8, 1.0, (S, n, G)).astype(np.float32)
    be = rng.uniform(0.0, 1.0, (S, n, G)).astype(np.float32)
    S0 = rng.standard_normal((S, G, HD, K)).astype(np.float32)
    q_len, snap = [6, 4, 0], [2, 9, -1]                               # snap clamps to [0, q_len]
    y, st = O.gdn_verify(q, k, v, al, be, S0, q_len, snap)
    # stream 0: the state after 2 rows, while y covers all 6
    y2, st2 = O.gdn_verify(q[:1, :2], k[:1, :2], v[:1, :2], al[:1, :2], be[:1, :2], S0[:1])
    assert np.array_equal(st[0], st2[0]) and np.array_equal(y[0, :2], y2[0])
    assert np.all(np.isfinite(y[0])) and np.all(np.isnan(y[1, 4:])) and np.all(np.isnan(y[2]))
    # stream 1: snap beyond q_len -> the state after its 4 rows; stream 2: no rows -> unchanged
    y4, st4 = O.gdn_verify(q[1:2, :4], k[1:2, :4], v[1:2, :4], al[1:2, :4], be[1:2, :4], S0[1:2])
    assert np.array_equal(st[1], st4[0]) and np.array_equal(y[1, :4], y4[0])
    assert np.array_equal(st[2], S0[2])


def reference_test_inputs(steps=8, G=16, K=64, HD=128):
    """The inputs of the reference's GDN kernel test (tests/test_cuda_kernels.cpp:263-293):
    16 groups, state size 64, head dim 128, 8 steps, alpha 0.9, beta 0.12."""
    iq = np.arange(G * K, dtype=np.int64)
    iv = np.arange(G * HD, dtype=np.int64)
    q = np.stack([np.sin(((st * 19 + iq).astype(np.float32) * np.float32(0.05))) * np.float32(0.2) for st in range(steps)])
    k = np.stack([np.cos(((st * 29 + iq).astype(np.float32) * np.float32(0.04))) * np.float32(0.2) for st in range(steps)])
    v = np.stack([np.sin(((st * 11 + iv).astype(np.float32) * np.float32(0.07))) * np.float32(0.6) for st in range(steps)])
    return (q.astype(np.float32).reshape(1, steps, G, K), k.astype(np.float32).reshape(1, steps, G, K),
            v.astype(np.float32).reshape(1, steps, G, HD), np.full((1, steps, G), 0.9, np.float32),
            np.full((1, steps, G), 0.12, np.float32), np.zeros((1, G, HD, K), np.float32))


def test_reference_test_case_against_float64():
    q, k, v, al, be, S0 = reference_test_inputs()
    y, st = O.gdn_verify(q, k, v, al, be, S0)
    S = np.zeros((16, 128, 64))
    for t in range(8):
        kt, qt = k[0, t].astype(np.float64), q[0, t].astype(np.float64)
        sk = np.einsum("ghs,gs->gh", S, kt)
        S = 0.9 * S + np.einsum("gh,gs->ghs", 0.12 * (v[0, t] - sk), kt)
        np.testing.assert_allclose(y[0, t], np.einsum("ghs,gs->gh", S, qt), atol=1e-6)
    np.testing.assert_allclose(st[0], S, atol=1e-6)
