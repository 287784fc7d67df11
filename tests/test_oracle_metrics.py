"""Pins of the oracle's diff_metrics, the restatement of the reference's compute_diff_metrics
(src/core/numeric.cpp:701-791).

- against the reference function itself, compiled from its own source into oracle/_ref;
- closed forms: a constant offset d gives max-abs = mean-abs = RMSE = |d| and KL = 0 (softmax
  is shift invariant); KL of two 2-element arrays against its textbook value; cosine of
  orthogonal, opposite and zero vectors; the first maximum is the top-1 index;
- non-finite inputs are rejected, as the reference does.
"""
import math

import numpy as np
import pytest

import oracle


def _ref():
    if oracle.ref_numeric() is None:
        pytest.skip("oracle/_ref not built (needs the reference tree; `make -C oracle ref`)")


@pytest.mark.parametrize("seed,n,scale", [(1, 1000, 1.0), (2, 4096, 30.0), (3, 7, 0.01), (4, 100_000, 3.0)])
def test_matches_the_reference_function(seed, n, scale):
    _ref()
    rng = np.random.default_rng(seed)
    r = (rng.standard_normal(n) * scale).astype(np.float32)
    c = (r + rng.standard_normal(n).astype(np.float32) * np.float32(1e-3 * scale)).astype(np.float32)
    got = oracle.diff_metrics(r, c)
    want = oracle.ref_diff_metrics(r, c)
    for key in ("max_abs", "mean_abs", "rmse", "cosine"):
        assert math.isclose(got[key], want[key], rel_tol=1e-9, abs_tol=1e-15), (key, got[key], want[key])
    # KL is a small difference of larger terms: numpy's pairwise float64 sums and the
    # reference's sequential ones differ by ~1e-9 relative at 1e5 elements
    assert math.isclose(got["kl"], want["kl"], rel_tol=1e-6, abs_tol=1e-15), (got["kl"], want["kl"])
    assert got["top1_match"] == want["top1_match"]
    assert got["ref_top1"] == want["ref_top1"] and got["test_top1"] == want["test_top1"]


def test_reference_rejects_non_finite_and_so_does_the_oracle():
    _ref()
    r = np.ones(8, np.float32)
    c = r.copy()
    c[3] = np.nan
    with pytest.raises(ValueError):
        oracle.ref_diff_metrics(r, c)
    with pytest.raises(ValueError):
        oracle.diff_metrics(r, c)
    c[3] = np.inf
    with pytest.raises(ValueError):
        oracle.diff_metrics(r, c)


def test_constant_offset():
    r = np.linspace(-3, 5, 257).astype(np.float32)
    c = (r + np.float32(0.25)).astype(np.float32)  # exact in f32 at these magnitudes
    m = oracle.diff_metrics(r, c)
    assert m["max_abs"] == m["mean_abs"] == m["rmse"] == 0.25
    assert m["kl"] == pytest.approx(0.0, abs=1e-12)  # softmax(x + d) = softmax(x)
    assert m["top1_match"] and m["ref_top1"] == 256


def test_kl_two_elements_textbook():
    r = np.array([0.0, math.log(3.0)], np.float32)  # softmax = (1/4, 3/4)
    c = np.array([0.0, 0.0], np.float32)            # softmax = (1/2, 1/2)
    p = np.array([0.25, 0.75])
    want = float(np.sum(p * np.log(p / 0.5)))
    assert oracle.diff_metrics(r, c)["kl"] == pytest.approx(want, rel=1e-6)


def test_cosine_cases_and_first_maximum():
    assert oracle.diff_metrics([1.0, 0.0], [0.0, 1.0])["cosine"] == 0.0
    assert oracle.diff_metrics([1.0, 2.0], [-1.0, -2.0])["cosine"] == pytest.approx(-1.0)
    assert oracle.diff_metrics([0.0, 0.0], [0.0, 0.0])["cosine"] == 1.0
    assert oracle.diff_metrics([0.0, 0.0], [0.0, 1.0])["cosine"] == 0.0
    m = oracle.diff_metrics([1.0, 5.0, 5.0], [5.0, 1.0, 5.0])
    assert m["ref_top1"] == 1 and m["test_top1"] == 0 and not m["top1_match"]
