"""GPU gated-delta-rule verify (sixi_gdn_verify) against the oracle, through the C ABI.

The bar is the reference's own for its GPU step (tests/test_cuda_kernels.cpp:330-339): max-abs
below 1e-4 and cosine above 0.99999 on y and on the state; here also rel-L2 below 1e-5.  Sums over
the state columns run in a different order than the reference's serial loops (partial sums of 16
columns, then a lane tree), so results agree to f32 rounding, not bitwise; repeated launches are
bitwise identical, as the reference's test requires of its kernel.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
import sixi_attn as sa
from test_oracle_gdn import reference_test_inputs

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def lib():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    return sa.load_library()


def _inputs(S, n, G, K, HD, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((S, n, G, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)                     # unit keys, as after the l2 norm
    q = rng.standard_normal((S, n, G, K)) / np.sqrt(K)
    v = rng.standard_normal((S, n, G, HD))
    al = rng.uniform(0.8, 1.0, (S, n, G))
    be = rng.uniform(0.0, 1.0, (S, n, G))
    S0 = rng.standard_normal((S, G, HD, K)) * 0.5
    return [x.astype(np.float32) for x in (q, k, v, al, be, S0)]


def _check(got, want, label):
    m = oracle.diff_metrics(want, got)
    _say(f"{label}: max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e} cos={m['cosine']:.7f}")
    assert np.all(np.isfinite(got)), label
    assert m["max_abs"] < 1e-4 and m["cosine"] > 0.99999 and m["rel_l2"] < 1e-5, (label, m)


def _run(q, k, v, al, be, S0, q_len=None, snap=None, decay_first=False, in_place=True, label=""):
    S, n, G, K = q.shape
    HD = v.shape[-1]
    _say(f"gdn {label}: S={S} n={n} G={G} K={K} HD={HD} q_len={q_len} snap={snap} decay_first={decay_first} "
         f"in_place={in_place}")
    d = [torch.from_numpy(x).cuda() for x in (q, k, v, al, be)]
    st_in = torch.from_numpy(S0).cuda()
    st_out = st_in if in_place else torch.full_like(st_in, float("nan"))
    y = torch.full((S, n, G, HD), float("nan"), dtype=torch.float32, device="cuda")
    ql = torch.tensor(q_len, dtype=torch.int32, device="cuda") if q_len is not None else None
    sn = torch.tensor(snap, dtype=torch.int32, device="cuda") if snap is not None else None
    sa.gdn_verify(*d, y, st_in, None if in_place else st_out, ql, sn, decay_first)
    torch.cuda.synchronize()
    want_y, want_st = oracle.gdn_verify(q, k, v, al, be, S0, q_len, snap, decay_first)
    got_y = y.cpu().numpy()
    assert np.array_equal(np.isnan(got_y), np.isnan(want_y)), f"{label}: rows past q_len written or missing"
    valid = ~np.isnan(want_y)
    _check(got_y[valid], want_y[valid], f"{label} y")
    _check(st_out.cpu().numpy(), want_st, f"{label} state")
    return got_y, st_out.cpu().numpy()


def test_reference_kernel_test_case():
    """tests/test_cuda_kernels.cpp:259-341: 16 groups, state 64, head 128, 8 steps."""
    args = reference_test_inputs()
    y1, s1 = _run(*args, label="reference test case")
    y2, s2 = _run(*args, label="reference test case, again")
    assert np.array_equal(y1, y2) and np.array_equal(s1, s2)        # bitwise repeatable


@pytest.mark.parametrize("decay_first", [False, True])
def test_qwen_verify_block(decay_first):
    # 48 value heads of 128 with 128-dim keys (ssm_time_step_rank 48, ssm_state_size 128), 16 rows
    args = _inputs(6, 16, 48, 128, 128, 11)
    _run(*args, q_len=[16, 16, 9, 1, 0, 16], snap=[16, 3, 9, 0, 0, 15], decay_first=decay_first,
         label="qwen verify")


@pytest.mark.parametrize("K,HD", [(64, 64), (64, 128), (128, 64)])
def test_other_shapes_out_of_place(K, HD):
    args = _inputs(3, 5, 7, K, HD, 20 + K + HD)
    _run(*args, q_len=[5, 2, 4], in_place=False, label=f"K={K} HD={HD}")


def test_long_block_several_staging_passes():
    args = _inputs(2, 40, 4, 128, 128, 31)                           # 16 + 16 + 8 rows
    _run(*args, q_len=[40, 33], snap=[17, 33], label="40 rows")


@pytest.mark.parametrize("decay_first", [False, True])
def test_several_items_per_work_group(decay_first):
    # 32 streams x 48 groups x 2 halves = 3072 items of 64 state rows: more than the work-groups
    # that fit the device at once (768 on MI355X), so each work-group runs several items and reads
    # the next item's state while it computes the current one; ragged lengths (0, 1, a chunk and a
    # half, every row), snapshot rows anywhere in the block, in place
    S, n, G = 32, 24, 48
    args = _inputs(S, n, G, 128, 128, 71 + int(decay_first))
    rng = np.random.default_rng(72 + int(decay_first))
    q_len = [int(x) for x in rng.integers(0, n + 1, S)]
    q_len[:4] = [0, 1, n, 16]
    snap = [int(rng.integers(0, ql + 1)) for ql in q_len]
    snap[2:4] = [17, 16]
    _run(*args, q_len=q_len, snap=snap, decay_first=decay_first, label="3072 items")


def test_strided_views():
    # ggml views that are not packed: q and k stored group-major ([S][G][n][K] seen as [S][n][G][K]),
    # v, y and both states in padded rows, alpha and beta every other float; out of place, so the
    # padding of y and of the output state must stay untouched; 16 streams x 48 groups = 1536 items
    # (several per work-group, the XCD pairing on), blocks of up to 20 rows
    S, n, G, K, HD = 16, 20, 48, 128, 128
    q, k, v, al, be, S0 = _inputs(S, n, G, K, HD, 81)
    rng = np.random.default_rng(82)
    q_len = [int(x) for x in rng.integers(0, n + 1, S)]
    q_len[:3] = [n, 0, 16]
    snap = [int(rng.integers(0, ql + 1)) for ql in q_len]
    snap[0] = 17

    def dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).cuda()

    def group_major(x):
        return dev(x.transpose(0, 2, 1, 3)).permute(0, 2, 1, 3)

    def padded(x, pad, fill=0.0):
        buf = torch.full(x.shape[:-1] + (x.shape[-1] + pad,), fill, dtype=torch.float32, device="cuda")
        buf[..., :x.shape[-1]] = dev(x)
        return buf, buf[..., :x.shape[-1]]

    def every_other(x):
        buf = torch.zeros(x.shape[:-1] + (2 * x.shape[-1],), dtype=torch.float32, device="cuda")
        buf[..., ::2] = dev(x)
        return buf[..., ::2]

    _, vd = padded(v, 4)
    _, st_in = padded(S0, 16)
    y_buf, yd = padded(np.full(v.shape, np.nan, np.float32), 8, float("nan"))
    so_buf, st_out = padded(np.full(S0.shape, np.nan, np.float32), 32, float("nan"))
    _say(f"gdn strided views: S={S} n={n} G={G} q_len={q_len} snap={snap}")
    sa.gdn_verify(group_major(q), group_major(k), vd, every_other(al), every_other(be), yd, st_in, st_out,
                  torch.tensor(q_len, dtype=torch.int32, device="cuda"),
                  torch.tensor(snap, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    want_y, want_st = oracle.gdn_verify(q, k, v, al, be, S0, q_len, snap)
    got_y = yd.cpu().numpy()
    assert np.array_equal(np.isnan(got_y), np.isnan(want_y)), "rows past q_len written or missing"
    valid = ~np.isnan(want_y)
    _check(got_y[valid], want_y[valid], "strided views y")
    _check(st_out.cpu().numpy(), want_st, "strided views state")
    assert torch.isnan(y_buf[..., HD:]).all() and torch.isnan(so_buf[..., K:]).all(), "padding written"


def test_no_lengths():
    _run(*_inputs(2, 3, 3, 128, 128, 41), label="no lengths")


def test_extreme_gates():
    # alpha 0 resets the state to the row's write, alpha 1 keeps it; beta 0 writes nothing, beta 1
    # writes the whole correction
    q, k, v, al, be, S0 = _inputs(2, 8, 6, 128, 128, 51)
    al[:, ::2] = 0.0
    al[:, 1::4] = 1.0
    be[:, :, ::3] = 0.0
    be[:, :, 1::3] = 1.0
    _run(q, k, v, al, be, S0, q_len=[8, 5], snap=[8, 4], label="alpha 0/1, beta 0/1")


@pytest.mark.parametrize("decay_first", [False, True])
def test_decays_that_leave_the_carried_scale_range(decay_first):
    # the kernel carries the state as a scalar times a matrix and folds the scalar in when the
    # running product of the gates leaves [2^-30, 2^30]: gates of 2^-20 (the product leaves the range
    # at the second), 2^-40 (at once), 0 (a reset) and 4 (growth, the product passes 2^30 at the
    # 16th row), across staging passes, against the oracle's step by step recurrence
    q, k, v, al, be, S0 = _inputs(4, 40, 6, 128, 128, 61)
    al[0, 3:6] = 2.0 ** -20
    al[1, 10] = 2.0 ** -40
    al[1, 20] = 0.0
    al[2, :] = 4.0
    al[3, 14:18] = 2.0 ** -20
    S, n, G, K = q.shape
    d = [torch.from_numpy(x).cuda() for x in (q, k, v, al, be)]
    st = torch.from_numpy(S0).cuda()
    y = torch.full((S, n, G, 128), float("nan"), dtype=torch.float32, device="cuda")
    snap = [40, 4, 17, 16]
    _say(f"gdn gate range: S={S} n={n} G={G} decay_first={decay_first} snap={snap}")
    sa.gdn_verify(*d, y, st, None, None, torch.tensor(snap, dtype=torch.int32, device="cuda"), decay_first)
    torch.cuda.synchronize()
    want_y, want_st = oracle.gdn_verify(q, k, v, al, be, S0, None, snap, decay_first)
    # the gates of 4 grow the state by up to 4^40: the bar is relative to each stream's scale
    for s in range(S):
        for got, want, what in ((y.cpu().numpy()[s], want_y[s], "y"), (st.cpu().numpy()[s], want_st[s], "state")):
            assert np.all(np.isfinite(got)), (s, what)
            m = oracle.diff_metrics(want, got)
            scale = float(np.abs(want).max())
            _say(f"stream {s} {what}: max_abs/scale={m['max_abs'] / scale:.3e} rel_l2={m['rel_l2']:.3e}")
            assert m["max_abs"] <= 1e-5 * scale and m["rel_l2"] < 1e-5 and m["cosine"] > 0.99999, (s, what, m)
