"""A multi-stream verify step end to end on the GPU: the batch former (include/sixi_plan.h)
plans the pass(es), sixi_kv_write stores each block's K/V, sixi_attn_forward attends; the
real rows of every stream must match the oracle, with the reference's padded parts and with
one ragged pass (pad rows never computed), and the two plans must agree with each other."""
import sys

import numpy as np
import pytest
import torch

import oracle
import sixi_attn as sa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
REL_L2 = 1e-3
H, HKV, D = 24, 4, 128
N_CTX = 4096


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def _stream_data(seed, cached, rows):
    """One stream's Q rows, cached K/V (f16 bits) and block K/V rows (f32, pads included)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((rows, H, D)).astype(np.float32)
    kc = rng.standard_normal((cached, HKV, D)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((cached, HKV, D)).astype(np.float16).view(np.uint16)
    kb = rng.standard_normal((rows, HKV, D)).astype(np.float32)
    vb = rng.standard_normal((rows, HKV, D)).astype(np.float32)
    return q, kc, vc, kb, vb


def _run_part(fa, data, ids, kv_len, q_len, R, n_cells):
    """One pass: store the blocks with sixi_kv_write, then attend; returns out[S, R, H, D]."""
    S = len(ids)
    q = np.zeros((S, R, H, D), np.float32)
    kcache = np.zeros((S, n_cells, HKV, D), np.uint16)
    vcache = np.zeros_like(kcache)
    kb = np.zeros((S, R, HKV, D), np.float32)
    vb = np.zeros_like(kb)
    for i, sid in enumerate(ids):
        dq, kc, vc, dkb, dvb = data[sid]
        q[i] = dq[:R]
        kcache[i, :kv_len[i]] = kc
        vcache[i, :kv_len[i]] = vc
        kb[i, :q_len[i]] = dkb[:q_len[i]]
        vb[i, :q_len[i]] = dvb[:q_len[i]]
    dk = torch.from_numpy(kcache.view(np.float16)).cuda()
    dv = torch.from_numpy(vcache.view(np.float16)).cuda()
    kl = torch.tensor(kv_len, dtype=torch.int32, device="cuda")
    ql = torch.tensor(q_len, dtype=torch.int32, device="cuda")
    sa.kv_write(torch.from_numpy(kb).cuda(), dk, kl, ql)
    sa.kv_write(torch.from_numpy(vb).cuda(), dv, kl, ql)
    out = torch.full((S, R, H, D), float("nan"), dtype=torch.float32, device="cuda")
    fa(torch.from_numpy(q).cuda(), dk, dv, out, kv_len=kl, q_len=ql, mask_mode=sa.MASK_BLOCK_CAUSAL)
    torch.cuda.synchronize()
    host = {"q": q, "k": dk.cpu().numpy().view(np.uint16), "v": dv.cpu().numpy().view(np.uint16),
            "kv_len": np.array(kv_len, np.int32), "q_len": np.array(q_len, np.int32)}
    return out.cpu().numpy(), host


def test_reference_parts_and_one_ragged_pass_agree_with_the_oracle():
    streams = [(0, 100, 16), (1, 4090, 4), (2, 50, 3), (3, 4085, 8), (4, 900, 16)]
    data = {sid: _stream_data(0x51A7_7000 + sid, cached, 16) for sid, cached, _ in streams}
    fa = sa.FlashAttnExt()
    real = {sid: r for sid, _, r in streams}
    results = {}
    for mode in (sa.PAD_REFERENCE, sa.PAD_NONE):
        n_parts, slots = sa.plan_verify(streams, N_CTX, mode)
        _say(f"plan mode={mode}: {n_parts} part(s) {slots}")
        for p in range(n_parts):
            ids, kv_len, q_len = sa.part_lengths(streams, slots, p, mode)
            R = max(q_len)
            got, host = _run_part(fa, data, ids, kv_len, q_len, R, n_cells=N_CTX + 16)
            want = oracle.attention_for_workload(host, oracle.F16)
            for i, sid in enumerate(ids):
                g = got[i, :real[sid]]
                m = oracle.diff_metrics(want[i, :real[sid]].ravel(), g.ravel())
                _say(f"mode {mode} part {p} stream {sid}: max_abs={m['max_abs']:.2e} rel_l2={m['rel_l2']:.2e}")
                assert np.all(np.isfinite(g))
                assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (mode, sid, m)
                results[(mode, sid)] = g
    for sid in real:
        a, b = results[(sa.PAD_REFERENCE, sid)], results[(sa.PAD_NONE, sid)]
        assert np.abs(a - b).max() <= MAX_ABS, sid
