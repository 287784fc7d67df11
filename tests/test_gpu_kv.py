"""GPU KV-cache store and stream copy (include/sixi_kv.h) against the oracle, through the C ABI.

Integer/byte work, so the bar is bit-exact: every byte of the cache after the call equals
the oracle's (rows written with the reference's f16 / q8_0 codecs, every other cell --
poisoned with random bits beforehand -- unchanged).
"""
import sys

import numpy as np
import pytest
import torch

import oracle
import sixi_attn as sa
from sixi_attn import workloads as wl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def lib():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    return sa.load_library()


def _poisoned_cache(S, n_cells, Hkv, D, q8, seed):
    rng = np.random.default_rng(seed)
    if q8:
        return rng.integers(0, 256, size=(S, n_cells, Hkv, D // 32 * 34), dtype=np.uint8)
    return rng.integers(0, 1 << 16, size=(S, n_cells, Hkv, D), dtype=np.uint16)


def _to_dev(cache):
    if cache.dtype == np.uint8:
        return torch.from_numpy(cache.copy()).cuda()
    return torch.from_numpy(cache.view(np.float16).copy()).cuda()


def _from_dev(t, like):
    a = t.cpu().numpy()
    return a if like.dtype == np.uint8 else a.view(np.uint16)


def _write_and_check(src, cache, kv_len, q_len, label):
    _say(f"kv_write {label}: src {src.dtype} {src.shape} cache {cache.dtype} {cache.shape}")
    dev_src = torch.from_numpy(src).cuda()
    dev_cache = _to_dev(cache)
    kl = torch.tensor(kv_len, dtype=torch.int32, device="cuda") if kv_len is not None else None
    ql = torch.tensor(q_len, dtype=torch.int32, device="cuda") if q_len is not None else None
    sa.kv_write(dev_src, dev_cache, kl, ql)
    torch.cuda.synchronize()
    got = _from_dev(dev_cache, cache)
    want = oracle.kv_write(src, cache, kv_len, q_len)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{label}: {len(bad)} bytes differ, first at {bad[:4].tolist()}"


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("src_f16", [False, True])
def test_ragged_block_store(q8, src_f16):
    S, n_rows, Hkv, D, n_cells = 5, 16, 4, 128, 300
    rng = np.random.default_rng(11)
    src = (rng.standard_normal((S, n_rows, Hkv, D)) * 3).astype(np.float16 if src_f16 else np.float32)
    cache = _poisoned_cache(S, n_cells, Hkv, D, q8, 12)
    kv_len = [0, 17, 284, 290, 299]   # the last two streams run past the cache: those rows are skipped
    q_len = [16, 1, 16, 16, 3]
    _write_and_check(src, cache, kv_len, q_len, f"ragged q8={q8} src_f16={src_f16}")


@pytest.mark.parametrize("q8", [False, True])
def test_edge_values(q8):
    D = 128
    rng = np.random.default_rng(21)
    special = np.array([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -(1 + 2.0 ** -11), 2.0 ** -25, 2.0 ** -24,
                        3 * 2.0 ** -26, 65504.0, 65520.0, 70000.0, -70000.0, 0.0, -0.0, 1e-30, 0.5, -0.5, 127.0],
                       dtype=np.float32)
    rows = [np.tile(special, D // 16),                      # f16 ties, subnormals, overflow
            np.zeros(D, np.float32),                        # zero blocks: d = 0, q = 0
            np.where(np.arange(D) % 32 == 0, 127.0, 0.5).astype(np.float32),   # q = x*id ties at .5
            (rng.standard_normal(D) * 1e-36).astype(np.float32),               # tiny blocks, 127/amax finite
            (rng.standard_normal(D) * 1e6).astype(np.float32),                 # f16 scale overflow
            np.full(D, -3.0, np.float32)]
    src = np.stack(rows).reshape(1, len(rows), 1, D)
    cache = _poisoned_cache(1, len(rows) + 2, 1, D, q8, 22)
    _write_and_check(src, cache, [1], None, f"edge values q8={q8}")


def test_defaults_and_empty_rows():
    S, n_rows, Hkv, D = 2, 4, 2, 64
    src = np.random.default_rng(31).standard_normal((S, n_rows, Hkv, D)).astype(np.float32)
    cache = _poisoned_cache(S, 8, Hkv, D, False, 32)
    _write_and_check(src, cache, None, None, "kv_len = q_len = NULL")
    _write_and_check(src, cache, [2, 5], [0, 0], "q_len 0")
    _write_and_check(src, cache, [-2, 7], [4, 4], "negative and last-cell starts")


def test_head_dim_256_and_strided_source():
    S, n_rows, Hkv, D = 3, 16, 4, 256
    rng = np.random.default_rng(41)
    big = rng.standard_normal((S, n_rows, Hkv + 2, D)).astype(np.float32)
    src_view = torch.from_numpy(big).cuda()[:, :, 1:Hkv + 1, :]   # heads strided in the source
    for q8 in (False, True):
        cache = _poisoned_cache(S, 64, Hkv, D, q8, 42 + q8)
        dev_cache = _to_dev(cache)
        kl = torch.tensor([0, 30, 48], dtype=torch.int32, device="cuda")
        _say(f"kv_write D=256 strided source q8={q8}")
        sa.kv_write(src_view, dev_cache, kl)
        torch.cuda.synchronize()
        want = oracle.kv_write(np.ascontiguousarray(big[:, :, 1:Hkv + 1, :]), cache, [0, 30, 48], None)
        assert np.array_equal(_from_dev(dev_cache, cache), want)


def test_store_then_attend_matches_a_host_built_cache():
    """The verify block stored by sixi_kv_write and then attended gives the bitwise output of
    the same cache written on the host."""
    w = wl.Workload("kv-store", 0x51A7_6100, 3, [700, 64, 2000], [16, 5, 12])
    host = wl.make_host(w, poison=True)
    dev = wl.to_device(host)
    fa = sa.FlashAttnExt()
    out_ref = torch.full((w.S, w.n_q, w.H, w.D), float("nan"), dtype=torch.float32, device="cuda")
    fa(dev["q"], dev["k"], dev["v"], out_ref, kv_len=dev["kv_len"], q_len=dev["q_len"])
    # the block's K/V as f32 rows, erased from a copy of the cache, then stored again
    kv_len, q_len = host["kv_len"], host["q_len"]
    k2, v2 = dev["k"].clone(), dev["v"].clone()
    kb = torch.zeros((w.S, w.n_q, w.Hkv, w.D), dtype=torch.float32, device="cuda")
    vb = torch.zeros_like(kb)
    for s in range(w.S):
        rows = slice(int(kv_len[s]), int(kv_len[s]) + int(q_len[s]))
        kb[s, :q_len[s]] = k2[s, rows].float()
        vb[s, :q_len[s]] = v2[s, rows].float()
        k2[s, rows] = float("nan")
        v2[s, rows] = float("nan")
    _say("store-then-attend: kv_write of the block, then attention")
    sa.kv_write(kb, k2, dev["kv_len"], dev["q_len"])
    sa.kv_write(vb, v2, dev["kv_len"], dev["q_len"])
    out = torch.full_like(out_ref, float("nan"))
    fa(dev["q"], k2, v2, out, kv_len=dev["kv_len"], q_len=dev["q_len"])
    torch.cuda.synchronize()
    assert torch.equal(k2.view(torch.int16), dev["k"].view(torch.int16))
    for s in range(w.S):
        assert torch.equal(out[s, :q_len[s]], out_ref[s, :q_len[s]]), s


@pytest.mark.parametrize("q8,offset", [(False, 0), (True, 0), (True, 2)])
def test_stream_copy(q8, offset):
    S, n_cells, Hkv, D = 4, 96, 4, 128
    cache = _poisoned_cache(S, n_cells, Hkv, D, q8, 51 + offset)
    if offset:
        # a q8_0 view 2 bytes into its buffer: rows are only 2-byte aligned (half-word copy)
        flat = np.frombuffer(np.random.default_rng(52).integers(0, 256, cache.nbytes + offset, dtype=np.uint8)
                             .tobytes(), dtype=np.uint8).copy()
        buf = torch.from_numpy(flat).cuda()
        dev = buf[offset:].view(S, n_cells, Hkv, D // 32 * 34)
        cache = flat[offset:].reshape(S, n_cells, Hkv, D // 32 * 34).copy()
    else:
        dev = _to_dev(cache)
    want = cache.copy()
    _say(f"kv_copy q8={q8} offset={offset}")
    sa.kv_copy(dev, 1, 3, 40, src_cell=5, dst_cell=50, head_dim=D)
    want[3, 50:90] = cache[1, 5:45]
    sa.kv_copy(dev, 2, 2, 10, src_cell=0, dst_cell=80, head_dim=D)   # same stream, disjoint ranges
    want[2, 80:90] = cache[2, 0:10]
    torch.cuda.synchronize()
    assert np.array_equal(_from_dev(dev, cache), want)
