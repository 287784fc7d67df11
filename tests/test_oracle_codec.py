"""Pins of the oracle's codecs and generator.

- fp16: exhaustive over all 65536 halves against the reference's own numeric.cpp
  (compiled into oracle/_ref) and numpy; f32->f16 on midpoints, boundaries and random bits.
- q8_0: bit-exact against the reference's quantize_row_q8_0 (src/core/numeric.cpp:349-384)
  and a numpy closed form, including exact-tie blocks.
- PCG32: the published pcg32 demo vector (seed 42, sequence 54).
- the package's synthetic generator equals the oracle's, bit for bit.
"""
import numpy as np
import pytest

import oracle
from sixi_attn import workloads


def _ref():
    lib = oracle.ref_numeric()
    if lib is None:
        pytest.skip("oracle/_ref not built (needs the reference tree; `make -C oracle ref`)")
    return lib


ALL_HALVES = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_fp16_to_fp32_exhaustive_matches_numpy():
    got = oracle.fp16_bits_to_fp32(ALL_HALVES)
    want = ALL_HALVES.view(np.float16).astype(np.float32)
    finite = np.isfinite(want) | np.isinf(want)
    assert np.array_equal(got.view(np.uint32)[finite], want.view(np.uint32)[finite])
    assert np.all(np.isnan(got[~finite]))


def test_fp16_to_fp32_exhaustive_matches_reference():
    ref = _ref()
    got = oracle.fp16_bits_to_fp32(ALL_HALVES).view(np.uint32)
    want = np.array([np.float32(ref.ref_fp16_to_fp32(int(h))).view(np.uint32) for h in ALL_HALVES])
    assert np.array_equal(got, want)


def _f32_probe_values():
    rng = np.random.default_rng(7)
    halves = ALL_HALVES.view(np.float16).astype(np.float32)
    fin = halves[np.isfinite(halves)]
    # exact values, neighbours, and exact midpoints between consecutive halves (ties)
    with np.errstate(over="ignore"):
        nxt = np.nextafter(fin.astype(np.float16), np.float16(np.inf)).astype(np.float32)
    ok = np.isfinite(nxt)
    mids = ((fin[ok].astype(np.float64) + nxt[ok].astype(np.float64)) / 2).astype(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e30, -1e30, 2.0**-24, 2.0**-25,
                        2.0**-25 * 1.0000001, 2.0**-26, 1e-40, -1e-40, np.inf, -np.inf], dtype=np.float32)
    rand_bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    vals = np.concatenate([fin, np.nextafter(fin, np.float32(np.inf)), np.nextafter(fin, np.float32(-np.inf)),
                           mids, -mids, special, rand_bits])
    return vals.astype(np.float32)


def test_fp32_to_fp16_matches_numpy_rne():
    vals = _f32_probe_values()
    vals = vals[~np.isnan(vals)]
    got = oracle.fp32_to_fp16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_fp32_to_fp16_matches_reference_bitwise():
    ref = _ref()
    vals = _f32_probe_values()
    got = oracle.fp32_to_fp16_bits(vals)
    want = np.empty(vals.shape, dtype=np.uint16)
    ref.ref_fp32_to_fp16_row(vals.ctypes.data, want.ctypes.data, vals.size)
    assert np.array_equal(got, want)  # NaN payloads included


def _q8_blocks():
    rng = np.random.default_rng(11)
    blocks = [rng.standard_normal(32 * 4096).astype(np.float32) * s for s in (1.0, 1e-3, 300.0)]
    zero = np.zeros(32, np.float32)
    onehot = np.zeros(32, np.float32); onehot[5] = -3.0
    # ties: amax = 127 makes id = 1 exactly, so x = k + 0.5 rounds half away from zero
    ties = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5] + [0.25] * 23, np.float32)
    neg_amax = -ties
    return np.concatenate(blocks + [zero, onehot, ties, neg_amax])


def _q8_closed_form(x):
    x = x.reshape(-1, 32).astype(np.float32)
    amax = np.max(np.abs(x), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    v = (x * idv[:, None]).astype(np.float32)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)), -127, 127).astype(np.int8)
    dh = d.astype(np.float16).view(np.uint16)
    out = np.empty((x.shape[0], 34), np.uint8)
    out[:, 0:2] = dh.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def test_q8_0_matches_closed_form():
    x = _q8_blocks()
    assert np.array_equal(oracle.quantize_q8_0(x), _q8_closed_form(x))


def test_q8_0_matches_reference_bitwise():
    ref = _ref()
    assert ref.ref_q8_0_block_bytes() == 34
    x = _q8_blocks()
    want = np.empty(x.size // 32 * 34, np.uint8)
    assert ref.ref_quantize_row_q8_0(x.ctypes.data, want.ctypes.data, x.size) == 0
    assert np.array_equal(oracle.quantize_q8_0(x), want)


def test_q8_0_roundtrip_and_dequant():
    x = np.random.default_rng(3).standard_normal(32 * 512).astype(np.float32)
    b = oracle.quantize_q8_0(x)
    y = oracle.dequantize_q8_0(b, x.size)
    cos = float(np.dot(x, y) / np.linalg.norm(x) / np.linalg.norm(y))
    assert cos > 0.9999  # as tests/test_routing_and_numerics.cpp:39-119 requires
    blk = b.reshape(-1, 34)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    q = blk[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(y.reshape(-1, 32), (d[:, None] * q).astype(np.float32))


def test_pcg32_published_vector():
    # pcg32-demo (pcg-c-basic): pcg32_srandom_r(&rng, 42u, 54u), first six outputs
    assert oracle.pcg32_u32(42, 54, 6) == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_normals_are_standard():
    x = oracle.fill_normal(0x51A70000, 1, 200_000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01


def test_package_generator_matches_oracle():
    for seed, seq, n, mul in ((0x51A70003, (2 << 32) | 5, 10_001, 1.0), (0x51A70004, 1 << 32, 4096, 0.5)):
        assert np.array_equal(workloads.normal_f32(seed, seq, n, mul).view(np.uint32),
                              oracle.fill_normal(seed, seq, n, mul).view(np.uint32))
    x = _q8_blocks()
    assert np.array_equal(workloads.quantize_q8_0(x), oracle.quantize_q8_0(x))


def test_vec_dot_f16_and_q8_0_against_exact_sums():
    rng = np.random.default_rng(5)
    lib = oracle.load()
    for n in (128, 256, 100):
        a = rng.standard_normal(n).astype(np.float16)
        b = rng.standard_normal(n).astype(np.float16)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        got = lib.oracle_vec_dot_f16(n, a.ctypes.data, b.ctypes.data)
        assert abs(got - exact) <= 1e-5 * (1 + abs(exact))
    x = rng.standard_normal(128).astype(np.float32)
    y = rng.standard_normal(128).astype(np.float32)
    bx, by = oracle.quantize_q8_0(x), oracle.quantize_q8_0(y)
    bxr, byr = bx.reshape(-1, 34), by.reshape(-1, 34)
    exact = 0.0
    for i in range(4):
        dx = float(bxr[i, :2].copy().view(np.float16)[0]); dy = float(byr[i, :2].copy().view(np.float16)[0])
        exact += dx * dy * int(np.dot(bxr[i, 2:].view(np.int8).astype(np.int64), byr[i, 2:].view(np.int8).astype(np.int64)))
    got = lib.oracle_vec_dot_q8_0(128, bx.ctypes.data, by.ctypes.data)
    assert abs(got - exact) <= 1e-5 * (1 + abs(exact))
