"""The oracle's KV-cache store (oracle.kv_write), pinned on the CPU.

Placement is pinned by a hand-built case whose written cells are listed explicitly; the
conversions by numpy's own float16 rounding (an independent round-to-nearest-even) and by
the q8_0 codec, itself pinned against the reference's numeric.cpp in test_oracle_codec.py.
"""
import numpy as np

import oracle


def _cache_f16(S, n_cells, Hkv, D, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, 1 << 16, size=(S, n_cells, Hkv, D), dtype=np.uint16)


def test_f16_store_places_rows_at_kv_len_plus_j_and_nowhere_else():
    S, n_rows, Hkv, D, n_cells = 3, 4, 2, 64, 7
    rng = np.random.default_rng(1)
    src = rng.standard_normal((S, n_rows, Hkv, D)).astype(np.float32)
    cache = _cache_f16(S, n_cells, Hkv, D, 2)
    kv_len, q_len = [3, 0, 6], [2, 4, 3]
    out = oracle.kv_write(src, cache, kv_len, q_len)
    written = {(0, 3): 0, (0, 4): 1, (1, 0): 0, (1, 1): 1, (1, 2): 2, (1, 3): 3, (2, 6): 0}
    for s in range(S):
        for c in range(n_cells):
            if (s, c) in written:
                want = src[s, written[(s, c)]].astype(np.float16).view(np.uint16)
                assert np.array_equal(out[s, c], want), (s, c)
            else:
                assert np.array_equal(out[s, c], cache[s, c]), (s, c)


def test_f16_store_rounds_like_numpy_on_ties_subnormals_and_overflow():
    D = 32
    x = np.array([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -(1 + 2.0 ** -11), 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                  65504.0, 65520.0, 70000.0, -70000.0, 0.0, -0.0, 1e-30, np.inf, -np.inf, 0.1] * 2,
                 dtype=np.float32)
    src = x.reshape(1, 1, 1, D)
    out = oracle.kv_write(src, np.zeros((1, 1, 1, D), np.uint16), [0], [1])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(out[0, 0, 0], want)


def test_q8_store_places_quantized_blocks():
    S, n_rows, Hkv, D, n_cells = 2, 3, 2, 64, 4
    rng = np.random.default_rng(3)
    src = rng.standard_normal((S, n_rows, Hkv, D)).astype(np.float32)
    cache = rng.integers(0, 256, size=(S, n_cells, Hkv, D // 32 * 34), dtype=np.uint8)
    out = oracle.kv_write(src, cache, [2, -1], [3, 2])
    # stream 0: rows 0, 1 -> cells 2, 3 (row 2 would be cell 4: outside); stream 1: row 1 -> cell 0
    written = {(0, 2): (0, 0), (0, 3): (0, 1), (1, 0): (1, 1)}
    for s in range(S):
        for c in range(n_cells):
            for h in range(Hkv):
                if (s, c) in written:
                    ss, j = written[(s, c)]
                    assert np.array_equal(out[s, c, h], oracle.quantize_q8_0(src[ss, j, h])), (s, c, h)
                else:
                    assert np.array_equal(out[s, c, h], cache[s, c, h]), (s, c, h)


def test_q8_store_of_zero_block_is_zero_scale_and_quants():
    src = np.zeros((1, 1, 1, 32), np.float32)
    out = oracle.kv_write(src, np.full((1, 1, 1, 34), 0xAB, np.uint8))
    assert not out.any()
