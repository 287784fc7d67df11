"""The verify batch former (include/sixi_plan.h) on the CPU.

Expected plans are worked out by hand from the reference's rule
(src/core/core_execution.cpp:2016-2049): R = longest block; rows = max(real, min(R, room))
with room = n_ctx_seq - N; streams grouped into parts by equal rows, first fit, stream-major
offsets inside a part.
"""
import ctypes

import pytest

import sixi_attn as sa


def test_all_streams_with_room_share_one_padded_part():
    n, slots = sa.plan_verify([(3, 100, 16), (7, 2000, 5), (9, 0, 1)], n_ctx_seq=8192)
    assert n == 1
    assert slots == [(0, 0, 0, 16), (0, 1, 16, 16), (0, 2, 32, 16)]


def test_streams_near_the_end_of_context_get_their_own_parts():
    streams = [(0, 100, 16), (1, 4090, 4), (2, 50, 3), (3, 4085, 8), (4, 4090, 2)]
    n, slots = sa.plan_verify(streams, n_ctx_seq=4096)
    # room: 3996, 6, 4046, 11, 6 -> rows 16, 6, 16, 11, 6
    assert n == 3
    assert slots == [(0, 0, 0, 16), (1, 0, 0, 6), (0, 1, 16, 16), (2, 0, 0, 11), (1, 1, 6, 6)]


def test_full_stream_keeps_its_real_rows_and_default_context_is_4096():
    n, slots = sa.plan_verify([(0, 4096, 3), (1, 5000, 2), (2, 10, 4)], n_ctx_seq=0)
    # room 0 -> rows = real (3, 2); stream 2: min(4, 4086) = 4
    assert n == 3
    assert slots == [(0, 0, 0, 3), (1, 0, 0, 2), (2, 0, 0, 4)]


def test_pad_none_is_one_ragged_part():
    streams = [(0, 100, 16), (1, 4090, 4), (2, 50, 3)]
    n, slots = sa.plan_verify(streams, n_ctx_seq=4096, pad_mode=sa.PAD_NONE)
    assert n == 1
    assert slots == [(0, 0, 0, 16), (0, 1, 16, 4), (0, 2, 20, 3)]
    ids, kv_len, q_len = sa.part_lengths(streams, slots, 0, sa.PAD_NONE)
    assert (ids, kv_len, q_len) == ([0, 1, 2], [100, 4090, 50], [16, 4, 3])


def test_part_lengths_reference_mode_counts_pad_rows():
    streams = [(0, 100, 16), (1, 4090, 4), (2, 50, 3)]
    _, slots = sa.plan_verify(streams, n_ctx_seq=4096)
    assert sa.part_lengths(streams, slots, 0) == ([0, 2], [100, 50], [16, 16])
    assert sa.part_lengths(streams, slots, 1) == ([1], [4090], [6])


def test_empty_and_invalid_inputs():
    assert sa.plan_verify([], 4096) == (0, [])
    lib = sa.load_library()
    one = (sa.SixiVerifyStream * 1)()
    one[0].stream, one[0].cached, one[0].real = 0, 10, 1
    out = (sa.SixiVerifySlot * 1)()
    n = ctypes.c_int32(0)
    assert lib.sixi_verify_plan(one, 1, 4096, 2, out, ctypes.byref(n)) == sa.E_INVALID_ARGUMENT
    assert lib.sixi_verify_plan(one, -1, 4096, 0, out, ctypes.byref(n)) == sa.E_INVALID_ARGUMENT
    assert lib.sixi_verify_plan(one, 1, 4096, 0, out, None) == sa.E_INVALID_ARGUMENT
    for cached, real in ((-1, 1), (5, 0)):
        one[0].cached, one[0].real = cached, real
        assert lib.sixi_verify_plan(one, 1, 4096, 0, out, ctypes.byref(n)) == sa.E_INVALID_ARGUMENT
    with pytest.raises(sa.SixiAttnError):
        sa.plan_verify([(0, 10, 0)], 4096)
