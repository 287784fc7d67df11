"""The page pool's bookkeeping on the host (include/sixi_kv.h sixi_kv_pool_*): page sharing
by seq_cp, release by seq_rm, copy-on-write page replacement before a write, exhaustion
errors, and -- over random operation sequences -- agreement with a plain model of which
stream holds which content.  No device is touched: no pool view is attached, so a
copy-on-write only swaps the page (the page data copy is covered by the GPU tests)."""
import random

import numpy as np
import pytest

import sixi_attn as sa

P = sa.PAGE_CELLS


def test_fresh_pages_and_sharing():
    pool = sa.KvPool(8, 3, 4)
    assert pool.free_pages() == 8
    pool.prepare_write(0, 0, 2 * P + 10)          # cells 0 .. 521: three pages
    t = pool.page_table()
    assert t[0].tolist() == [0, 1, 2, -1] and (t[1:] == -1).all()
    assert pool.stream_pages(0) == 3 and pool.free_pages() == 5
    pool.seq_cp(0, 1)                              # share, no new page
    t = pool.page_table()
    assert t[1].tolist() == t[0].tolist() and pool.free_pages() == 5
    assert [pool.page_refs(i) for i in range(3)] == [2, 2, 2]
    # stream 1 appends into its last page (shared): that page alone is replaced
    pool.prepare_write(1, 2 * P + 10, 5)
    t = pool.page_table()
    assert t[1, :2].tolist() == t[0, :2].tolist() and t[1, 2] not in (t[0, 2], -1)
    assert pool.page_refs(int(t[0, 2])) == 1 and pool.page_refs(int(t[1, 2])) == 1
    assert pool.free_pages() == 4


def test_seq_cp_prefix_and_seq_rm():
    pool = sa.KvPool(10, 2, 8)
    pool.prepare_write(0, 0, 5 * P)
    pool.seq_cp(0, 1, 2 * P + 1)                   # cells [0, 513): three pages
    assert pool.stream_pages(1) == 3
    assert [pool.page_refs(i) for i in range(5)] == [2, 2, 2, 1, 1]
    pool.seq_rm(0, P + 1)                          # stream 0 keeps cells [0, 257): two pages
    assert pool.stream_pages(0) == 2
    assert [pool.page_refs(i) for i in range(5)] == [2, 2, 1, 0, 0]
    assert pool.free_pages() == 7
    pool.seq_rm(1, -1)                             # drop everything
    assert pool.stream_pages(1) == 0 and pool.free_pages() == 8
    pool.seq_rm(0, 0)
    assert pool.free_pages() == 10 and (pool.page_table() == -1).all()


def test_copy_onto_itself_and_writes_in_the_middle():
    pool = sa.KvPool(6, 2, 4)
    pool.prepare_write(0, 0, 3 * P)
    before = pool.page_table().copy()
    pool.seq_cp(0, 0)                              # no-op
    assert (pool.page_table() == before).all() and pool.page_refs(0) == 1
    # a write into cells a stream does not have yet allocates the gap too (pages stay a prefix)
    pool.prepare_write(1, 2 * P + 3, 1)
    assert pool.stream_pages(1) == 3 and pool.free_pages() == 0


def test_errors_change_nothing():
    pool = sa.KvPool(4, 2, 3)
    pool.prepare_write(0, 0, 3 * P)
    with pytest.raises(sa.SixiAttnError) as e:
        pool.prepare_write(0, 3 * P, 1)            # beyond max_pages
    assert e.value.code == sa.E_OUT_OF_BOUNDS
    pool.seq_cp(0, 1)
    before = pool.page_table().copy()
    with pytest.raises(sa.SixiAttnError) as e:
        pool.prepare_write(1, 0, 3 * P)            # three shared pages, one free
    assert e.value.code == sa.E_OUT_OF_BOUNDS
    assert (pool.page_table() == before).all() and pool.free_pages() == 1
    with pytest.raises(sa.SixiAttnError):
        pool.seq_cp(0, 1, 4 * P)                   # more cells than stream 0 holds
    with pytest.raises(sa.SixiAttnError):
        pool.seq_rm(2, 0)                          # no such stream
    with pytest.raises(sa.SixiAttnError):
        sa.KvPool(0, 1, 1)
    with pytest.raises(sa.SixiAttnError):
        pool.page_refs(4)


def test_random_operations_match_a_content_model():
    """Model: each stream is a list of page-content ids (what its cells hold).  seq_cp copies
    the list prefix, seq_rm cuts it, a write gives the written pages fresh content.  The pool
    must map two streams to the same page exactly when the model says they share content
    that neither has written since, keep reference counts equal to the number of holders,
    and free every page no stream holds."""
    rng = random.Random(1234)
    n_pages, n_streams, max_pages = 24, 5, 6
    pool = sa.KvPool(n_pages, n_streams, max_pages)
    model = [[] for _ in range(n_streams)]
    next_id = [0]

    def fresh():
        next_id[0] += 1
        return next_id[0]

    for _ in range(600):
        op = rng.random()
        s = rng.randrange(n_streams)
        try:
            if op < 0.45:
                first = rng.randrange(0, max_pages * P)
                n = rng.randrange(1, 2 * P)
                last = (first + n - 1) // P
                held = len(model[s])
                pool.prepare_write(s, first, n)
                model[s].extend(fresh() for _ in range(held, last + 1))
                for i in range(first // P, min(last + 1, held)):
                    if sum(ids.count(model[s][i]) for ids in model) > 1:
                        model[s][i] = fresh()
            elif op < 0.7:
                d = rng.randrange(n_streams)
                n = rng.choice([-1, rng.randrange(0, len(model[s]) * P + 1)])
                pool.seq_cp(s, d, n)
                if d != s:
                    k = len(model[s]) if n < 0 else (n + P - 1) // P
                    model[d] = list(model[s][:k])
            else:
                p0 = rng.randrange(-1, max_pages * P)
                pool.seq_rm(s, p0)
                keep = 0 if p0 <= 0 else (p0 + P - 1) // P
                model[s] = model[s][:keep]
        except sa.SixiAttnError as e:
            assert e.code == sa.E_OUT_OF_BOUNDS  # full pool or a too-long stream: model unchanged
            continue
        t = pool.page_table()
        owner = {}
        for st in range(n_streams):
            assert pool.stream_pages(st) == len(model[st])
            assert (t[st, len(model[st]):] == -1).all()
            for i, cid in enumerate(model[st]):
                page = int(t[st, i])
                assert 0 <= page < n_pages
                # one page per content, one content per page
                assert owner.setdefault(cid, page) == page
        assert len(set(owner.values())) == len(owner)
        holders = {}
        for st in range(n_streams):
            for cid in model[st]:
                holders[cid] = holders.get(cid, 0) + 1
        for cid, page in owner.items():
            assert pool.page_refs(page) == holders[cid]
        assert pool.free_pages() == n_pages - len(owner)
