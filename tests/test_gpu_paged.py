"""Paged KV caches on the GPU: attention through a page table (include/sixi_attn.h
page_table) equals the attention over the same cells laid out contiguously, bit for bit, on
every kernel path (split-K 16- and 32-cell kernels, f16 and q8_0, 128- and 256-dim heads, the
explicit-mask path, the prefill kernel over f16 tiles, over q8_0 caches staged as f16 and,
with FLAG_BOUNDED_WORKSPACE, over q8_0 tiles converted in LDS); and the page pool's seq_cp
shares pages without moving cells while a write into a shared page copies it first
(include/sixi_kv.h sixi_kv_pool_*), checked bitwise against the data-copy path (sixi_kv_copy)
and against the oracle.

Pages are shuffled over a pool larger than the streams need; unused pages hold NaN, so a
wrong page or a cell read past a page shows up in the output."""
import sys

import numpy as np
import pytest
import torch

import oracle
import sixi_attn as sa
from sixi_attn import workloads as wl

pytestmark = pytest.mark.gpu

P = sa.PAGE_CELLS
MAX_ABS = 2e-3
REL_L2 = 1e-3


def _say(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def fa():
    assert torch.cuda.is_available(), "the gpu tests need a GPU"
    sa.load_library()
    return sa.FlashAttnExt()


def _nan_fill(t):
    if t.dtype == torch.uint8:  # q8_0 blocks: NaN scales
        t.view(-1, 34)[:, 0:2].copy_(torch.tensor([0x00, 0x7E], dtype=torch.uint8, device=t.device))
    else:
        t.fill_(float("nan"))


def _paginate(cache, perm, n_pages, head_major=False):
    """cache [S, cap, Hkv, X] -> (pool [n_pages, P, Hkv, X], page table [S, cap/P] int32) with
    stream s's page i at pool page perm[s * cap/P + i].  head_major: each page stores its kv-heads
    one after the other ([n_pages, Hkv, P, X] in memory, viewed as [n_pages, P, Hkv, X])."""
    S, cap = cache.shape[0], cache.shape[1]
    per = cap // P
    Hkv, X = cache.shape[2], cache.shape[3]
    base = torch.empty((n_pages, Hkv, P, X) if head_major else (n_pages, P, Hkv, X), dtype=cache.dtype,
                       device=cache.device)
    _nan_fill(base)
    pool = base.permute(0, 2, 1, 3) if head_major else base
    table = torch.tensor(np.asarray(perm[:S * per], dtype=np.int32).reshape(S, per), device=cache.device)
    idx = table.reshape(-1).long()
    pool[idx] = cache.reshape(S * per, P, *cache.shape[2:])
    return pool, table


CASES = [
    # label, kv_type, D, kv_len, q_len, H, Hkv, explicit mask
    ("verify 96 rows (32-cell kernel)", sa.TYPE_F16, 128, [700, 2000, 255, 513], [16, 16, 3, 9], 24, 4, False),
    ("decode (16-cell kernel)", sa.TYPE_F16, 128, [1000, 257, 4000], [1, 1, 1], 24, 4, False),
    ("48 rows", sa.TYPE_F16, 128, [767, 1300], [8, 5], 24, 4, False),
    ("explicit mask", sa.TYPE_F16, 128, [700, 2000, 255, 513], [16, 16, 3, 9], 24, 4, True),
    ("256-dim verify", sa.TYPE_F16, 256, [600, 1025], [16, 7], 24, 4, False),
    ("q8_0 decode", sa.TYPE_Q8_0, 128, [1500, 256, 3000], [1, 4, 8], 24, 4, False),
    ("q8_0 96 rows (32-cell q8_0 kernel)", sa.TYPE_Q8_0, 128, [900, 300], [16, 16], 24, 4, False),
    ("q8_0 256-dim", sa.TYPE_Q8_0, 256, [700, 120], [8, 3], 24, 4, False),
    ("q8_0 256-dim prefill rows", sa.TYPE_Q8_0, 256, [300, 0], [130, 200], 24, 4, False),
    ("prefill rows", sa.TYPE_F16, 128, [300, 0], [130, 200], 24, 4, False),
    ("q8_0 prefill rows", sa.TYPE_Q8_0, 128, [300, 0], [130, 200], 24, 4, False),
    ("q8_0 prefill rows, explicit mask", sa.TYPE_Q8_0, 128, [700, 40], [150, 260], 24, 4, True),
]


@pytest.mark.parametrize("head_major", [False, True], ids=["token-major pages", "head-major pages"])
@pytest.mark.parametrize("label,kv_type,D,kv_len,q_len,H,Hkv,explicit", CASES, ids=[c[0] for c in CASES])
def test_paged_equals_contiguous(fa, label, kv_type, D, kv_len, q_len, H, Hkv, explicit, head_major):
    """The pool's pages may hold a page token-major (cell rows of all kv-heads together, as
    llama.cpp's cache) or head-major (each kv-head's 256 cells together): the kernels take the
    strides as they are, so both give the contiguous cache's output bit for bit."""
    w = wl.Workload(label, 0x51A7_9300 + len(label), len(kv_len), kv_len, q_len, H=H, Hkv=Hkv, D=D, kv_type=kv_type)
    host = wl.make_host(w, poison=not explicit)
    dev = wl.to_device(host)
    S, cap = w.S, dev["k"].shape[1]
    per = cap // P
    n_pages = S * per + 5
    rng = np.random.default_rng(len(label))
    perm = rng.permutation(n_pages)
    kpool, table = _paginate(dev["k"], perm, n_pages, head_major)
    vpool, _ = _paginate(dev["v"], perm, n_pages, head_major)
    mask = None
    if explicit:
        mask = torch.from_numpy(wl.kq_mask(cap, w.n_q, w.kv_len, w.q_len)).view(torch.float16).cuda()
    mode = sa.MASK_EXPLICIT if explicit else sa.MASK_BLOCK_CAUSAL
    _say(f"{label}: S={S} kv_len={kv_len} q_len={q_len} D={D} type={kv_type} pages={n_pages} head_major={head_major}")
    out_c = torch.full((S, w.n_q, H, D), float("nan"), device="cuda")
    out_p = torch.full_like(out_c, float("nan"))
    fa(dev["q"], dev["k"], dev["v"], out_c, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=mode, mask=mask)
    fa(dev["q"], kpool, vpool, out_p, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=mode, mask=mask,
       page_table=table)
    torch.cuda.synchronize()
    for s in range(S):
        a, b = out_c[s, :q_len[s]], out_p[s, :q_len[s]]
        assert torch.isfinite(b).all(), (label, s)
        assert torch.equal(a, b), (label, s, (a - b).abs().max().item())
    if kv_type == sa.TYPE_Q8_0:
        # with FLAG_BOUNDED_WORKSPACE prefill-sized blocks read the q8_0 pages themselves
        # (converted in LDS) instead of a staged f16 copy: the same output
        out_b = torch.full_like(out_c, float("nan"))
        fa(dev["q"], kpool, vpool, out_b, kv_len=dev["kv_len"], q_len=dev["q_len"], mask_mode=mode, mask=mask,
           page_table=table, bounded_workspace=True)
        torch.cuda.synchronize()
        for s in range(S):
            assert torch.equal(out_c[s, :q_len[s]], out_b[s, :q_len[s]]), (label, "bounded", s)


def test_paged_matches_the_oracle_on_shared_pages(fa):
    """Streams that share pages (one page table row pointing at another's pages) read the
    same cells; the output equals the oracle on the gathered cells."""
    kv_len, q_len = [1000, 1000, 600], [16, 16, 16]
    w = wl.Workload("shared", 0x51A7_9310, 3, kv_len, q_len)
    host = wl.make_host(w)
    # stream 1's cells are stream 0's (its own Q)
    host["k"][1] = host["k"][0]
    host["v"][1] = host["v"][0]
    dev = wl.to_device(host)
    cap = dev["k"].shape[1]
    per = cap // P
    n_pages = 3 * per + 2
    perm = np.random.default_rng(7).permutation(n_pages)
    kpool, table = _paginate(dev["k"], perm, n_pages)
    vpool, _ = _paginate(dev["v"], perm, n_pages)
    table[1] = table[0]  # shared pages; stream 1's own pages are left unused
    out = torch.full((3, 16, w.H, w.D), float("nan"), device="cuda")
    fa(dev["q"], kpool, vpool, out, kv_len=dev["kv_len"], q_len=dev["q_len"], page_table=table)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = oracle.attention_for_workload(host, w.kv_type)
    m = oracle.diff_metrics(want.ravel(), got.ravel())
    _say(f"shared pages: max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m


@pytest.mark.parametrize("head_major", [False, True], ids=["token-major pages", "head-major pages"])
@pytest.mark.parametrize("kv_type", [sa.TYPE_F16, sa.TYPE_Q8_0])
def test_pool_seq_cp_shares_and_writes_copy_on_write(fa, kv_type, head_major):
    """Through the page pool: stream 0 is written (kv_write through the page table), copied to
    stream 1 with seq_cp (no cell moves: stream 1's row of the page table is stream 0's),
    then both append 16 different rows -- the shared last page is copied for the first
    writer.  The attention over both streams equals the contiguous cache built with
    sixi_kv_copy, bit for bit, and the oracle."""
    D, Hkv, H, L, n = 128, 4, 24, 700, 16
    torch.manual_seed(3)
    row = D // 32 * 34 if kv_type == sa.TYPE_Q8_0 else D
    dt = torch.uint8 if kv_type == sa.TYPE_Q8_0 else torch.float16
    max_pages, n_pages = 4, 9
    pool = sa.KvPool(n_pages, 2, max_pages)
    shape = (n_pages, Hkv, P, row) if head_major else (n_pages, P, Hkv, row)
    kb, vb = torch.zeros(shape, dtype=dt, device="cuda"), torch.zeros(shape, dtype=dt, device="cuda")
    _nan_fill(kb)
    _nan_fill(vb)
    kp = kb.permute(0, 2, 1, 3) if head_major else kb  # [n_pages, P, Hkv, row] either way
    vp = vb.permute(0, 2, 1, 3) if head_major else vb
    pool.attach(kp, D)
    pool.attach(vp, D)
    cap = max_pages * P
    kc = torch.zeros((2, cap, Hkv, row), dtype=dt, device="cuda")
    vc = torch.zeros_like(kc)

    def write(cache_k, cache_v, src_k, src_v, s, first, table=None):
        rows = src_k.shape[0]
        kl = torch.tensor([first], dtype=torch.int32, device="cuda")
        ql = torch.tensor([rows], dtype=torch.int32, device="cuda")
        if table is None:
            sa.kv_write(src_k[None], cache_k[s:s + 1], kl, ql)
            sa.kv_write(src_v[None], cache_v[s:s + 1], kl, ql)
        else:
            sa.kv_write(src_k[None], cache_k, kl, ql, page_table=table[s:s + 1])
            sa.kv_write(src_v[None], cache_v, kl, ql, page_table=table[s:s + 1])

    k0, v0 = torch.randn((L, Hkv, D), device="cuda"), torch.randn((L, Hkv, D), device="cuda")
    pool.prepare_write(0, 0, L)
    write(kp, vp, k0, v0, 0, 0, pool.upload())
    write(kc, vc, k0, v0, 0, 0)
    # the copy: pages shared, no cells move; the contiguous cache copies cells
    free_before = pool.free_pages()
    pool.seq_cp(0, 1, L)
    t = pool.page_table()
    assert (t[1, :3] == t[0, :3]).all() and pool.free_pages() == free_before
    sa.kv_copy(kc, 0, 1, L, head_dim=D)
    sa.kv_copy(vc, 0, 1, L, head_dim=D)
    # both streams append their own rows at cell L (page 2, shared): stream 1 writes first
    extra = [(torch.randn((n, Hkv, D), device="cuda"), torch.randn((n, Hkv, D), device="cuda")) for _ in range(2)]
    for s in (1, 0):
        pool.prepare_write(s, L, n)
        write(kp, vp, extra[s][0], extra[s][1], s, L, pool.upload())
        write(kc, vc, extra[s][0], extra[s][1], s, L)
    t = pool.page_table()
    assert (t[1, :2] == t[0, :2]).all() and t[1, 2] != t[0, 2], t
    assert pool.free_pages() == free_before - 1  # one copied page
    table = pool.upload()

    q = torch.randn((2, n, H, D), device="cuda")
    kl = torch.tensor([L, L], dtype=torch.int32, device="cuda")
    ql = torch.tensor([n, n], dtype=torch.int32, device="cuda")
    out_c = torch.full((2, n, H, D), float("nan"), device="cuda")
    out_p = torch.full_like(out_c, float("nan"))
    fa(q, kc, vc, out_c, kv_len=kl, q_len=ql)
    fa(q, kp, vp, out_p, kv_len=kl, q_len=ql, page_table=table)
    torch.cuda.synchronize()
    assert torch.isfinite(out_p).all()
    assert torch.equal(out_c, out_p), (out_c - out_p).abs().max().item()
    host = {"q": q.cpu().numpy(), "k": kc.cpu().numpy(), "v": vc.cpu().numpy(),
            "kv_len": np.array([L, L], np.int32), "q_len": np.array([n, n], np.int32)}
    if kv_type == sa.TYPE_F16:
        host["k"] = host["k"].view(np.uint16)
        host["v"] = host["v"].view(np.uint16)
    want = oracle.attention_for_workload(host, kv_type)
    m = oracle.diff_metrics(want.ravel(), out_p.cpu().numpy().ravel())
    _say(f"pool seq_cp + copy-on-write ({'q8_0' if kv_type == sa.TYPE_Q8_0 else 'f16'}): "
         f"max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}")
    assert m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2, m
    # the pages of the shared prefix were never written again: stream 1's first two pages
    # hold exactly stream 0's cells
    gathered = kp[torch.tensor(t[1, :2], dtype=torch.long, device="cuda")].reshape(2 * P, Hkv, row)
    assert torch.equal(gathered, kc[0, :2 * P])
    pool.close()


@pytest.mark.parametrize("head_major", [False, True], ids=["token-major pages", "head-major pages"])
@pytest.mark.parametrize("q8", [False, True])
def test_prologue_store_through_the_page_table(q8, head_major):
    """The layer prologue's fused KV store (include/sixi_layer.h) into a paged cache writes the
    same bytes, cell for cell, as into the contiguous cache; the pages the block does not touch
    (and the cells of touched pages outside the block) keep their bytes."""
    S, R, H, Hkv, D = 3, 16, 24, 4, 256
    kv_len, q_len = [250, 1000, 0], [16, 9, 16]  # stream 0's block crosses a page boundary
    per = 5
    n_pages = S * per + 3
    torch.manual_seed(11)
    qg = torch.randn((S, R, H, 2 * D), device="cuda")
    k = torch.randn((S, R, Hkv, D), device="cuda")
    v = torch.randn((S, R, Hkv, D), device="cuda")
    wq = torch.rand(D, device="cuda") + 0.5
    wk = torch.rand(D, device="cuda") + 0.5
    row = D // 32 * 34 if q8 else D
    dt = torch.uint8 if q8 else torch.float16
    gen = torch.Generator(device="cuda").manual_seed(5)
    kc = torch.randint(0, 255, (S, per * P, Hkv, row), dtype=torch.uint8, device="cuda", generator=gen)
    if not q8:  # finite f16 values
        kc = (kc.to(torch.float16) - 127.0) / 64.0
    vc = kc.clone()
    perm = np.random.default_rng(3).permutation(n_pages)
    kp, table = _paginate(kc, perm, n_pages, head_major)
    vp, _ = _paginate(vc, perm, n_pages, head_major)
    kp0, vp0 = kp.clone(), vp.clone()
    kl = torch.tensor(kv_len, dtype=torch.int32, device="cuda")
    ql = torch.tensor(q_len, dtype=torch.int32, device="cuda")
    qo_c = torch.full((S, R, H, D), float("nan"), device="cuda")
    qo_p = torch.full_like(qo_c, float("nan"))
    sa.qk_prologue(qg, k, v, wq, wk, qo_c, kc, vc, kl, ql)
    sa.qk_prologue(qg, k, v, wq, wk, qo_p, kp, vp, kl, ql, page_table=table)
    torch.cuda.synchronize()
    assert torch.equal(torch.nan_to_num(qo_c, 7.0), torch.nan_to_num(qo_p, 7.0))
    idx = table.reshape(-1).long()
    for name, pool, cont, before in (("K", kp, kc, kp0), ("V", vp, vc, vp0)):
        gathered = pool[idx].reshape(S, per * P, Hkv, row)
        assert torch.equal(gathered.view(torch.uint8), cont.view(torch.uint8)), name
        unused = torch.ones(n_pages, dtype=torch.bool, device="cuda")
        unused[idx] = False
        assert torch.equal(pool[unused].view(torch.uint8), before[unused].view(torch.uint8)), name


def test_pool_upload_snapshots_without_waiting():
    """sixi_kv_pool_upload copies from pinned snapshots that alternate between calls, with no
    stream synchronisation: several uploads queued behind busy work each land the table as it
    was at their call, including the third, which reuses the first snapshot buffer."""
    _say("pool upload: queued snapshots")
    pool = sa.KvPool(n_pages=64, n_streams=3, max_pages=8)
    busy = torch.randn(4096, 4096, device="cuda")
    want, dsts = [], []
    for step in range(5):
        pool.prepare_write(step % 3, 256 * step, 256)   # the table changes between uploads
        if step % 2:
            pool.seq_cp(step % 3, (step + 1) % 3)
        for _ in range(3):
            busy = busy @ busy.T * 1e-3                     # keep the stream busy meanwhile
        dsts.append(pool.upload())
        want.append(pool.page_table())
    torch.cuda.synchronize()
    for step, (d, w) in enumerate(zip(dsts, want)):
        assert np.array_equal(d.cpu().numpy(), w), step
    pool.close()


def test_pool_upload_under_graph_capture_keeps_the_captured_table():
    """Captured into a HIP graph, the upload stores the table as it was at capture on every
    replay (the values travel in kernel arguments), whatever the pool holds by then; eager
    uploads between the replays still see the current table."""
    _say("pool upload: graph capture")
    pool = sa.KvPool(n_pages=64, n_streams=4, max_pages=300)  # 1200 entries: two launches
    for s in range(4):
        pool.prepare_write(s, 0, 256 * (s + 1))
    captured = pool.page_table()
    dst = torch.full((4, 300), 7, dtype=torch.int32, device="cuda")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        pool.upload(dst)  # warm the eager path on this stream before capturing
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        pool.upload(dst, stream=side.cuda_stream)
    pool.seq_rm(0, 0)
    pool.seq_cp(3, 1)
    now = pool.page_table()
    assert not np.array_equal(now, captured)
    for rep in range(3):
        dst.fill_(-5)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dst.cpu().numpy(), captured), rep
        eager = pool.upload()
        torch.cuda.synchronize()
        assert np.array_equal(eager.cpu().numpy(), now), rep
    pool.close()
