"""The C ABI on any host: the library loads, exports what include/*.h declare, and rejects
bad descriptions with the documented status codes before touching a device."""
import ctypes
import pathlib
import re

import pytest

import sixi_attn as sa

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared():
    names = set()
    for h in HEADERS:
        names |= set(re.findall(r"^\s*(?:int|int32_t|void|const char\*|size_t)\s+(sixi_\w+)\(", h.read_text(), re.M))
    return sorted(names)


def test_library_loads_and_exports_every_declared_symbol():
    lib = sa.load_library()
    declared = _declared()
    assert declared == sorted(sa.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.sixi_attn_abi_version() == 3


def test_status_strings():
    for code in (sa.OK, sa.E_INVALID_ARGUMENT, sa.E_OUT_OF_BOUNDS, sa.E_ALIGNMENT, sa.E_UNSUPPORTED,
                 sa.E_BACKEND, sa.E_INTEGER_OVERFLOW):
        assert sa.strerror(code) and sa.strerror(code) != "unknown status"
    assert sa.strerror(12345) == "unknown status"


FAKE = 0x7F0000000000  # aligned host address; validation never dereferences it
# each view of an attention description in an address range of its own (the ABI rejects a
# written view that overlaps anything the call reads)
ADDR = {name: FAKE + (i << 36) for i, name in enumerate(("q", "k", "v", "out", "kv_len", "mask", "ws", "pt"))}


def _params(S=2, n_q=16, H=24, Hkv=4, D=128, n_kv=4096, q_type=sa.TYPE_F32, kv_type=sa.TYPE_F16,
            mode=sa.MASK_BLOCK_CAUSAL, kv_len=True):
    p = sa.SixiAttnParams()
    qes = 4 if q_type == sa.TYPE_F32 else 2
    kves = 2
    p.q = sa.make_view(ADDR["q"], q_type, [D, n_q, H, S], [qes, H * D * qes, D * qes, n_q * H * D * qes])
    row = D * kves if kv_type == sa.TYPE_F16 else D // 32 * 34
    nb0 = kves if kv_type == sa.TYPE_F16 else 34
    kv_nb = [nb0, Hkv * row, row, n_kv * Hkv * row]
    p.k = sa.make_view(ADDR["k"], kv_type, [D, n_kv, Hkv, S], kv_nb)
    p.v = sa.make_view(ADDR["v"], kv_type, [D, n_kv, Hkv, S], kv_nb)
    p.out = sa.make_view(ADDR["out"], sa.TYPE_F32, [D, H, n_q, S], [4, D * 4, H * D * 4, n_q * H * D * 4])
    p.kv_len = ADDR["kv_len"] if kv_len else None
    p.q_len = None
    p.mask_mode = mode
    p.scale = 1.0 / D ** 0.5
    return p


def _validate(p):
    return sa.load_library().sixi_attn_validate(ctypes.byref(p))


def test_valid_descriptions_pass_and_size_a_workspace():
    lib = sa.load_library()
    for n_q in (1, 8, 16):
        p = _params(n_q=n_q)
        assert _validate(p) == sa.OK
        n = ctypes.c_size_t(0)
        assert lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n)) == sa.OK
        assert n.value > 0 and n.value % 256 == 0


def _launched_rows(rows, D):
    """Rows of one partial slot of the split-K kernel launched for `rows` rows per kv-head
    group: 16-row tiles; 128-dim heads run 1-3 tiles on the 16-cell kernel, then 64 or 96 rows
    (two row groups); 256-dim heads run at most two tiles per wave, so 33-64 rows run as 64."""
    t = -(-rows // 16)
    if t <= 2 or (t == 3 and D == 128):
        return 16 * t
    return 64 if t <= 4 else 96


@pytest.mark.parametrize("D", [128, 256])
def test_workspace_holds_the_launched_slots(D):
    """The workspace has room for (S*Hkv + 2048) partial slots of the rows the launched kernel
    writes: normalised rows in f16 (D/2 floats each) plus m and l."""
    lib = sa.load_library()
    for G, n_q in ((6, 1), (6, 2), (6, 5), (6, 6), (6, 7), (6, 8), (6, 10), (6, 13), (6, 16), (3, 16), (1, 33)):
        S, Hkv = 3, 4
        p = _params(S=S, n_q=n_q, H=G * Hkv, Hkv=Hkv, D=D)
        n = ctypes.c_size_t(0)
        assert lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n)) == sa.OK
        rows = _launched_rows(G * n_q, D)
        need = (S * Hkv + 2048) * rows * (D // 2 + 2) * 4
        assert n.value >= need, (G, n_q, D, n.value, need)


def test_q8_prefill_workspace_is_independent_of_the_cache_length():
    """q8_0 prefill stages K, V and Q as f16 while that copy takes at most STAGE_CAP_BYTES and
    reads the q8_0 tiles itself beyond it (a token workspace, whatever the cache length), or
    always with FLAG_BOUNDED_WORKSPACE.  256-dim rows that are not 16-byte aligned are always
    staged, so that workspace grows with the cells."""
    lib = sa.load_library()

    def ws(flags=0, **kw):
        p = _params(**kw)
        p.flags = flags
        n = ctypes.c_size_t(0)
        assert lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n)) == sa.OK
        return n.value

    token = ws(n_q=512, n_kv=1024, kv_type=sa.TYPE_F16)
    assert token <= 4096
    d128 = [ws(n_q=512, n_kv=n_kv, kv_type=sa.TYPE_Q8_0) for n_kv in (1024, 8192, 65536, 1 << 20)]
    # staged (2 streams x 4 heads x n_kv x 256 B for K and for V, plus Q) up to the cap
    assert 2 * 2 * 4 * 8192 * 256 <= d128[1] <= sa.STAGE_CAP_BYTES and d128[1] > d128[0] > token, d128
    assert d128[2:] == [token, token], d128
    assert ws(n_q=512, n_kv=65536, kv_type=sa.TYPE_Q8_0, mode=sa.MASK_NONE, kv_len=False) == token
    assert [ws(sa.FLAG_BOUNDED_WORKSPACE, n_q=512, n_kv=n_kv, kv_type=sa.TYPE_Q8_0)
            for n_kv in (1024, 65536)] == [token, token]
    d256 = [ws(n_q=512, n_kv=n_kv, D=256, kv_type=sa.TYPE_Q8_0) for n_kv in (1024, 4096, 65536, 1 << 20)]
    # staged (2 streams x 4 heads x n_kv x 512 B for K and for V, plus Q) up to the cap
    assert 2 * 2 * 4 * 4096 * 512 <= d256[1] <= sa.STAGE_CAP_BYTES and d256[1] > d256[0] > token, d256
    assert d256[2:] == [token, token], d256
    bounded = [ws(sa.FLAG_BOUNDED_WORKSPACE, n_q=512, n_kv=n_kv, D=256, kv_type=sa.TYPE_Q8_0)
               for n_kv in (1024, 65536, 1 << 20)]
    assert bounded == [token] * 3, bounded

    def ws_unaligned(n_kv, flags=0):
        p = _params(n_q=512, n_kv=n_kv, D=256, kv_type=sa.TYPE_Q8_0)
        p.flags = flags
        for t in (p.k, p.v):  # 4 spare bytes per cell: no row starts 16-byte aligned
            t.nb[1] = 4 * 272 + 4
            t.nb[3] = n_kv * t.nb[1]
        n = ctypes.c_size_t(0)
        assert lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n)) == sa.OK
        return n.value

    staged = [ws_unaligned(n_kv) for n_kv in (1024, 65536)]
    assert staged[1] > staged[0] >= 2 * 2 * 1024 * 4 * 256 * 2
    # only the staging can read such rows: the flag does not change it
    assert [ws_unaligned(n_kv, sa.FLAG_BOUNDED_WORKSPACE) for n_kv in (1024, 65536)] == staged


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p, "flags", 2), sa.E_INVALID_ARGUMENT),            # unknown flag bit
    (lambda p: setattr(p.q, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: p.q.ne.__setitem__(0, 96), sa.E_INVALID_ARGUMENT),          # q/k head dims differ
    (lambda p: p.q.ne.__setitem__(2, 25), sa.E_INVALID_ARGUMENT),          # H % Hkv != 0
    (lambda p: p.out.ne.__setitem__(2, 15), sa.E_INVALID_ARGUMENT),        # out rows != n_q
    (lambda p: p.k.nb.__setitem__(1, 1032), sa.E_ALIGNMENT),              # cell stride not 16-B
    (lambda p: setattr(p.k, "data", ADDR["k"] + 8), sa.E_ALIGNMENT),
    (lambda p: p.k.nb.__setitem__(1, 128), sa.E_INVALID_ARGUMENT),         # rows would overlap
    (lambda p: setattr(p, "mask_mode", 7), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p, "kv_len", None), sa.E_INVALID_ARGUMENT),         # block-causal needs lengths
    (lambda p: setattr(p, "max_bias", 1.0), sa.E_INVALID_ARGUMENT),        # ALiBi needs an explicit mask
    (lambda p: setattr(p, "scale", float("nan")), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.k, "type", 2), sa.E_UNSUPPORTED),                 # q4_0 KV not built
    (lambda p: p.q.ne.__setitem__(3, 5000), sa.E_INVALID_ARGUMENT),        # S mismatch with k
])
def test_invalid_descriptions_are_rejected(mutate, code):
    p = _params()
    mutate(p)
    assert _validate(p) == code


def test_stream_count_and_head_dim_limits():
    assert _validate(_params(D=96)) == sa.E_UNSUPPORTED
    assert _validate(_params(S=4096)) == sa.E_UNSUPPORTED


def test_explicit_mask_view_is_checked():
    p = _params(mode=sa.MASK_EXPLICIT)
    assert _validate(p) == sa.E_INVALID_ARGUMENT  # no mask view given
    p.mask = sa.make_view(ADDR["mask"], sa.TYPE_F16, [4096, 16, 1, 2], [2, 8192, 8192 * 16, 8192 * 16])
    assert _validate(p) == sa.OK
    p.mask.ne[1] = 8
    assert _validate(p) == sa.E_INVALID_ARGUMENT  # fewer mask rows than n_q
    p.mask.ne[1] = 16
    p.mask.data = ADDR["out"] + 4096  # the output would overwrite the mask it reads
    assert _validate(p) == sa.E_INVALID_ARGUMENT


@pytest.mark.parametrize("mutate", [
    lambda p: p.out.nb.__setitem__(2, p.out.nb[1]),          # rows j and head h+1 of row j-1 alias
    lambda p: p.out.nb.__setitem__(3, 4096),                 # streams inside one another's rows
    lambda p: setattr(p.out, "data", ADDR["q"]),             # output over Q
    lambda p: setattr(p.out, "data", ADDR["k"] + (1 << 20)),  # output inside the K cache
    lambda p: setattr(p.out, "data", ADDR["v"]),
    lambda p: setattr(p, "kv_len", ADDR["out"] + 256),       # the lengths under the output
])
def test_output_must_not_alias_itself_or_what_the_call_reads(mutate):
    """Work-groups write output rows in no fixed order, while others still read Q, K, V, the
    mask and the lengths: every output row must be its own and touch nothing that is read."""
    p = _params()
    assert _validate(p) == sa.OK
    mutate(p)
    assert _validate(p) == sa.E_INVALID_ARGUMENT


def test_workspace_must_not_overlap_the_views():
    """The split kernel writes its partials into the workspace while it reads the views; an
    overlapping workspace is rejected before any launch (so this runs without a GPU)."""
    lib = sa.load_library()
    p = _params()
    n = ctypes.c_size_t(0)
    assert lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n)) == sa.OK
    for where in ("q", "k", "v", "out", "kv_len"):
        p.workspace = ADDR[where] - 256 if where != "q" else ADDR["q"]
        p.workspace_bytes = n.value + 512
        assert lib.sixi_attn_forward(ctypes.byref(p)) == sa.E_INVALID_ARGUMENT, where


def _paged_params(S, stride, n_q=1, n_pages=1024):
    """A paged call: K and V pools of 256-cell pages, a page table of `stride` pages per stream."""
    p = _params(S=S, n_q=n_q)
    D, Hkv, row = 128, 4, 256
    nb = [2, Hkv * row, row, 256 * Hkv * row]
    p.k = sa.make_view(ADDR["k"], sa.TYPE_F16, [D, 256, Hkv, n_pages], nb)
    p.v = sa.make_view(ADDR["v"], sa.TYPE_F16, [D, 256, Hkv, n_pages], nb)
    p.page_table = ADDR["pt"]
    p.page_table_stride = stride
    return p


def test_paged_cost_line_stays_within_32_bits():
    """The split kernels sum the streams' tile counts in 32-bit integers.  A paged description
    may give every stream 2^26 cells; 512 such streams on the 16-cell kernel (2^22 tiles each)
    would overflow the sum, so the call is refused; half the cells per stream fit."""
    assert _validate(_paged_params(S=512, stride=1 << 18)) == sa.E_UNSUPPORTED
    assert _validate(_paged_params(S=512, stride=1 << 17)) == sa.OK
    assert _validate(_paged_params(S=2, stride=1 << 18)) == sa.OK


def test_forward_without_workspace_fails_before_any_launch():
    p = _params()
    p.workspace = None
    p.workspace_bytes = 0
    assert sa.load_library().sixi_attn_forward(ctypes.byref(p)) == sa.E_OUT_OF_BOUNDS


# ---- include/sixi_kv.h ---------------------------------------------------------------------

def _kv_write_params(S=3, n_rows=16, Hkv=4, D=128, n_cells=4096, src_type=sa.TYPE_F32, dst_type=sa.TYPE_F16):
    p = sa.SixiKvWriteParams()
    es = 4 if src_type == sa.TYPE_F32 else 2
    p.src = sa.make_view(FAKE, src_type, [D, n_rows, Hkv, S], [es, Hkv * D * es, D * es, n_rows * Hkv * D * es])
    row = D * 2 if dst_type == sa.TYPE_F16 else D // 32 * 34
    nb0 = 2 if dst_type == sa.TYPE_F16 else 34
    p.dst = sa.make_view(FAKE, dst_type, [D, n_cells, Hkv, S], [nb0, Hkv * row, row, n_cells * Hkv * row])
    p.kv_len = FAKE
    p.q_len = None
    return p


def _kv_validate(p):
    return sa.load_library().sixi_kv_write_validate(ctypes.byref(p))


def test_kv_write_valid_descriptions_pass():
    for st in (sa.TYPE_F32, sa.TYPE_F16):
        for dt in (sa.TYPE_F16, sa.TYPE_Q8_0):
            for D in (128, 256):
                assert _kv_validate(_kv_write_params(D=D, src_type=st, dst_type=dt)) == sa.OK


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p, "flags", 2), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.src, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.dst, "type", sa.TYPE_F32), sa.E_INVALID_ARGUMENT),      # cache must be f16/q8_0
    (lambda p: setattr(p.src, "type", sa.TYPE_Q8_0), sa.E_INVALID_ARGUMENT),     # source must be f32/f16
    (lambda p: p.dst.ne.__setitem__(0, 64), sa.E_INVALID_ARGUMENT),              # head dims differ
    (lambda p: (p.src.ne.__setitem__(0, 48), p.dst.ne.__setitem__(0, 48)), sa.E_INVALID_ARGUMENT),  # D % 32
    (lambda p: p.dst.ne.__setitem__(2, 8), sa.E_INVALID_ARGUMENT),               # kv-heads differ
    (lambda p: p.dst.ne.__setitem__(3, 2), sa.E_INVALID_ARGUMENT),               # streams differ
    (lambda p: p.src.nb.__setitem__(0, 8), sa.E_INVALID_ARGUMENT),               # rows not contiguous
    (lambda p: p.dst.nb.__setitem__(1, 128), sa.E_INVALID_ARGUMENT),             # cells would alias
    (lambda p: p.dst.nb.__setitem__(3, 1024), sa.E_INVALID_ARGUMENT),            # streams would alias
    (lambda p: setattr(p.src, "data", FAKE + 4), sa.E_ALIGNMENT),
    (lambda p: p.src.nb.__setitem__(1, 2056), sa.E_ALIGNMENT),
    (lambda p: setattr(p.dst, "data", FAKE + 8), sa.E_ALIGNMENT),                # f16 rows 16-B aligned
    (lambda p: p.src.nb.__setitem__(3, 1 << 62), sa.E_INTEGER_OVERFLOW),
])
def test_kv_write_rejects(mutate, code):
    p = _kv_write_params()
    mutate(p)
    assert _kv_validate(p) == code
    assert sa.load_library().sixi_kv_write(ctypes.byref(p)) == code


def test_kv_write_q8_rows_need_only_2_byte_alignment():
    p = _kv_write_params(dst_type=sa.TYPE_Q8_0)
    p.dst.data = FAKE + 2
    assert _kv_validate(p) == sa.OK


def _kv_copy_params(S=4, Hkv=4, D=128, n_cells=1024, dst_type=sa.TYPE_F16):
    p = sa.SixiKvCopyParams()
    row = D * 2 if dst_type == sa.TYPE_F16 else D // 32 * 34
    nb0 = 2 if dst_type == sa.TYPE_F16 else 34
    p.cache = sa.make_view(FAKE, dst_type, [D, n_cells, Hkv, S], [nb0, Hkv * row, row, n_cells * Hkv * row])
    p.src_stream, p.dst_stream, p.src_cell, p.dst_cell, p.n_cells = 0, 1, 0, 0, 512
    return p


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p.cache, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.cache, "type", sa.TYPE_F32), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p, "dst_stream", 4), sa.E_OUT_OF_BOUNDS),
    (lambda p: setattr(p, "src_stream", -1), sa.E_OUT_OF_BOUNDS),
    (lambda p: setattr(p, "src_cell", 600), sa.E_OUT_OF_BOUNDS),                  # 600 + 512 > 1024
    (lambda p: setattr(p, "n_cells", -1), sa.E_INVALID_ARGUMENT),
    (lambda p: (setattr(p, "dst_stream", 0), setattr(p, "dst_cell", 256)), sa.E_INVALID_ARGUMENT),  # overlap
    (lambda p: p.cache.nb.__setitem__(1, 64), sa.E_INVALID_ARGUMENT),             # cells would alias
    (lambda p: setattr(p.cache, "data", FAKE + 1), sa.E_ALIGNMENT),
    (lambda p: (setattr(p, "src_cell", 1), setattr(p, "n_cells", (1 << 63) - 1)), sa.E_INTEGER_OVERFLOW),
])
def test_kv_copy_rejects(mutate, code):
    p = _kv_copy_params()
    mutate(p)
    assert sa.load_library().sixi_kv_copy(ctypes.byref(p)) == code


def test_kv_copy_of_nothing_is_ok_without_a_launch():
    p = _kv_copy_params()
    p.n_cells = 0
    assert sa.load_library().sixi_kv_copy(ctypes.byref(p)) == sa.OK


def _prologue_params(S=2, R=16, H=24, Hkv=4, D=256, n_cells=4096, cache_type=sa.TYPE_F16, n_rot=64):
    p = sa.SixiQkPrologueParams()
    p.qg = sa.make_view(FAKE, sa.TYPE_F32, [2 * D, H, R, S], [4, 2 * D * 4, H * 2 * D * 4, R * H * 2 * D * 4])
    kv = [4, D * 4, Hkv * D * 4, R * Hkv * D * 4]
    p.k = sa.make_view(FAKE, sa.TYPE_F32, [D, Hkv, R, S], kv)
    p.v = sa.make_view(FAKE, sa.TYPE_F32, [D, Hkv, R, S], kv)
    p.q_norm = p.k_norm = FAKE
    p.eps, p.rope_base, p.n_rot, p.flags = 1e-6, 1e7, n_rot, 0
    p.kv_len = FAKE
    p.q_out = sa.make_view(FAKE, sa.TYPE_F32, [D, R, H, S], [4, H * D * 4, D * 4, R * H * D * 4])
    row = D * 2 if cache_type == sa.TYPE_F16 else D // 32 * 34
    nb0 = 2 if cache_type == sa.TYPE_F16 else 34
    for name in ("k_cache", "v_cache"):
        setattr(p, name, sa.make_view(FAKE, cache_type, [D, n_cells, Hkv, S], [nb0, Hkv * row, row, n_cells * Hkv * row]))
    return p


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p, "flags", 2), sa.E_INVALID_ARGUMENT),            # unknown flag bit
    (lambda p: setattr(p, "q_norm", None), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.k_cache, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: (p.q_out.ne.__setitem__(0, 64), p.qg.ne.__setitem__(0, 128)), sa.E_UNSUPPORTED),   # head of 64
    (lambda p: p.qg.ne.__setitem__(0, 256), sa.E_INVALID_ARGUMENT),            # no gate half
    (lambda p: p.q_out.ne.__setitem__(2, 16), sa.E_INVALID_ARGUMENT),          # q-heads differ
    (lambda p: p.v.ne.__setitem__(1, 2), sa.E_INVALID_ARGUMENT),               # kv-heads differ
    (lambda p: p.v_cache.ne.__setitem__(1, 2048), sa.E_INVALID_ARGUMENT),      # caches differ
    (lambda p: setattr(p.v_cache, "type", sa.TYPE_Q8_0), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.q_out, "type", sa.TYPE_F16), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p, "n_rot", 66), sa.E_INVALID_ARGUMENT),                # not a multiple of D/32
    (lambda p: setattr(p, "n_rot", 264), sa.E_INVALID_ARGUMENT),               # more than D
    (lambda p: setattr(p, "eps", -1.0), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p, "rope_base", 0.0), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p, "eps", float("nan")), sa.E_INVALID_ARGUMENT),
    (lambda p: p.q_out.nb.__setitem__(2, 512), sa.E_INVALID_ARGUMENT),         # q-heads would alias
    (lambda p: p.k_cache.nb.__setitem__(1, 64), sa.E_INVALID_ARGUMENT),        # cells would alias
    (lambda p: setattr(p.qg, "data", FAKE + 8), sa.E_ALIGNMENT),
    (lambda p: setattr(p, "k_norm", FAKE + 4), sa.E_ALIGNMENT),
    (lambda p: setattr(p.k_cache, "data", FAKE + 2), sa.E_ALIGNMENT),          # f16 rows 16-B aligned
    (lambda p: p.k.nb.__setitem__(2, 1 << 62), sa.E_INTEGER_OVERFLOW),        # 15 rows of 2^62 bytes
])
def test_qk_prologue_rejects(mutate, code):
    p = _prologue_params()
    mutate(p)
    assert sa.load_library().sixi_qk_prologue(ctypes.byref(p)) == code


def test_qk_prologue_takes_an_f16_q_out():
    D, R, H = 256, 16, 24
    f16 = lambda p: setattr(p, "q_out", sa.make_view(FAKE, sa.TYPE_F16, [D, R, H, 0], [2, H * D * 2, D * 2, R * H * D * 2]))
    p = _prologue_params(S=0)
    f16(p)
    assert sa.load_library().sixi_qk_prologue(ctypes.byref(p)) == sa.OK      # (no rows: no launch)
    p.q_out.nb[1] = H * D * 2 + 2                                            # rows not 16-byte aligned
    assert sa.load_library().sixi_qk_prologue(ctypes.byref(p)) == sa.E_ALIGNMENT
    p.q_out.nb[1] = H * D * 2
    p.q_out.nb[2] = D                                                         # heads would alias
    assert sa.load_library().sixi_qk_prologue(ctypes.byref(p)) == sa.E_INVALID_ARGUMENT
    p = _prologue_params(S=0, cache_type=sa.TYPE_Q8_0)                       # q8_0 cache: f32 Q only
    f16(p)
    assert sa.load_library().sixi_qk_prologue(ctypes.byref(p)) == sa.E_INVALID_ARGUMENT


def test_qk_prologue_q8_cache_and_empty_block():
    p = _prologue_params(cache_type=sa.TYPE_Q8_0)
    p.k_cache.data = FAKE + 2                      # q8_0 rows need 2-byte alignment only
    p.flags = 1
    assert sa.load_library().sixi_qk_prologue(ctypes.byref(p)) == sa.E_INVALID_ARGUMENT
    for cache_type, D in ((sa.TYPE_F16, 128), (sa.TYPE_Q8_0, 256)):
        p = _prologue_params(S=0, D=D, cache_type=cache_type, n_rot=D)   # nothing to do: no launch
        assert sa.load_library().sixi_qk_prologue(ctypes.byref(p)) == sa.OK


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p.out, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: p.qg.ne.__setitem__(0, 256), sa.E_INVALID_ARGUMENT),
    (lambda p: (p.out.ne.__setitem__(0, 96), p.qg.ne.__setitem__(0, 192)), sa.E_UNSUPPORTED),
    (lambda p: p.out.nb.__setitem__(1, 0), sa.E_INVALID_ARGUMENT),             # heads would alias
    (lambda p: setattr(p.out, "data", FAKE + 4), sa.E_ALIGNMENT),
])
def test_attn_gate_rejects(mutate, code):
    D, H, R, S = 256, 24, 16, 2
    p = sa.SixiAttnGateParams()
    p.out = sa.make_view(FAKE, sa.TYPE_F32, [D, H, R, S], [4, D * 4, H * D * 4, R * H * D * 4])
    p.qg = sa.make_view(FAKE, sa.TYPE_F32, [2 * D, H, R, S], [4, 2 * D * 4, H * 2 * D * 4, R * H * 2 * D * 4])
    mutate(p)
    assert sa.load_library().sixi_attn_gate(ctypes.byref(p)) == code


def _gdn_params(S=2, n=16, G=48, K=128, HD=128):
    base = [FAKE]

    def v4(ne):  # each view in an address range of its own
        nb = [4]
        for d in range(3):
            nb.append(nb[-1] * ne[d])
        base[0] += 1 << 32
        return sa.make_view(base[0], sa.TYPE_F32, ne, nb)
    p = sa.SixiGdnParams()
    p.q, p.k = v4([K, G, n, S]), v4([K, G, n, S])
    p.v, p.y = v4([HD, G, n, S]), v4([HD, G, n, S])
    p.alpha, p.beta = v4([G, n, S, 1]), v4([G, n, S, 1])
    p.state_in = p.state_out = v4([K, HD, G, S])
    p.flags = 0
    return p


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p, "flags", 4), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.q, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.v, "type", sa.TYPE_F16), sa.E_INVALID_ARGUMENT),
    (lambda p: (p.q.ne.__setitem__(0, 96), p.k.ne.__setitem__(0, 96)), sa.E_UNSUPPORTED),     # state size 96
    (lambda p: p.k.ne.__setitem__(1, 16), sa.E_INVALID_ARGUMENT),               # groups differ
    (lambda p: p.alpha.ne.__setitem__(1, 8), sa.E_INVALID_ARGUMENT),            # rows differ
    (lambda p: p.state_out.ne.__setitem__(2, 24), sa.E_INVALID_ARGUMENT),
    (lambda p: p.y.nb.__setitem__(1, 0), sa.E_INVALID_ARGUMENT),                # outputs would alias
    (lambda p: setattr(p.state_out, "data", p.state_in.data + 4096), sa.E_INVALID_ARGUMENT),  # overlaps the input state
    (lambda p: setattr(p.y, "data", p.q.data + 512), sa.E_INVALID_ARGUMENT),   # y over an input
    (lambda p: setattr(p.y, "data", p.beta.data), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.y, "data", p.state_in.data), sa.E_INVALID_ARGUMENT),  # y over the (in-place) state
    (lambda p: setattr(p.q, "data", p.state_out.data + 64), sa.E_INVALID_ARGUMENT),  # the state written over q
    (lambda p: setattr(p.q, "data", p.q.data + 4), sa.E_ALIGNMENT),
    (lambda p: setattr(p.beta, "data", p.beta.data + 2), sa.E_ALIGNMENT),
    (lambda p: p.v.nb.__setitem__(2, 1 << 62), sa.E_INTEGER_OVERFLOW),
])
def test_gdn_verify_rejects(mutate, code):
    p = _gdn_params()
    mutate(p)
    assert sa.load_library().sixi_gdn_verify(ctypes.byref(p)) == code


def test_gdn_verify_without_streams_launches_nothing():
    for K, HD in ((64, 64), (128, 128)):
        assert sa.load_library().sixi_gdn_verify(ctypes.byref(_gdn_params(S=0, K=K, HD=HD))) == sa.OK


def test_gdn_verify_input_state_rows_must_not_overlap():
    p = _gdn_params()
    p.state_out = sa.make_view(FAKE + (1 << 44), sa.TYPE_F32, list(p.state_in.ne), list(p.state_in.nb))
    p.state_in.nb[1] = 256                       # input rows of 512 bytes 256 apart
    assert sa.load_library().sixi_gdn_verify(ctypes.byref(p)) == sa.E_INVALID_ARGUMENT


GATE = FAKE + (8 << 36)  # the fused gate's qg view, in an address range of its own


def _gated(S=2, n_q=16, H=24, D=128):
    p = _params(S=S, n_q=n_q, H=H, D=D)
    p.flags = sa.FLAG_GATE
    p.gate_qg = sa.make_view(GATE, sa.TYPE_F32, [2 * D, H, n_q, S], [4, 2 * D * 4, H * 2 * D * 4, n_q * H * 2 * D * 4])
    return p


def test_gated_descriptions_pass():
    for D in (128, 256):
        for n_q in (1, 16, 300):
            assert _validate(_gated(n_q=n_q, D=D)) == sa.OK, (D, n_q)
    p = _gated()
    p.gate_qg.ne[2] = 20  # more rows than the call's (a padded block)
    assert _validate(p) == sa.OK


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p.gate_qg, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.gate_qg, "type", sa.TYPE_F16), sa.E_INVALID_ARGUMENT),
    (lambda p: p.gate_qg.ne.__setitem__(0, 128), sa.E_INVALID_ARGUMENT),   # not 2D per head
    (lambda p: p.gate_qg.ne.__setitem__(1, 12), sa.E_INVALID_ARGUMENT),    # not H heads
    (lambda p: p.gate_qg.ne.__setitem__(2, 15), sa.E_INVALID_ARGUMENT),    # fewer rows than n_q
    (lambda p: p.gate_qg.ne.__setitem__(3, 1), sa.E_INVALID_ARGUMENT),     # not S streams
    (lambda p: p.gate_qg.nb.__setitem__(0, 8), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.gate_qg, "data", GATE + 8), sa.E_ALIGNMENT),
    (lambda p: p.gate_qg.nb.__setitem__(2, 24 * 256 * 4 + 4), sa.E_ALIGNMENT),
    (lambda p: setattr(p.gate_qg, "data", ADDR["out"] + 4096), sa.E_INVALID_ARGUMENT),  # the output over the gate
    (lambda p: setattr(p, "flags", sa.FLAG_GATE | 4), sa.E_INVALID_ARGUMENT),           # an unknown flag
])
def test_gated_descriptions_are_checked(mutate, code):
    p = _gated()
    mutate(p)
    assert _validate(p) == code


def test_gate_is_not_read_without_its_flag():
    p = _gated()
    p.flags = 0
    p.gate_qg = sa.make_view(0, sa.TYPE_F16, [1, 1, 1, 1], [0, 0, 0, 0])  # garbage, ignored
    assert _validate(p) == sa.OK


def test_workspace_must_not_overlap_the_gate():
    lib = sa.load_library()
    p = _gated()
    n = ctypes.c_size_t(0)
    assert lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n)) == sa.OK
    p.workspace = GATE - 256
    p.workspace_bytes = n.value + 512
    assert lib.sixi_attn_forward(ctypes.byref(p)) == sa.E_INVALID_ARGUMENT
