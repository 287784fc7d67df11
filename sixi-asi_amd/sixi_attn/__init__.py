"""Python binding of the MI355X attention hot path (libsixi_attn.so, include/sixi_attn.h).

The operator mirrors ggml's ``ggml_flash_attn_ext(q, k, v, mask, scale, max_bias,
logit_softcap)`` -- the op the reference reaches through ``llama_decode`` at
src/core/core_execution.cpp:2074 (verify), :3536 (prefill chunk) and :3811 (decode) --
with per-stream device lengths in place of the host-built KQ mask.  Tensors use the
row-major mirror of ggml's views: ``q[S, n_q, H, D]``, ``k/v[S, n_kv, Hkv, D]`` (f16, or
uint8 ``[S, n_kv, Hkv, D/32*34]`` q8_0 blocks), ``out[S, n_q, H, D]`` f32; strides are
taken from the tensors, so cache slices and paged layouts pass through unchanged.

torch provides device memory and the stream; the computation is the HIP library.  There is
no CPU fallback: a missing library raises ``SixiAttnUnavailable``.
"""
from __future__ import annotations

import ctypes
import math
import os
import pathlib
from typing import Optional

PKG_DIR = pathlib.Path(__file__).resolve().parent.parent
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libsixi_attn.so"

# ggml type ids
TYPE_F32, TYPE_F16, TYPE_Q8_0 = 0, 1, 8
# mask modes
MASK_NONE, MASK_BLOCK_CAUSAL, MASK_EXPLICIT = 0, 1, 2
# sixi_attn_params.flags; the f16 staging of a q8_0 cache stays under STAGE_CAP_BYTES
FLAG_BOUNDED_WORKSPACE = 1
FLAG_GATE = 2
STAGE_CAP_BYTES = 64 << 20
# status codes (negated sixi_asi::ErrorCode, include/sixi_asi/common.hpp:40-67)
OK = 0
E_INVALID_ARGUMENT = -1
E_OUT_OF_BOUNDS = -2
E_INTEGER_OVERFLOW = -3
E_ALIGNMENT = -15
E_BACKEND = -23
E_UNSUPPORTED = -24

EXPORTED_SYMBOLS = (
    "sixi_attn_forward",
    "sixi_attn_forward_noalloc",
    "sixi_attn_workspace_bytes",
    "sixi_attn_validate",
    "sixi_attn_strerror",
    "sixi_attn_abi_version",
    "sixi_kv_write",
    "sixi_kv_write_validate",
    "sixi_kv_copy",
    "sixi_kv_pool_create",
    "sixi_kv_pool_destroy",
    "sixi_kv_pool_attach",
    "sixi_kv_pool_prepare_write",
    "sixi_kv_pool_seq_rm",
    "sixi_kv_pool_seq_cp",
    "sixi_kv_pool_page_table",
    "sixi_kv_pool_upload",
    "sixi_kv_pool_free_pages",
    "sixi_kv_pool_stream_pages",
    "sixi_kv_pool_page_refs",
    "sixi_verify_plan",
    "sixi_qk_prologue",
    "sixi_attn_gate",
    "sixi_gdn_verify",
)


class SixiAttnUnavailable(RuntimeError):
    """The HIP library is not built or cannot be loaded."""


class SixiAttnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"sixi_attn status {code}: {msg}")
        self.code = code


class SixiView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_int64 * 4),
    ]


class SixiAttnParams(ctypes.Structure):
    _fields_ = [
        ("q", SixiView),
        ("k", SixiView),
        ("v", SixiView),
        ("out", SixiView),
        ("kv_len", ctypes.c_void_p),
        ("q_len", ctypes.c_void_p),
        ("mask_mode", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("mask", SixiView),
        ("scale", ctypes.c_float),
        ("max_bias", ctypes.c_float),
        ("logit_softcap", ctypes.c_float),
        ("reserved_f", ctypes.c_float),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("stream", ctypes.c_void_p),
        ("page_table", ctypes.c_void_p),
        ("page_table_stride", ctypes.c_int64),
        ("gate_qg", SixiView),
    ]


class SixiKvWriteParams(ctypes.Structure):
    _fields_ = [
        ("src", SixiView),
        ("dst", SixiView),
        ("kv_len", ctypes.c_void_p),
        ("q_len", ctypes.c_void_p),
        ("flags", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("stream", ctypes.c_void_p),
        ("page_table", ctypes.c_void_p),
        ("page_table_stride", ctypes.c_int64),
    ]


class SixiKvCopyParams(ctypes.Structure):
    _fields_ = [
        ("cache", SixiView),
        ("src_stream", ctypes.c_int32),
        ("dst_stream", ctypes.c_int32),
        ("src_cell", ctypes.c_int64),
        ("dst_cell", ctypes.c_int64),
        ("n_cells", ctypes.c_int64),
        ("stream", ctypes.c_void_p),
    ]


class SixiQkPrologueParams(ctypes.Structure):
    _fields_ = [
        ("qg", SixiView),
        ("k", SixiView),
        ("v", SixiView),
        ("q_norm", ctypes.c_void_p),
        ("k_norm", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("rope_base", ctypes.c_float),
        ("n_rot", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("kv_len", ctypes.c_void_p),
        ("q_len", ctypes.c_void_p),
        ("q_out", SixiView),
        ("k_cache", SixiView),
        ("v_cache", SixiView),
        ("stream", ctypes.c_void_p),
        ("page_table", ctypes.c_void_p),
        ("page_table_stride", ctypes.c_int64),
    ]


class SixiAttnGateParams(ctypes.Structure):
    _fields_ = [
        ("out", SixiView),
        ("qg", SixiView),
        ("q_len", ctypes.c_void_p),
        ("stream", ctypes.c_void_p),
    ]


class SixiGdnParams(ctypes.Structure):
    _fields_ = [
        ("q", SixiView),
        ("k", SixiView),
        ("v", SixiView),
        ("alpha", SixiView),
        ("beta", SixiView),
        ("y", SixiView),
        ("state_in", SixiView),
        ("state_out", SixiView),
        ("q_len", ctypes.c_void_p),
        ("snap", ctypes.c_void_p),
        ("flags", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("stream", ctypes.c_void_p),
    ]


GDN_DECAY_FIRST = 1


class SixiVerifyStream(ctypes.Structure):
    _fields_ = [("stream", ctypes.c_int32), ("cached", ctypes.c_int32), ("real", ctypes.c_int32)]


class SixiVerifySlot(ctypes.Structure):
    _fields_ = [("part", ctypes.c_int32), ("index", ctypes.c_int32), ("row_offset", ctypes.c_int32),
                ("rows", ctypes.c_int32)]


PAD_REFERENCE, PAD_NONE = 0, 1

_lib = None


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Loads libsixi_attn.so (built in-tree by sixi-asi_amd/build.py)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path) if path else LIB_PATH
    if not p.exists():
        raise SixiAttnUnavailable(f"{p} is missing: run `python sixi-asi_amd/build.py`")
    try:
        lib = ctypes.CDLL(str(p))
    except OSError as e:  # pragma: no cover - loader failure is environment specific
        raise SixiAttnUnavailable(f"cannot load {p}: {e}") from e
    P = ctypes.POINTER(SixiAttnParams)
    lib.sixi_attn_forward.argtypes = [P]
    lib.sixi_attn_forward.restype = ctypes.c_int
    lib.sixi_attn_forward_noalloc.argtypes = [P]
    lib.sixi_attn_forward_noalloc.restype = ctypes.c_int
    lib.sixi_attn_validate.argtypes = [P]
    lib.sixi_attn_validate.restype = ctypes.c_int
    lib.sixi_attn_workspace_bytes.argtypes = [P, ctypes.POINTER(ctypes.c_size_t)]
    lib.sixi_attn_workspace_bytes.restype = ctypes.c_int
    lib.sixi_attn_strerror.argtypes = [ctypes.c_int]
    lib.sixi_attn_strerror.restype = ctypes.c_char_p
    lib.sixi_attn_abi_version.argtypes = []
    lib.sixi_attn_abi_version.restype = ctypes.c_int
    PW = ctypes.POINTER(SixiKvWriteParams)
    lib.sixi_kv_write.argtypes = [PW]
    lib.sixi_kv_write.restype = ctypes.c_int
    lib.sixi_kv_write_validate.argtypes = [PW]
    lib.sixi_kv_write_validate.restype = ctypes.c_int
    lib.sixi_kv_copy.argtypes = [ctypes.POINTER(SixiKvCopyParams)]
    lib.sixi_kv_copy.restype = ctypes.c_int
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    for name, args, res in (
            ("sixi_kv_pool_create", [i32, i32, i32, ctypes.POINTER(vp)], ctypes.c_int),
            ("sixi_kv_pool_destroy", [vp], None),
            ("sixi_kv_pool_attach", [vp, ctypes.POINTER(SixiView)], ctypes.c_int),
            ("sixi_kv_pool_prepare_write", [vp, i32, i64, i64, vp], ctypes.c_int),
            ("sixi_kv_pool_seq_rm", [vp, i32, i64], ctypes.c_int),
            ("sixi_kv_pool_seq_cp", [vp, i32, i32, i64], ctypes.c_int),
            ("sixi_kv_pool_page_table", [vp, vp], ctypes.c_int),
            ("sixi_kv_pool_upload", [vp, vp, vp], ctypes.c_int),
            ("sixi_kv_pool_free_pages", [vp], i32),
            ("sixi_kv_pool_stream_pages", [vp, i32], i32),
            ("sixi_kv_pool_page_refs", [vp, i32], i32)):
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    lib.sixi_verify_plan.argtypes = [ctypes.POINTER(SixiVerifyStream), ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                     ctypes.POINTER(SixiVerifySlot), ctypes.POINTER(ctypes.c_int32)]
    lib.sixi_verify_plan.restype = ctypes.c_int
    lib.sixi_qk_prologue.argtypes = [ctypes.POINTER(SixiQkPrologueParams)]
    lib.sixi_qk_prologue.restype = ctypes.c_int
    lib.sixi_attn_gate.argtypes = [ctypes.POINTER(SixiAttnGateParams)]
    lib.sixi_attn_gate.restype = ctypes.c_int
    lib.sixi_gdn_verify.argtypes = [ctypes.POINTER(SixiGdnParams)]
    lib.sixi_gdn_verify.restype = ctypes.c_int
    if path is None:
        _lib = lib
    return lib


def strerror(code: int) -> str:
    return load_library().sixi_attn_strerror(code).decode()


def make_view(data_ptr: int, type_id: int, ne, nb) -> SixiView:
    v = SixiView()
    v.data = data_ptr
    v.type = type_id
    for i in range(4):
        v.ne[i] = int(ne[i])
        v.nb[i] = int(nb[i])
    return v


def view_of(t, type_id: Optional[int] = None, head_dim: Optional[int] = None,
            tokens_heads: bool = True) -> SixiView:
    """ggml view of a 4-d torch tensor whose last dim is innermost.

    tokens_heads=True: t is (S, tokens, heads, D) and the view is ggml's [D, tokens, heads, S]
    (Q, K, V as llama.cpp permutes them); False: the plain reversal (out, mask).
    For q8_0 pass a uint8 tensor whose last dim holds the packed blocks and ``head_dim``.
    """
    import torch

    if t.dim() != 4:
        raise ValueError("expected a 4-d tensor")
    es = t.element_size()
    order = (3, 1, 2, 0) if tokens_heads else (3, 2, 1, 0)
    nb = [t.stride(i) * es for i in order]
    ne = [t.shape[i] for i in order]
    if type_id is None:
        type_id = {torch.float32: TYPE_F32, torch.float16: TYPE_F16}[t.dtype]
    if type_id == TYPE_Q8_0:
        if t.dtype != torch.uint8 or head_dim is None or t.shape[-1] != head_dim // 32 * 34:
            raise ValueError("q8_0 view needs a uint8 tensor of D/32*34 bytes per row and head_dim")
        if t.stride(-1) != 1:
            raise ValueError("q8_0 rows must be contiguous")
        ne[0] = head_dim
        nb[0] = 34
    return make_view(t.data_ptr(), type_id, ne, nb)


class FlashAttnExt:
    """``ggml_flash_attn_ext`` over per-stream KV caches on one gfx950 GPU.

    Keeps a device workspace (grown on demand) so repeated calls allocate nothing.  A buffer
    that a larger call supersedes stays allocated for the life of the object, so a HIP graph
    captured over an earlier call still owns the memory its kernels write.  A caller may
    also pass its own ``workspace`` (a uint8 device tensor of at least
    :meth:`workspace_bytes`), e.g. one sized once before capture.
    """

    def __init__(self, device=None):
        import torch

        self.lib = load_library()
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self._ws = None
        self._retired = []  # superseded workspaces: graphs captured before a regrowth still use them

    def params(self, q, k, v, out, kv_len=None, q_len=None, mask_mode=MASK_BLOCK_CAUSAL, mask=None,
               scale=None, max_bias=0.0, logit_softcap=0.0, kv_type=None, stream=None,
               page_table=None, bounded_workspace=False, gate=None) -> SixiAttnParams:
        """``page_table`` (an int32 device tensor [S, pages per stream]): k and v are page pools
        ``[n_pages, 256, Hkv, D]`` (uint8 q8_0 blocks as for a cache) read through it.
        ``bounded_workspace`` sets SIXI_ATTN_FLAG_BOUNDED_WORKSPACE (no f16 staging of a q8_0
        cache: the workspace does not grow with the cache).  ``gate`` (the layer prologue's qg,
        f32 [S, rows, H, 2D]) sets SIXI_ATTN_FLAG_GATE: out = attention * sigmoid(qg[..., D:])."""
        import torch

        D = q.shape[-1]
        kvt = kv_type if kv_type is not None else (TYPE_Q8_0 if k.dtype == torch.uint8 else None)
        p = SixiAttnParams()
        p.q = view_of(q)
        p.k = view_of(k, kvt, D if kvt == TYPE_Q8_0 else None)
        p.v = view_of(v, kvt, D if kvt == TYPE_Q8_0 else None)
        p.out = view_of(out, tokens_heads=False)
        p.kv_len = kv_len.data_ptr() if kv_len is not None else None
        p.q_len = q_len.data_ptr() if q_len is not None else None
        p.mask_mode = mask_mode
        p.flags = FLAG_BOUNDED_WORKSPACE if bounded_workspace else 0
        if gate is not None:
            p.flags |= FLAG_GATE
            p.gate_qg = view_of(gate, tokens_heads=False)
        if mask is not None:
            # mask tensor [S or 1, 1, n_q_pad, n_kv] f16
            p.mask = view_of(mask, TYPE_F16, tokens_heads=False)
        p.scale = 1.0 / math.sqrt(D) if scale is None else scale
        p.max_bias = max_bias
        p.logit_softcap = logit_softcap
        p.stream = stream
        if page_table is not None:
            p.page_table = page_table.data_ptr()
            p.page_table_stride = page_table.stride(0)
        return p

    def workspace_bytes(self, p: SixiAttnParams) -> int:
        n = ctypes.c_size_t(0)
        rc = self.lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n))
        if rc != OK:
            raise SixiAttnError(rc, strerror(rc))
        return n.value

    def _workspace(self, nbytes: int):
        import torch

        if self._ws is None or self._ws.numel() < nbytes:
            if self._ws is not None:
                self._retired.append(self._ws)
            self._ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        return self._ws

    def __call__(self, q, k, v, out, kv_len=None, q_len=None, mask_mode=MASK_BLOCK_CAUSAL, mask=None,
                 scale=None, max_bias=0.0, logit_softcap=0.0, kv_type=None, stream=None, check=True,
                 workspace=None, noalloc=False, page_table=None, bounded_workspace=False, gate=None) -> int:
        """One call.  ``noalloc=True`` runs sixi_attn_forward_noalloc (the library's fixed
        device scratch, no workspace); ``page_table`` reads k and v as page pools;
        ``bounded_workspace`` never stages a q8_0 cache as f16; ``gate`` fuses the layer's
        output gate (see :meth:`params`)."""
        import torch

        p = self.params(q, k, v, out, kv_len, q_len, mask_mode, mask, scale, max_bias, logit_softcap,
                        kv_type, stream, page_table, bounded_workspace, gate)
        if p.stream is None:
            p.stream = torch.cuda.current_stream(self.device).cuda_stream
        if noalloc:
            rc = self.lib.sixi_attn_forward_noalloc(ctypes.byref(p))
            if check and rc != OK:
                raise SixiAttnError(rc, strerror(rc))
            return rc
        n = ctypes.c_size_t(0)
        rc = self.lib.sixi_attn_workspace_bytes(ctypes.byref(p), ctypes.byref(n))
        if rc == OK:
            ws = self._workspace(n.value) if workspace is None else workspace
            p.workspace = ws.data_ptr()
            p.workspace_bytes = ws.numel() * ws.element_size()
            rc = self.lib.sixi_attn_forward(ctypes.byref(p))
        if check and rc != OK:
            raise SixiAttnError(rc, strerror(rc))
        return rc


def _cache_view(cache, head_dim):
    import torch

    if cache.dtype == torch.uint8:
        return view_of(cache, TYPE_Q8_0, head_dim)
    return view_of(cache)


def kv_write_params(src, cache, kv_len=None, q_len=None, stream=None, page_table=None) -> SixiKvWriteParams:
    """Parameters of ``sixi_kv_write`` for torch tensors: ``src[S, n_rows, Hkv, D]`` f32 or
    f16, ``cache[S, n_cells, Hkv, D]`` f16 (or uint8 q8_0 blocks ``[..., D/32*34]``); with
    ``page_table`` (int32 device [S, pages per stream]) the cache is a page pool
    ``[n_pages, 256, Hkv, D]``."""
    p = SixiKvWriteParams()
    p.src = view_of(src)
    p.dst = _cache_view(cache, src.shape[-1])
    p.kv_len = kv_len.data_ptr() if kv_len is not None else None
    p.q_len = q_len.data_ptr() if q_len is not None else None
    p.flags = 0
    p.stream = stream
    if page_table is not None:
        p.page_table = page_table.data_ptr()
        p.page_table_stride = page_table.stride(0)
    return p


def kv_write(src, cache, kv_len=None, q_len=None, stream=None, check=True, page_table=None) -> int:
    """Stores the new K (or V) rows of each stream in its cache cells.

    Row j < q_len[s] of stream s goes to cell kv_len[s] + j, converted to the cache type with
    the reference's codecs (src/core/numeric.cpp:28-106 f16, :349-384 q8_0) -- the store
    llama.cpp makes (ggml_set_rows into the cache view) inside every llama_decode the
    reference calls at src/core/core_execution.cpp:2074, :3536 and :3811.  Rows whose cell
    falls outside the cache are skipped.  Asynchronous on the current stream.
    """
    import torch

    lib = load_library()
    p = kv_write_params(src, cache, kv_len, q_len, stream, page_table)
    if p.stream is None:
        p.stream = torch.cuda.current_stream(src.device).cuda_stream
    rc = lib.sixi_kv_write(ctypes.byref(p))
    if check and rc != OK:
        raise SixiAttnError(rc, strerror(rc))
    return rc


def kv_copy(cache, src_stream: int, dst_stream: int, n_cells: int, src_cell: int = 0, dst_cell: int = 0,
            head_dim: Optional[int] = None, stream=None, check=True) -> int:
    """Copies cells [src_cell, src_cell + n_cells) of one stream to another stream's cells --
    the data movement of llama_memory_seq_cp between sequences kept in separate streams
    (src/core/core_execution.cpp:3215-3216, :3245-3246).  ``cache[S, n_cells, Hkv, D]`` f16,
    or uint8 q8_0 blocks with ``head_dim``.  Overlapping ranges raise."""
    import torch

    lib = load_library()
    p = SixiKvCopyParams()
    if cache.dtype == torch.uint8:
        if head_dim is None:
            raise ValueError("a q8_0 cache needs head_dim")
        p.cache = view_of(cache, TYPE_Q8_0, head_dim)
    else:
        p.cache = view_of(cache)
    p.src_stream, p.dst_stream = int(src_stream), int(dst_stream)
    p.src_cell, p.dst_cell, p.n_cells = int(src_cell), int(dst_cell), int(n_cells)
    p.stream = stream if stream is not None else torch.cuda.current_stream(cache.device).cuda_stream
    rc = lib.sixi_kv_copy(ctypes.byref(p))
    if check and rc != OK:
        raise SixiAttnError(rc, strerror(rc))
    return rc


PAGE_CELLS = 256  # SIXI_KV_PAGE_CELLS


class KvPool:
    """A page pool over 256-cell pages (include/sixi_kv.h ``sixi_kv_pool_*``): which pages of
    the K/V page pools (tensors ``[n_pages, 256, Hkv, D]``) hold each stream's cells.

    ``seq_cp`` shares pages (llama_memory_seq_cp, src/core/core_execution.cpp:3215-3216,
    :3245-3246) and ``seq_rm`` releases them (llama_memory_seq_rm, :4021-4062); no cell data
    moves.  ``prepare_write`` gives a stream the pages a write needs, copying a page it shares
    with another stream first (every attached pool tensor, on the current stream)."""

    def __init__(self, n_pages: int, n_streams: int, max_pages: int):
        self.lib = load_library()
        h = ctypes.c_void_p()
        self._check(self.lib.sixi_kv_pool_create(int(n_pages), int(n_streams), int(max_pages), ctypes.byref(h)))
        self.h = h
        self.n_pages, self.n_streams, self.max_pages = int(n_pages), int(n_streams), int(max_pages)
        self._views = []  # attached tensors stay alive with the pool

    @staticmethod
    def _check(rc: int) -> int:
        if rc != OK:
            raise SixiAttnError(rc, strerror(rc))
        return rc

    def close(self) -> None:
        if self.h:
            self.lib.sixi_kv_pool_destroy(self.h)
            self.h = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    def attach(self, pages, head_dim: Optional[int] = None) -> None:
        """Registers a page pool tensor ``[n_pages, 256, Hkv, D]`` f16 (or uint8 q8_0 blocks with
        ``head_dim``) whose pages copy-on-write duplicates."""
        v = _cache_view(pages, head_dim if head_dim is not None else pages.shape[-1])
        self._check(self.lib.sixi_kv_pool_attach(self.h, ctypes.byref(v)))
        self._views.append(pages)

    def prepare_write(self, s: int, first: int, n: int, stream=None) -> None:
        """Pages for stream s's cells [first, first + n), shared pages in that range copied."""
        st = stream
        if st is None and self._views:
            import torch

            st = torch.cuda.current_stream().cuda_stream
        self._check(self.lib.sixi_kv_pool_prepare_write(self.h, int(s), int(first), int(n), st))

    def seq_rm(self, s: int, p0: int) -> None:
        self._check(self.lib.sixi_kv_pool_seq_rm(self.h, int(s), int(p0)))

    def seq_cp(self, src: int, dst: int, n: int = -1) -> None:
        self._check(self.lib.sixi_kv_pool_seq_cp(self.h, int(src), int(dst), int(n)))

    def page_table(self):
        """The page table as a numpy int32 array [n_streams, max_pages] (-1: no page)."""
        import numpy as np

        t = np.empty((self.n_streams, self.max_pages), dtype=np.int32)
        self._check(self.lib.sixi_kv_pool_page_table(self.h, t.ctypes.data))
        return t

    def upload(self, dst=None, stream=None):
        """The page table in an int32 device tensor [n_streams, max_pages] (``dst`` or new)."""
        import torch

        if dst is None:
            dst = torch.empty((self.n_streams, self.max_pages), dtype=torch.int32, device="cuda")
        st = stream if stream is not None else torch.cuda.current_stream(dst.device).cuda_stream
        self._check(self.lib.sixi_kv_pool_upload(self.h, dst.data_ptr(), st))
        return dst

    def free_pages(self) -> int:
        return self._count(self.lib.sixi_kv_pool_free_pages(self.h))

    def stream_pages(self, s: int) -> int:
        return self._count(self.lib.sixi_kv_pool_stream_pages(self.h, int(s)))

    def page_refs(self, page: int) -> int:
        return self._count(self.lib.sixi_kv_pool_page_refs(self.h, int(page)))

    @staticmethod
    def _count(n: int) -> int:
        if n < 0:
            raise SixiAttnError(n, strerror(n))
        return n


def plan_verify(streams, n_ctx_seq: int = 0, pad_mode: int = PAD_REFERENCE):
    """Forms the verify pass(es) of several streams (include/sixi_plan.h): ``streams`` is a list
    of (stream id, cached tokens N, block rows).  Returns (n_parts, slots) with one
    (part, index, row_offset, rows) per input stream.  PAD_REFERENCE reproduces the reference's
    exec_verify_group (src/core/core_execution.cpp:2016-2212); PAD_NONE puts every stream in one
    pass with its own row count."""
    n = len(streams)
    arr = (SixiVerifyStream * max(n, 1))()
    for i, (sid, cached, real) in enumerate(streams):
        arr[i].stream, arr[i].cached, arr[i].real = int(sid), int(cached), int(real)
    out = (SixiVerifySlot * max(n, 1))()
    n_parts = ctypes.c_int32(0)
    rc = load_library().sixi_verify_plan(arr, n, int(n_ctx_seq), int(pad_mode), out, ctypes.byref(n_parts))
    if rc != OK:
        raise SixiAttnError(rc, strerror(rc))
    return n_parts.value, [(out[i].part, out[i].index, out[i].row_offset, out[i].rows) for i in range(n)]


def part_lengths(streams, slots, part: int, pad_mode: int = PAD_REFERENCE):
    """(stream ids, kv_len, q_len) of one part, in the part's stream order: kv_len = cached
    tokens, q_len = padded rows (PAD_REFERENCE: pad rows are computed and stored) or real rows
    (PAD_NONE)."""
    members = sorted((sl[1], i) for i, sl in enumerate(slots) if sl[0] == part)
    ids = [streams[i][0] for _, i in members]
    kv_len = [streams[i][1] for _, i in members]
    q_len = [slots[i][3] if pad_mode == PAD_REFERENCE else streams[i][2] for _, i in members]
    return ids, kv_len, q_len


def qk_prologue_params(qg, k, v, q_norm, k_norm, q_out, k_cache, v_cache, kv_len=None, q_len=None,
                       eps: float = 1e-6, rope_base: float = 1e7, n_rot: int = 64,
                       stream=None, page_table=None) -> SixiQkPrologueParams:
    """Parameters of ``sixi_qk_prologue`` for torch tensors: ``qg[S, n_rows, H, 2D]`` (per head
    the query, then its gate), ``k/v[S, n_rows, Hkv, D]`` f32, ``q_norm/k_norm[D]`` f32,
    ``q_out[S, n_rows, H, D]`` f32 or f16 (the attention's Q), caches ``[S, n_cells, Hkv, D]`` f16 or
    uint8 q8_0 blocks (with ``page_table``, int32 device [S, pages per stream]: page pools
    ``[n_pages, 256, Hkv, D]``)."""
    D = q_out.shape[-1]
    p = SixiQkPrologueParams()
    p.qg = view_of(qg, tokens_heads=False)
    p.k = view_of(k, tokens_heads=False)
    p.v = view_of(v, tokens_heads=False)
    p.q_norm = q_norm.data_ptr()
    p.k_norm = k_norm.data_ptr()
    p.eps = eps
    p.rope_base = rope_base
    p.n_rot = n_rot
    p.flags = 0
    p.kv_len = kv_len.data_ptr() if kv_len is not None else None
    p.q_len = q_len.data_ptr() if q_len is not None else None
    p.q_out = view_of(q_out)
    p.k_cache = _cache_view(k_cache, D)
    p.v_cache = _cache_view(v_cache, D)
    p.stream = stream
    if page_table is not None:
        p.page_table = page_table.data_ptr()
        p.page_table_stride = page_table.stride(0)
    return p


def qk_prologue(qg, k, v, q_norm, k_norm, q_out, k_cache, v_cache, kv_len=None, q_len=None,
                eps: float = 1e-6, rope_base: float = 1e7, n_rot: int = 64, stream=None, check=True,
                page_table=None) -> int:
    """The Q/K prologue of a Qwen3.8 full-attention layer (include/sixi_layer.h) fused with the
    KV store: RMS norm times the attn_q_norm / attn_k_norm weight, NEOX RoPE on the first
    ``n_rot`` dims at position kv_len[s] + j, Q to ``q_out``, K and V into cell kv_len[s] + j of
    the caches (the codecs of :func:`kv_write`).  Defaults are configs/qwen3.8-27b-ud-q4-k-xl.sixi's
    rms_norm_eps, rope_freq_base and rope_dim_count.  Asynchronous on the current stream."""
    import torch

    p = qk_prologue_params(qg, k, v, q_norm, k_norm, q_out, k_cache, v_cache, kv_len, q_len, eps, rope_base,
                           n_rot, stream, page_table)
    if p.stream is None:
        p.stream = torch.cuda.current_stream(q_out.device).cuda_stream
    rc = load_library().sixi_qk_prologue(ctypes.byref(p))
    if check and rc != OK:
        raise SixiAttnError(rc, strerror(rc))
    return rc


def attn_gate(out, qg, q_len=None, stream=None, check=True) -> int:
    """``out[S, n_rows, H, D] *= sigmoid(gate)`` in place, the gate being the second half of
    each head of ``qg[S, n_rows, H, 2D]`` (include/sixi_layer.h)."""
    import torch

    p = SixiAttnGateParams()
    p.out = view_of(out, tokens_heads=False)
    p.qg = view_of(qg, tokens_heads=False)
    p.q_len = q_len.data_ptr() if q_len is not None else None
    p.stream = stream if stream is not None else torch.cuda.current_stream(out.device).cuda_stream
    rc = load_library().sixi_attn_gate(ctypes.byref(p))
    if check and rc != OK:
        raise SixiAttnError(rc, strerror(rc))
    return rc


def _plain_view(t) -> SixiView:
    """ggml view of a torch tensor of up to 4 dims (the reversed shape, missing dims of 1)."""
    import torch

    es = t.element_size()
    ne = list(reversed(t.shape)) + [1] * (4 - t.dim())
    nb = [t.stride(i) * es for i in reversed(range(t.dim()))]
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1] if nb else es)
    return make_view(t.data_ptr(), {torch.float32: TYPE_F32, torch.float16: TYPE_F16}[t.dtype], ne, nb)


def gdn_verify_params(q, k, v, alpha, beta, y, state_in, state_out=None, q_len=None, snap=None,
                      decay_first: bool = False, stream=None) -> SixiGdnParams:
    """Parameters of ``sixi_gdn_verify`` for torch tensors: ``q/k[S, n_rows, G, K]``,
    ``v/y[S, n_rows, G, HD]``, ``alpha/beta[S, n_rows, G]``, ``state[S, G, HD, K]`` f32."""
    p = SixiGdnParams()
    p.q, p.k, p.v, p.y = (_plain_view(t) for t in (q, k, v, y))
    p.alpha, p.beta = _plain_view(alpha), _plain_view(beta)
    p.state_in = _plain_view(state_in)
    p.state_out = _plain_view(state_in if state_out is None else state_out)
    p.q_len = q_len.data_ptr() if q_len is not None else None
    p.snap = snap.data_ptr() if snap is not None else None
    p.flags = GDN_DECAY_FIRST if decay_first else 0
    p.stream = stream
    return p


def gdn_verify(q, k, v, alpha, beta, y, state_in, state_out=None, q_len=None, snap=None,
               decay_first: bool = False, stream=None, check=True) -> int:
    """The gated-delta-rule recurrent verify (include/sixi_gdn.h): rows j < q_len[s] of every
    stream through its state -- the reference's GdnOperator::step_token
    (src/core/core_execution.cpp:254-335) once per row -- writing y and the state after snap[s]
    rows to ``state_out`` (``state_in`` itself when None: in place)."""
    import torch

    p = gdn_verify_params(q, k, v, alpha, beta, y, state_in, state_out, q_len, snap, decay_first, stream)
    if p.stream is None:
        p.stream = torch.cuda.current_stream(q.device).cuda_stream
    rc = load_library().sixi_gdn_verify(ctypes.byref(p))
    if check and rc != OK:
        raise SixiAttnError(rc, strerror(rc))
    return rc
