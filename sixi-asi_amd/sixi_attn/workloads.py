"""Seeded synthetic workloads of the attention path and their algorithmic cost.

Shapes follow the engine's attention geometry: 24 query heads sharing 4 KV heads (GQA 6:1,
the Qwen3.8 layout of configs/qwen3.8-27b-ud-q4-k-xl.sixi with head_dim 128 here), per-stream
KV caches of uniform capacity in 256-cell pages (include/sixi_asi/manifest.hpp:124-127),
stream-major verify blocks with positions N_s + j (src/core/core_execution.cpp:2047-2062)
and 2048-row prefill chunks (apps/sixi_server_main.cpp:95).

Inputs come from libsixi_synth.so: PCG32 seeded ``0x51A70000 + config``, Box-Muller normals
in float64, f16 by round-to-nearest-even, q8_0 by the codec of src/core/numeric.cpp:349-384.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os
from typing import List, Optional

import numpy as np

from . import LIB_DIR, MASK_BLOCK_CAUSAL, TYPE_F16, TYPE_F32, TYPE_Q8_0

SEED_BASE = 0x51A70000
PAGE = 256
TENSOR_Q, TENSOR_K, TENSOR_V = 1, 2, 3

_synth = None


def synth_lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        path = LIB_DIR / "libsixi_synth.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run `python sixi-asi_amd/build.py`")
        lib = ctypes.CDLL(str(path))
        vp, i64, u64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int32
        lib.sixi_synth_normal_f32.argtypes = [u64, u64, ctypes.c_float, vp, i64]
        lib.sixi_synth_f32_to_f16.argtypes = [vp, vp, i64]
        lib.sixi_synth_f16_to_f32.argtypes = [vp, vp, i64]
        lib.sixi_synth_quantize_q8_0.argtypes = [vp, vp, i64]
        lib.sixi_synth_quantize_q8_0.restype = ctypes.c_int
        lib.sixi_synth_lengths.argtypes = [u64, i64, i32, i32, vp]
        lib.sixi_synth_q.argtypes = [u64, i32, ctypes.c_float, vp, i64, i64, i64, i64, ctypes.c_int]
        lib.sixi_synth_q.restype = ctypes.c_int
        lib.sixi_synth_kv.argtypes = [u64, u64, i32, ctypes.c_float, vp, i64, i64, i64, vp, i64, i64, i64,
                                      ctypes.c_int]
        lib.sixi_synth_kv.restype = ctypes.c_int
        _synth = lib
    return _synth


def _threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def normal_f32(seed: int, seq: int, n: int, mul: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    synth_lib().sixi_synth_normal_f32(seed, seq, mul, out.ctypes.data, n)
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    if synth_lib().sixi_synth_quantize_q8_0(x.ctypes.data, out.ctypes.data, x.size) != 0:
        raise ValueError("q8_0 needs a multiple of 32 elements")
    return out


@dataclasses.dataclass
class Workload:
    """One attention call: S streams, per-stream cached length and block rows."""

    name: str
    seed: int
    S: int
    kv_len: List[int]          # cached cells before the block, per stream
    q_len: List[int]           # block rows per stream
    H: int = 24
    Hkv: int = 4
    D: int = 128
    kv_type: int = TYPE_F16
    q_type: int = TYPE_F32
    mask_mode: int = MASK_BLOCK_CAUSAL
    mul: float = 1.0           # value scale of Q, K and V
    q_row0: int = 0            # first row of the Q draw (prefill chunks share one draw)
    q_rows_total: Optional[int] = None
    cache_cells: Optional[int] = None  # cells generated per stream (defaults to kv_len + q_len)

    @property
    def n_q(self) -> int:
        return max(self.q_len)

    def cells(self) -> List[int]:
        if self.cache_cells is not None:
            return [self.cache_cells] * self.S
        return [l + q for l, q in zip(self.kv_len, self.q_len)]

    @property
    def capacity(self) -> int:
        need = max(max(self.cells()), max(l + q for l, q in zip(self.kv_len, self.q_len)))
        return (need + PAGE - 1) // PAGE * PAGE

    @property
    def row_bytes(self) -> int:
        return self.D // 32 * 34 if self.kv_type == TYPE_Q8_0 else self.D * 2

    # ---- cost model (algorithmic, counted once per call) ----
    def attended_cells(self) -> int:
        return sum(l + q for l, q in zip(self.kv_len, self.q_len))

    def bytes(self) -> int:
        kv = 2 * self.Hkv * self.row_bytes * self.attended_cells()
        q_es = 4 if self.q_type == TYPE_F32 else 2
        rows = sum(self.q_len) * self.H * self.D
        return kv + rows * q_es + rows * 4

    def flops(self) -> int:
        vis = 0
        for l, q in zip(self.kv_len, self.q_len):
            if self.mask_mode == MASK_BLOCK_CAUSAL:
                vis += q * l + q * (q + 1) // 2
            else:
                vis += q * (l + q)
        return 4 * self.D * self.H * vis


def kq_mask(n_kv: int, n_q_pad: int, kv_len, q_len, causal: bool = True) -> np.ndarray:
    """The llama-style f16 KQ mask of a stream-major block, [S, 1, n_q_pad, n_kv] as f16 bits
    (uint16): row j of stream s sees cell i when j < q_len[s], i < kv_len[s] + q_len[s] and
    (causal) i <= kv_len[s] + j -- positions N_s + j, one sequence per stream
    (src/core/core_execution.cpp:2047-2062) -- 0 there and -inf elsewhere."""
    kl = np.asarray(kv_len, dtype=np.int64)[:, None, None]
    ql = np.asarray(q_len, dtype=np.int64)[:, None, None]
    if np.any(kl + ql > n_kv) or np.any(ql > n_q_pad) or np.any(kl < 0) or np.any(ql < 0):
        raise ValueError("stream cells exceed the mask")
    j = np.arange(n_q_pad, dtype=np.int64)[None, :, None]
    i = np.arange(n_kv, dtype=np.int64)[None, None, :]
    vis = (j < ql) & (i < kl + ql)
    if causal:
        vis &= i <= kl + j
    return np.where(vis, np.uint16(0), np.uint16(0xFC00)).astype(np.uint16)[:, None]


def config(name: str) -> Workload:
    """The five configurations of the attention path (decode, verify, batched verify,
    chunked prefill, long q8_0 decode/verify)."""
    if name == "decode":
        return Workload("decode", SEED_BASE + 1, 1, [4095], [1])
    if name == "verify":
        return Workload("verify", SEED_BASE + 2, 1, [8192], [16])
    if name == "batched_verify":
        S = 32
        lens = np.empty(S, dtype=np.int32)
        synth_lib().sixi_synth_lengths(SEED_BASE + 3, S, 512, 15873, lens.ctypes.data)
        return Workload("batched_verify", SEED_BASE + 3, S, [int(x) for x in lens], [16] * S)
    if name in ("prefill_chunk0", "prefill_chunk1"):
        c = int(name[-1])
        return Workload(name, SEED_BASE + 4, 1, [2048 + 2048 * c], [2048], q_type=TYPE_F16, mul=0.5,
                        q_row0=2048 * c, q_rows_total=4096, cache_cells=6144)
    if name in ("long_q8_decode", "long_q8_verify"):
        ql = 1 if name.endswith("decode") else 8
        return Workload(name, SEED_BASE + 5, 8, [65536] * 8, [ql] * 8, kv_type=TYPE_Q8_0)
    if name in ("decode_d256", "batched_verify_d256"):
        # the real model's 256-dim heads (configs/qwen3.8-27b-ud-q4-k-xl.sixi: key/value length 256)
        w = config(name[:-5])
        return dataclasses.replace(w, name=name, seed=SEED_BASE + 6, D=256)
    raise KeyError(name)


CONFIGS = ("decode", "verify", "batched_verify", "prefill_chunk0", "prefill_chunk1",
           "long_q8_decode", "long_q8_verify")


def make_host(w: Workload, poison: bool = False) -> dict:
    """Host arrays: q [S, n_q, H, D], k/v [S, cap, Hkv, D] (f16 bits as uint16, or uint8 q8_0
    rows), kv_len/q_len int32.  Cells past a stream's generated cells hold NaN f16 (or NaN
    q8_0 scales) when ``poison`` is set, zeros otherwise."""
    lib = synth_lib()
    nt = _threads()
    n_q = w.n_q
    rows_total = w.q_rows_total or n_q
    q_es_type = 0 if w.q_type == TYPE_F32 else 1
    qd = np.empty((w.S, rows_total, w.H, w.D), dtype=np.float32 if q_es_type == 0 else np.float16)
    lib.sixi_synth_q(w.seed, q_es_type, w.mul, qd.ctypes.data, w.S, rows_total, w.H, w.D, nt)
    q = np.ascontiguousarray(qd[:, w.q_row0:w.q_row0 + n_q])

    cap = w.capacity
    cells = np.array(w.cells(), dtype=np.int32)
    if w.kv_type == TYPE_Q8_0:
        shape, dt = (w.S, cap, w.Hkv, w.row_bytes), np.uint8
    else:
        shape, dt = (w.S, cap, w.Hkv, w.D), np.uint16
    out = {}
    for name, tid in (("k", TENSOR_K), ("v", TENSOR_V)):
        arr = np.zeros(shape, dtype=dt)
        if poison:
            if w.kv_type == TYPE_Q8_0:
                arr.reshape(-1, 34)[:, 0:2] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)
            else:
                arr.fill(0x7E00)
        es = arr.itemsize
        nb1, nb2, nb3 = arr.strides[1], arr.strides[2], arr.strides[0]
        rc = lib.sixi_synth_kv(w.seed, tid, w.kv_type, w.mul, arr.ctypes.data, w.S, w.Hkv, w.D,
                               cells.ctypes.data, nb1, nb2, nb3, nt)
        assert rc == 0 and es in (1, 2)
        out[name] = arr
    out["q"] = q
    out["kv_len"] = np.array(w.kv_len, dtype=np.int32)
    out["q_len"] = np.array(w.q_len, dtype=np.int32)
    return out


def to_device(host: dict, device="cuda"):
    import torch

    dev = {}
    for key, arr in host.items():
        t = torch.from_numpy(arr)
        if arr.dtype == np.uint16:
            t = t.view(torch.float16)
        dev[key] = t.to(device)
    return dev
