"""ctypes binding of the CPU oracle (liboracle.so) -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module; the
product path never does.  See fa_oracle.h for what each function restates (reference
file:line) and how it is pinned.  ``ref_numeric()`` loads the reference's own codec source
(src/core/numeric.cpp) compiled into _ref/ by this directory's Makefile, when present.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess
from typing import Optional, Sequence

import numpy as np

ORACLE_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"
REF_PATH = ORACLE_DIR / "_ref" / "libref_numeric.so"

F32, F16, Q8_0 = 0, 1, 8


class View(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_int64 * 4),
    ]


class Pcg32(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64), ("inc", ctypes.c_uint64)]


_lib = None
_ref = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "liboracle.so"], check=True)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, i64, u64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64
        VP = ctypes.POINTER(View)
        lib.oracle_set_simd.argtypes = [ctypes.c_int]
        lib.oracle_set_simd.restype = ctypes.c_int
        lib.oracle_have_simd.restype = ctypes.c_int
        lib.oracle_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        lib.oracle_fp16_to_fp32.restype = ctypes.c_float
        lib.oracle_fp32_to_fp16.argtypes = [ctypes.c_float]
        lib.oracle_fp32_to_fp16.restype = ctypes.c_uint16
        lib.oracle_fp32_to_fp16_row.argtypes = [vp, vp, i64]
        lib.oracle_fp16_to_fp32_row.argtypes = [vp, vp, i64]
        lib.oracle_quantize_row_q8_0.argtypes = [vp, vp, i64]
        lib.oracle_quantize_row_q8_0.restype = ctypes.c_int
        lib.oracle_dequantize_row_q8_0.argtypes = [vp, vp, i64]
        lib.oracle_vec_dot_f16.argtypes = [i64, vp, vp]
        lib.oracle_vec_dot_f16.restype = ctypes.c_float
        lib.oracle_vec_dot_q8_0.argtypes = [i64, vp, vp]
        lib.oracle_vec_dot_q8_0.restype = ctypes.c_float
        lib.oracle_flash_attn_ext.argtypes = [VP, VP, VP, VP, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                              vp, ctypes.c_int, ctypes.c_int]
        lib.oracle_flash_attn_ext.restype = ctypes.c_int
        lib.oracle_build_kq_mask.argtypes = [vp, i64, i64, i64, vp, vp, ctypes.c_int]
        lib.oracle_build_kq_mask.restype = ctypes.c_int
        lib.oracle_pcg32_seed.argtypes = [ctypes.POINTER(Pcg32), u64, u64]
        lib.oracle_pcg32_next.argtypes = [ctypes.POINTER(Pcg32)]
        lib.oracle_pcg32_next.restype = ctypes.c_uint32
        lib.oracle_pcg32_uniform01.argtypes = [ctypes.POINTER(Pcg32)]
        lib.oracle_pcg32_uniform01.restype = ctypes.c_double
        lib.oracle_fill_normal_f32.argtypes = [u64, u64, ctypes.c_float, vp, i64]
        lib.oracle_gdn_verify.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, ctypes.c_int]
        lib.oracle_gdn_verify.restype = None
        _lib = lib
    return _lib


def ref_numeric() -> Optional[ctypes.CDLL]:
    """The reference's own fp16/q8_0 codecs (oracle/_ref), or None when not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        lib = ctypes.CDLL(str(REF_PATH))
        lib.ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        lib.ref_fp16_to_fp32.restype = ctypes.c_float
        lib.ref_fp32_to_fp16.argtypes = [ctypes.c_float]
        lib.ref_fp32_to_fp16.restype = ctypes.c_uint16
        lib.ref_fp32_to_fp16_row.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.ref_quantize_row_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.ref_quantize_row_q8_0.restype = ctypes.c_int
        lib.ref_q8_0_block_bytes.restype = ctypes.c_int
        lib.ref_diff_metrics.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.ref_diff_metrics.restype = ctypes.c_int
        _ref = lib
    return _ref


# ---------------------------------------------------------------------------------------
def fp32_to_fp16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().oracle_fp32_to_fp16_row(x.ctypes.data, out.ctypes.data, x.size)
    return out


def fp16_bits_to_fp32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    load().oracle_fp16_to_fp32_row(h.ctypes.data, out.ctypes.data, h.size)
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    if load().oracle_quantize_row_q8_0(x.ctypes.data, out.ctypes.data, x.size) != 0:
        raise ValueError("q8_0 needs a multiple of 32 elements")
    return out


def dequantize_q8_0(b: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    load().oracle_dequantize_row_q8_0(b.ctypes.data, out.ctypes.data, n)
    return out


def kv_write(src: np.ndarray, cache: np.ndarray, kv_len: Optional[Sequence[int]] = None,
             q_len: Optional[Sequence[int]] = None) -> np.ndarray:
    """CPU restatement of the KV-cache store (include/sixi_kv.h, sixi_kv_write): row
    j < q_len[s] of stream s goes to cell kv_len[s] + j of every kv-head, converted with the
    reference's codecs (src/core/numeric.cpp:28-106 f16, :349-384 q8_0 -- this module's
    fp32_to_fp16_bits / quantize_q8_0, pinned against the compiled reference source);
    rows whose cell lies outside the cache are skipped.  ``src[S, n_rows, Hkv, D]`` float32
    or float16; ``cache[S, n_cells, Hkv, D]`` uint16 f16 bits, or uint8 q8_0 blocks
    ``[S, n_cells, Hkv, D/32*34]``.  Returns the updated copy of ``cache``."""
    out = cache.copy()
    S, n_rows, Hkv, D = src.shape
    n_cells = cache.shape[1]
    q8 = cache.dtype == np.uint8
    for s in range(S):
        ql = n_rows if q_len is None else int(q_len[s])
        base = 0 if kv_len is None else int(kv_len[s])
        for j in range(min(ql, n_rows)):
            cell = base + j
            if cell < 0 or cell >= n_cells:
                continue
            x = src[s, j].astype(np.float32)
            for h in range(Hkv):
                out[s, cell, h] = quantize_q8_0(x[h]) if q8 else fp32_to_fp16_bits(x[h])
    return out


# ---------------------------------------------------------------------------------------
# Layer prologue / epilogue around the attention (include/sixi_layer.h).  Upstream llama.cpp
# (pinned at a691b234 by scripts/build_llamacpp.sh:12, not in the reference tree) builds these
# ops for the qwen35 layers of configs/qwen3.8-27b-ud-q4-k-xl.sixi; restated from ggml's CPU
# ops (ggml_compute_forward_rms_norm_f32, ggml_rope_cache_init + the NEOX rotation,
# ggml_vec_sigmoid_f32).  Pins: tests/test_oracle_layer.py (closed forms and invariants).

_libm = None


def rope_theta_scale(rope_base: float, n_rot: int) -> np.float32:
    """ggml's theta_scale = powf(freq_base, -2.0f/n_dims) in f32, through the C library's powf
    (the same function the host side of libsixi_attn.so calls)."""
    global _libm
    if _libm is None:
        import ctypes.util

        _libm = ctypes.CDLL(ctypes.util.find_library("m"))
        _libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
        _libm.powf.restype = ctypes.c_float
    if n_rot == 0:
        return np.float32(1.0)
    e = np.float32(-2.0) / np.float32(n_rot)
    return np.float32(_libm.powf(float(np.float32(rope_base)), float(e)))


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """ggml_rms_norm then ggml_mul by the weight, over the last axis: squares in f32 summed in
    double, mean = f32(sum / D), scale = 1/sqrtf(mean + eps), y = (x * scale) * w."""
    x = np.asarray(x, dtype=np.float32)
    ss = (x * x).astype(np.float64).sum(axis=-1, keepdims=True)
    mean = (ss / x.shape[-1]).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(mean + np.float32(eps))
    return (x * scale) * np.asarray(w, dtype=np.float32)


def rope_neox(x: np.ndarray, pos: np.ndarray, n_rot: int, theta_scale) -> np.ndarray:
    """NEOX RoPE of ``x[S, n_rows, heads, D]`` at positions ``pos[S, n_rows]``: pair
    (i, i + n_rot/2), angle t_i with t_0 = f32(pos), t_{i+1} = t_i * theta_scale in f32 (ggml's
    rope cache), cos/sin of the f32 angle rounded to f32; dims >= n_rot unchanged."""
    x = np.asarray(x, dtype=np.float32)
    out = x.copy()
    if n_rot == 0:
        return out
    half = n_rot // 2
    ts = np.float32(theta_scale)
    t = np.asarray(pos).astype(np.float32)
    theta = np.empty(t.shape + (half,), dtype=np.float32)
    for i in range(half):
        theta[..., i] = t
        t = (t * ts).astype(np.float32)
    c = np.cos(theta.astype(np.float64)).astype(np.float32)[..., None, :]
    sn = np.sin(theta.astype(np.float64)).astype(np.float32)[..., None, :]
    x0, x1 = x[..., :half], x[..., half:n_rot]
    out[..., :half] = x0 * c - x1 * sn
    out[..., half:n_rot] = x0 * sn + x1 * c
    return out


def qk_prologue(qg: np.ndarray, k: np.ndarray, v: np.ndarray, q_norm: np.ndarray, k_norm: np.ndarray,
                k_cache: np.ndarray, v_cache: np.ndarray, kv_len: Optional[Sequence[int]] = None,
                q_len: Optional[Sequence[int]] = None, eps: float = 1e-6, rope_base: float = 1e7,
                n_rot: int = 64):
    """CPU restatement of sixi_qk_prologue: ``qg[S, n_rows, H, 2D]`` (query then gate per head),
    ``k/v[S, n_rows, Hkv, D]``.  Returns (q_out[S, n_rows, H, D] with NaN in rows >= q_len,
    k_rot[S, n_rows, Hkv, D] (K before the store), k_cache', v_cache')."""
    S, n_rows, H, D2 = qg.shape
    D = D2 // 2
    kl = np.zeros(S, dtype=np.int64) if kv_len is None else np.asarray(kv_len, dtype=np.int64)
    pos = kl[:, None] + np.arange(n_rows, dtype=np.int64)[None, :]
    ts = rope_theta_scale(rope_base, n_rot)
    q = rope_neox(rms_norm(qg[..., :D], q_norm, eps), pos, n_rot, ts)
    kr = rope_neox(rms_norm(k, k_norm, eps), pos, n_rot, ts)
    if q_len is not None:
        for s in range(S):
            q[s, int(q_len[s]):] = np.nan
    kc = kv_write(kr, k_cache, kl, q_len)
    vc = kv_write(np.asarray(v, dtype=np.float32), v_cache, kl, q_len)
    return q, kr, kc, vc


def attn_gate(out: np.ndarray, qg: np.ndarray, q_len: Optional[Sequence[int]] = None) -> np.ndarray:
    """out * sigmoid(gate) with ggml's sigmoid 1/(1 + expf(-g)) in f32; ``out[S, n_rows, H, D]``,
    the gate is ``qg[..., D:]``; rows >= q_len keep their value."""
    out = np.asarray(out, dtype=np.float32)
    D = out.shape[-1]
    g = np.asarray(qg[..., D:], dtype=np.float32)
    with np.errstate(over="ignore"):  # e^-g beyond f32 range is inf, and the sigmoid 0
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
    sig = np.float32(1.0) / (np.float32(1.0) + e)
    res = out * sig
    if q_len is not None:
        for s in range(out.shape[0]):
            res[s, int(q_len[s]):] = out[s, int(q_len[s]):]
    return res


def gdn_verify(q: np.ndarray, k: np.ndarray, v: np.ndarray, alpha: np.ndarray, beta: np.ndarray,
               state: np.ndarray, q_len: Optional[Sequence[int]] = None, snap: Optional[Sequence[int]] = None,
               decay_first: bool = False):
    """The reference's gated-delta-rule step (GdnOperator::step_token,
    src/core/core_execution.cpp:254-335) over every row of every stream (fa_oracle.c).
    ``q/k[S, n_rows, G, K]``, ``v[S, n_rows, G, HD]``, ``alpha/beta[S, n_rows, G]``,
    ``state[S, G, HD, K]``.  Returns (y[S, n_rows, G, HD] with NaN past q_len, the state after
    snap[s] rows)."""
    q, k, v, alpha, beta = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v, alpha, beta))
    S, n_rows, G, K = q.shape
    HD = v.shape[-1]
    st = np.ascontiguousarray(state, dtype=np.float32).copy()
    y = np.full((S, n_rows, G, HD), np.nan, dtype=np.float32)
    ql = None if q_len is None else np.ascontiguousarray(q_len, dtype=np.int32)
    sn = None if snap is None else np.ascontiguousarray(snap, dtype=np.int32)
    load().oracle_gdn_verify(q.ctypes.data, k.ctypes.data, v.ctypes.data, alpha.ctypes.data, beta.ctypes.data,
                             st.ctypes.data, y.ctypes.data, S, n_rows, G, K, HD,
                             ql.ctypes.data if ql is not None else None, sn.ctypes.data if sn is not None else None,
                             1 if decay_first else 0)
    return y, st


def fill_normal(seed: int, seq: int, n: int, mul: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().oracle_fill_normal_f32(seed, seq, mul, out.ctypes.data, n)
    return out


def pcg32_u32(seed: int, seq: int, n: int) -> list:
    lib = load()
    r = Pcg32()
    lib.oracle_pcg32_seed(ctypes.byref(r), seed, seq)
    return [lib.oracle_pcg32_next(ctypes.byref(r)) for _ in range(n)]


def view(arr: np.ndarray, type_id: int, head_dim: Optional[int] = None, tokens_heads: bool = True) -> View:
    """ggml view of a 4-d numpy array whose last axis is innermost.

    tokens_heads=True: arr is (S, tokens, heads, D) and the view is ggml's [D, tokens, heads, S]
    (how llama.cpp permutes Q/K/V); False: the plain reversal (out [D, H, n_q, S], mask)."""
    assert arr.ndim == 4
    v = View()
    v.data = arr.ctypes.data
    v.type = type_id
    order = (3, 1, 2, 0) if tokens_heads else (3, 2, 1, 0)
    ne = [arr.shape[i] for i in order]
    nb = [arr.strides[i] for i in order]
    if type_id == Q8_0:
        ne[0] = head_dim
        nb[0] = 34
    for i in range(4):
        v.ne[i] = ne[i]
        v.nb[i] = nb[i]
    return v


def build_kq_mask(n_kv: int, n_q_pad: int, kv_len: Sequence[int], q_len: Sequence[int],
                  causal: bool = True) -> np.ndarray:
    """llama-style f16 mask [S, 1, n_q_pad, n_kv] (f16 bits as uint16)."""
    S = len(kv_len)
    kl = np.ascontiguousarray(kv_len, dtype=np.int32)
    ql = np.ascontiguousarray(q_len, dtype=np.int32)
    m = np.empty((S, 1, n_q_pad, n_kv), dtype=np.uint16)
    if load().oracle_build_kq_mask(m.ctypes.data, n_kv, n_q_pad, S, kl.ctypes.data, ql.ctypes.data,
                                   1 if causal else 0) != 0:
        raise ValueError("stream cells exceed n_kv")
    return m


def flash_attn_ext(q: np.ndarray, k: np.ndarray, v: np.ndarray, kv_type: int = F16,
                   mask: Optional[np.ndarray] = None, scale: Optional[float] = None,
                   max_bias: float = 0.0, logit_softcap: float = 0.0, v_acc_f16: bool = False,
                   n_threads: int = 0) -> np.ndarray:
    """out[S, n_q, H, D] = ggml CPU flash_attn_ext(q[S,n_q,H,D] f32, k/v[S,n_kv,Hkv,D|D/32*34])."""
    q = np.asarray(q, dtype=np.float32)
    S, n_q, H, D = q.shape
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.empty((S, n_q, H, D), dtype=np.float32)
    qv = view(q, F32)
    kv_ = view(k, kv_type, D)
    vv = view(v, kv_type, D)
    mv = view(mask, F16, tokens_heads=False) if mask is not None else None
    rc = load().oracle_flash_attn_ext(ctypes.byref(qv), ctypes.byref(kv_), ctypes.byref(vv),
                                      ctypes.byref(mv) if mv is not None else None,
                                      float(scale), float(max_bias), float(logit_softcap),
                                      out.ctypes.data, 1 if v_acc_f16 else 0, int(n_threads))
    if rc != 0:
        raise ValueError(f"oracle_flash_attn_ext rejected the description ({rc})")
    return out


def attention_for_workload(host: dict, kv_type: int, streams: Optional[Sequence[int]] = None,
                           causal: bool = True, v_acc_f16: bool = False, n_threads: int = 0,
                           scale: Optional[float] = None) -> np.ndarray:
    """Oracle output for (a subset of) the streams of a synthetic workload."""
    idx = list(range(host["q"].shape[0])) if streams is None else list(streams)
    q = host["q"][idx]
    if q.dtype == np.float16:
        q = q.astype(np.float32)
    kl = host["kv_len"][idx]
    ql = host["q_len"][idx]
    n_kv = int((kl + ql).max())
    k = np.ascontiguousarray(host["k"][idx][:, :n_kv])
    v = np.ascontiguousarray(host["v"][idx][:, :n_kv])
    mask = build_kq_mask(n_kv, q.shape[1], kl, ql, causal)
    return flash_attn_ext(np.ascontiguousarray(q), k, v, kv_type, mask, scale=scale,
                          v_acc_f16=v_acc_f16, n_threads=n_threads)


def diff_metrics(ref: np.ndarray, out: np.ndarray) -> dict:
    """The reference's compute_diff_metrics (src/core/numeric.cpp:701-791) in float64, plus
    rel-L2 = ||out - ref|| / ||ref||: max-abs, mean-abs and RMSE of |out - ref|; cosine (1 when
    both norms are 0, 0 when one is); the top-1 indices (first maximum) and whether they match;
    KL(softmax(ref) || softmax(out)) over the flat arrays, log-partition functions taken from the
    maxima, terms with p_ref = 0 skipped, clamped at 0.  Like the reference, non-finite values
    are an error (ValueError)."""
    r = np.asarray(ref, dtype=np.float32).astype(np.float64).ravel()
    o = np.asarray(out, dtype=np.float32).astype(np.float64).ravel()
    if r.size != o.size:
        raise ValueError("reference and candidate differ in size")
    if r.size == 0:
        return {"max_abs": 0.0, "mean_abs": 0.0, "rmse": 0.0, "rel_l2": 0.0, "cosine": 1.0, "kl": 0.0,
                "top1_match": True, "ref_top1": -1, "test_top1": -1}
    if not (np.all(np.isfinite(r)) and np.all(np.isfinite(o))):
        raise ValueError("NaN or Inf encountered in diff_metrics")
    d = np.abs(r - o)
    nr2, no2 = float(np.dot(r, r)), float(np.dot(o, o))
    if nr2 > 0.0 and no2 > 0.0:
        cos = float(np.dot(r, o)) / (np.sqrt(nr2) * np.sqrt(no2))
    else:
        cos = 1.0 if nr2 == 0.0 and no2 == 0.0 else 0.0
    log_z_r = r.max() + np.log(np.sum(np.exp(r - r.max())))
    log_z_o = o.max() + np.log(np.sum(np.exp(o - o.max())))
    lp_r, lp_o = r - log_z_r, o - log_z_o
    p_r = np.exp(lp_r)
    pos = p_r > 0.0
    kl = float(np.sum(p_r[pos] * (lp_r[pos] - lp_o[pos])))
    i_r, i_o = int(np.argmax(r)), int(np.argmax(o))
    return {
        "max_abs": float(d.max()),
        "mean_abs": float(d.sum() / d.size),
        "rmse": float(np.sqrt(np.dot(d, d) / d.size)),
        "rel_l2": float(np.sqrt(np.dot(d, d)) / np.sqrt(nr2)) if nr2 > 0 else float(np.sqrt(np.dot(d, d))),
        "cosine": cos,
        "kl": max(0.0, kl),
        "top1_match": i_r == i_o,
        "ref_top1": i_r,
        "test_top1": i_o,
    }


def ref_diff_metrics(ref: np.ndarray, out: np.ndarray) -> Optional[dict]:
    """compute_diff_metrics of the reference itself (oracle/_ref), or None when not built.
    Raises ValueError with the reference's error code on a rejected input."""
    lib = ref_numeric()
    if lib is None:
        return None
    r = np.ascontiguousarray(ref, dtype=np.float32).ravel()
    o = np.ascontiguousarray(out, dtype=np.float32).ravel()
    res = np.zeros(8, dtype=np.float64)
    rc = lib.ref_diff_metrics(r.ctypes.data, o.ctypes.data, r.size, res.ctypes.data)
    if rc != 0:
        raise ValueError(f"compute_diff_metrics rejected the input (ErrorCode {rc})")
    return {"max_abs": res[0], "mean_abs": res[1], "rmse": res[2], "cosine": res[3], "kl": res[4],
            "top1_match": bool(res[5]), "ref_top1": int(res[6]), "test_top1": int(res[7])}


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
