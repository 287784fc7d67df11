"""The C ABI on any host: the library loads, exports what include/sixi_attn.h declares, and
rejects bad descriptions with the documented status codes before touching a device."""
import ctypes
import pathlib
import re

import pytest

import sixi_attn as sa

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "sixi_attn.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|size_t)\s+(sixi_attn_\w+)\(", text, re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = sa.load_library()
    declared = _declared()
    assert declared == sorted(sa.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.sixi_attn_abi_version() == 1


def test_status_strings():
    for code in (sa.OK, sa.E_INVALID_ARGUMENT, sa.E_OUT_OF_BOUNDS, sa.E_ALIGNMENT, sa.E_UNSUPPORTED,
                 sa.E_BACKEND, sa.E_INTEGER_OVERFLOW):
        assert sa.strerror(code) and sa.strerror(code) != "unknown status"
    assert sa.strerror(12345) == "unknown status"


FAKE = 0x7F0000000000  # aligned host address; validation never dereferences it


def _params(S=2, n_q=16, H=24, Hkv=4, D=128, n_kv=4096, q_type=sa.TYPE_F32, kv_type=sa.TYPE_F16,
            mode=sa.MASK_BLOCK_CAUSAL, kv_len=True):
    p = sa.SixiAttnParams()
    qes = 4 if q_type == sa.TYPE_F32 else 2
    kves = 2
    p.q = sa.make_view(FAKE, q_type, [D, n_q, H, S], [qes, H * D * qes, D * qes, n_q * H * D * qes])
    row = D * kves if kv_type == sa.TYPE_F16 else D // 32 * 34
    nb0 = kves if kv_type == sa.TYPE_F16 else 34
    kv_nb = [nb0, Hkv * row, row, n_kv * Hkv * row]
    p.k = sa.make_view(FAKE, kv_type, [D, n_kv, Hkv, S], kv_nb)
    p.v = sa.make_view(FAKE, kv_type, [D, n_kv, Hkv, S], kv_nb)
    p.out = sa.make_view(FAKE, sa.TYPE_F32, [D, H, n_q, S], [4, D * 4, H * D * 4, n_q * H * D * 4])
    p.kv_len = FAKE if kv_len else None
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


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p, "flags", 1), sa.E_INVALID_ARGUMENT),
    (lambda p: setattr(p.q, "data", None), sa.E_INVALID_ARGUMENT),
    (lambda p: p.q.ne.__setitem__(0, 96), sa.E_INVALID_ARGUMENT),          # q/k head dims differ
    (lambda p: p.q.ne.__setitem__(2, 25), sa.E_INVALID_ARGUMENT),          # H % Hkv != 0
    (lambda p: p.out.ne.__setitem__(2, 15), sa.E_INVALID_ARGUMENT),        # out rows != n_q
    (lambda p: p.k.nb.__setitem__(1, 1032), sa.E_ALIGNMENT),              # cell stride not 16-B
    (lambda p: setattr(p.k, "data", FAKE + 8), sa.E_ALIGNMENT),
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
    p.mask = sa.make_view(FAKE, sa.TYPE_F16, [4096, 16, 1, 2], [2, 8192, 8192 * 16, 8192 * 16])
    assert _validate(p) == sa.OK
    p.mask.ne[1] = 8
    assert _validate(p) == sa.E_INVALID_ARGUMENT  # fewer mask rows than n_q


def test_forward_without_workspace_fails_before_any_launch():
    p = _params()
    p.workspace = None
    p.workspace_bytes = 0
    assert sa.load_library().sixi_attn_forward(ctypes.byref(p)) == sa.E_OUT_OF_BOUNDS
