"""CPU-side checks of the C ABI: the library loads, exports every entry point
include/bread_moe.h declares, and rejects bad arguments on the host (no
device call is made: argument checks run before any HIP call)."""
import ctypes
import os
import re

import pytest

import breadv2_amd as B
from breadv2_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bread_moe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bread_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ["bread_matvec", "bread_matvec_f32", "bread_dequant_rows", "bread_route", "bread_route_layer",
              "bread_moe_forward", "bread_moe_ctx_create", "bread_arena_create"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_status_strings():
    for code in range(-9, 1):
        assert B.status_str(code) and B.status_str(code) != "unknown status"
    assert B.status_str(-99) == "unknown status"


def test_default_shape_matches_reference_constants():
    s = _lib.default_shape()
    # bread.h:16-69
    assert (s.hidden, s.expert_inter, s.shared_inter, s.n_experts, s.top_k) == (2048, 512, 512, 256, 8)
    assert abs(s.rms_eps - 1e-6) < 1e-12


FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: every call below fails its host-side check


@pytest.mark.parametrize(
    "args,status",
    [
        ((None, FAKE, FAKE, 8, 256, 12), _lib.ERR_ARG),
        ((FAKE, FAKE, FAKE, -1, 256, 12), _lib.ERR_ARG),
        ((FAKE, FAKE, FAKE, 8, 256, 3), _lib.ERR_QTYPE),
        ((FAKE, FAKE, FAKE, 8, 300, 12), _lib.ERR_SHAPE),
        ((FAKE, FAKE, FAKE, 8, 48, 8), _lib.ERR_SHAPE),
        ((ctypes.c_void_p(0x10002), FAKE, FAKE, 8, 256, 14), _lib.ERR_ALIGN),
        ((FAKE, ctypes.c_void_p(0x10004), FAKE, 8, 256, 12), _lib.ERR_ALIGN),
    ],
)
def test_matvec_rejects_bad_arguments(args, status):
    assert _lib.lib.bread_matvec(*args, None) == status
    assert _lib.lib.bread_matvec_f32(*args, None) == status


def test_dequant_rejects_bad_arguments():
    assert _lib.lib.bread_dequant_rows(None, 12, 1, 256, FAKE, None) == _lib.ERR_ARG
    assert _lib.lib.bread_dequant_rows(FAKE, 13, 1, 256, FAKE, None) == _lib.ERR_QTYPE
    assert _lib.lib.bread_dequant_rows(FAKE, 14, 1, 100, FAKE, None) == _lib.ERR_SHAPE


def test_ctx_create_rejects_bad_shapes():
    out = ctypes.c_void_p()
    for fields in [(2048, 512, 512, 256, 300, 1e-6), (2000, 512, 512, 256, 8, 1e-6), (2048, 500, 512, 256, 8, 1e-6),
                   (2048, 512, 512, 0, 8, 1e-6)]:
        s = _lib.MoeShape(*fields)
        rc = _lib.lib.bread_moe_ctx_create(ctypes.byref(s), 1, ctypes.byref(out))
        assert rc in (_lib.ERR_ARG, _lib.ERR_SHAPE)
    s = _lib.default_shape()
    assert _lib.lib.bread_moe_ctx_create(ctypes.byref(s), 0, ctypes.byref(out)) == _lib.ERR_ARG


def test_moe_calls_reject_null_context():
    layer = _lib.MoeLayer()
    assert _lib.lib.bread_moe_forward(None, ctypes.byref(layer), FAKE, FAKE, 1, None, None, None, None) == _lib.ERR_ARG
    assert _lib.lib.bread_route(None, ctypes.byref(layer), FAKE, 1, FAKE, FAKE, FAKE, None) == _lib.ERR_ARG
    assert _lib.lib.bread_moe_ctx_check(None, None) == _lib.ERR_ARG
    assert _lib.lib.bread_moe_ctx_set_spin_limit(None, 0) == _lib.ERR_ARG
    assert _lib.lib.bread_arena_layer(None, 0, ctypes.byref(layer)) == _lib.ERR_ARG


def test_route_noalloc_rejects_beyond_workspace_on_host():
    """n_tokens * n_experts above the 1048576-float workspace is refused
    before any device call (and NULL outputs before that)."""
    from breadv2_amd import api
    s = api.shape()
    layer = _lib.MoeLayer()
    T = (1 << 20) // s.n_experts + 1
    st = _lib.lib.bread_route_noalloc(ctypes.byref(s), ctypes.byref(layer), FAKE, T, FAKE, FAKE, FAKE, None)
    assert st == _lib.ERR_CAPACITY
    st = _lib.lib.bread_route_noalloc(ctypes.byref(s), ctypes.byref(layer), FAKE, 4, None, FAKE, FAKE, None)
    assert st == _lib.ERR_ARG
