"""CPU-side checks of the C ABI: the library loads, exports every entry point
include/bread_moe.h declares, and rejects bad arguments on the host (no
device call is made: argument checks run before any HIP call)."""
import ctypes
import os
import re
import subprocess

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


def _cpp_type_checks() -> str:
    """A C++ translation unit of static_asserts that every declaration in
    include/bread_moe.h has the arity, return type and argument types the
    ctypes binding (_lib.SIGNATURES) passes: a prototype that drifts from
    the binding (an argument added, dropped, reordered or retyped) stops it
    compiling.  An untyped ctypes pointer (c_void_p) only requires a
    pointer."""
    scalar = {ctypes.c_int: "int", ctypes.c_int32: "int32_t", ctypes.c_float: "float", ctypes.c_double: "double",
              ctypes.c_uint16: "uint16_t", ctypes.c_uint32: "uint32_t"}
    # 64-bit integers by size and sign: ctypes aliases c_int64 / c_longlong
    # and c_uint64 / c_size_t, and C spells them long or long long
    wide = {ctypes.c_longlong: "signed", ctypes.c_int64: "signed", ctypes.c_uint64: "unsigned",
            ctypes.c_size_t: "unsigned"}
    structs = {_lib.MoeShape: "bread_moe_shape_t", _lib.MoeLayer: "bread_moe_layer_t",
               _lib.GgufTensor: "bread_gguf_tensor_t"}

    def check(t, expr, what):
        if t is None:
            return [f'static_assert(std::is_void<{expr}>::value, "{what}: void");']
        if t is ctypes.c_void_p:
            return [f'static_assert(std::is_pointer<{expr}>::value, "{what}: a pointer");']
        if t is ctypes.c_char_p:
            return [f'static_assert(std::is_same<{expr}, const char *>::value || std::is_same<{expr}, char *>::value, '
                    f'"{what}: char pointer");']
        if t in scalar:
            return [f'static_assert(std::is_same<{expr}, {scalar[t]}>::value, "{what}: {scalar[t]}");']
        if t in wide:
            return [f'static_assert(std::is_integral<{expr}>::value && sizeof({expr}) == 8 && '
                    f'std::is_{wide[t]}<{expr}>::value, "{what}: {wide[t]} 64-bit integer");']
        if hasattr(t, "_type_"):  # POINTER(x)
            inner = t._type_
            base = f"std::remove_cv_t<std::remove_pointer_t<{expr}>>"
            out = [f'static_assert(std::is_pointer<{expr}>::value, "{what}: a pointer");']
            if inner is ctypes.c_void_p:
                out.append(f'static_assert(std::is_pointer<{base}>::value, "{what}: pointer to a pointer");')
            elif inner in structs:
                out.append(f'static_assert(std::is_same<{base}, {structs[inner]}>::value, "{what}: {structs[inner]}");')
            elif inner in scalar:
                out.append(f'static_assert(std::is_same<{base}, {scalar[inner]}>::value, "{what}: {scalar[inner]} *");')
            elif inner in wide:
                out.append(f'static_assert(std::is_integral<{base}>::value && sizeof({base}) == 8 && '
                           f'std::is_{wide[inner]}<{base}>::value, "{what}: {wide[inner]} 64-bit integer *");')
            return out
        raise AssertionError(f"no C type for {t} ({what})")

    lines = ["#include <stddef.h>", "#include <stdint.h>", "#include <tuple>", "#include <type_traits>",
             '#include "bread_moe.h"',
             "template <typename F> struct fn;",
             "template <typename R, typename... A> struct fn<R(A...)> {",
             "    using ret = R; using args = std::tuple<A...>; static constexpr size_t n = sizeof...(A);",
             "};",
             "template <size_t I, typename F> using arg_t = std::tuple_element_t<I, typename fn<F>::args>;"]
    for name, (res, args) in sorted(_lib.SIGNATURES.items()):
        f = f"decltype({name})"
        lines.append(f'static_assert(fn<{f}>::n == {len(args)}, "{name}: {len(args)} arguments");')
        lines += check(res, f"fn<{f}>::ret", f"{name} returns")
        for i, a in enumerate(args):
            lines += check(a, f"arg_t<{i}, {f}>", f"{name} argument {i}")
    return "\n".join(lines) + "\n"


def test_header_prototypes_match_the_binding(tmp_path):
    src = tmp_path / "types.cpp"
    src.write_text(_cpp_type_checks())
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]


def test_type_check_catches_a_drifted_prototype(tmp_path):
    """The same check against a copy of the header with two int arguments of
    bread_matvec swapped for a size_t: it must fail."""
    text = open(HEADER).read()
    old = "int bread_matvec(const void *w, const uint16_t *x, uint16_t *y, int rows, int cols,"
    assert old in text
    (tmp_path / "bread_moe.h").write_text(text.replace(old, old.replace("int rows", "size_t rows")))
    src = tmp_path / "types.cpp"
    src.write_text(_cpp_type_checks())
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", str(tmp_path), str(src)],
                       capture_output=True, text=True)
    assert r.returncode != 0 and "bread_matvec argument 3" in r.stderr


def test_header_compiles_as_c99_and_cpp():
    for cmd in (["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-x", "c"],
                ["g++", "-std=c++11", "-Wall", "-Wextra", "-Werror", "-x", "c++"]):
        r = subprocess.run(cmd + ["-fsyntax-only", "-I", os.path.join(ROOT, "include"), HEADER],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-1000:]


def test_reference_cpp_prototype_links(tmp_path):
    """tests/abi_caller.cpp declares bread_matvec exactly as the reference's
    translation units do (one_layer.cu:46-47, with HIP's spelling of half and
    cudaStream_t) and calls the C entry points; it compiles and links
    against the library, which exports that C++ overload beside the C one."""
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "tests"), "-B"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    assert os.access(os.path.join(ROOT, "tests", "_build", "abi_caller"), os.X_OK)
    nm = subprocess.run(["nm", "-DC", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split(" ", 2)[2] for line in nm.splitlines() if " T " in line}
    assert "bread_matvec(void*, __half*, __half*, int, int, int, ihipStream_t*)" in exported
    assert "bread_matvec" in exported


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
    assert _lib.lib.bread_moe_ctx_route_stats(None, None, 0, 0) == _lib.ERR_ARG
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
