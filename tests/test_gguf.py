"""CPU checks of the GGUF parser (bread_gguf_*): files written by the
independent writer in tests/gguf_writer.py are parsed back field by field,
compared with the reference's own parser (gguf.c, compiled from the
reference tree into oracle/_ref/libref_gguf.so when that tree is present),
and malformed files must return BREAD_ERR_FORMAT instead of crashing or
exiting (gguf.c exits on them, so only well-formed files go to it)."""
import ctypes
import os
import struct

import numpy as np
import pytest

import breadv2_amd as B
from breadv2_amd import _lib

import gguf_writer as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_GGUF = os.path.join(ROOT, "oracle", "_ref", "libref_gguf.so")

H, I, ISH, E = 256, 256, 512, 8

KVS = [
    ("general.architecture", W.STRING, "qwen3moe"),
    ("general.name", W.STRING, "tiny synthetic"),
    ("qwen3moe.expert_used_count", W.U32, 4),
    ("qwen3moe.attention.layer_norm_rms_epsilon", W.F32, 1e-5),
    ("t.u8", W.U8, 200),
    ("t.i8", W.I8, -100),
    ("t.u16", W.U16, 60000),
    ("t.i16", W.I16, -30000),
    ("t.i32", W.I32, -2_000_000_000),
    ("t.u64", W.U64, 2**63 + 5),
    ("t.i64", W.I64, -(2**62)),
    ("t.f64", W.F64, 3.141592653589793),
    ("t.bool", W.BOOL, True),
    ("t.arr_i32", W.ARRAY, (W.I32, [1, -2, 3])),
    ("t.arr_str", W.ARRAY, (W.STRING, ["a", "bc", ""])),
    ("t.arr_arr", W.ARRAY, (W.ARRAY, [(W.U8, [1, 2]), (W.F32, [0.5])])),
]


def model_file(tmp_path, version=3, alignment=None, name="m.gguf", layers=(0, 1), **kw):
    tensors = [("token_embd.weight", W.GGML_Q8_0, [H, 3], np.arange(3 * 8 * 34, dtype=np.uint8))]
    for l in layers:
        tensors += W.moe_layer_tensors(l, H, I, ISH, E, seed=100 + l, **kw)
    p = str(tmp_path / name)
    meta = W.write_gguf(p, KVS, tensors, version=version, alignment=alignment)
    return p, tensors, meta


@pytest.mark.parametrize("version,alignment", [(3, None), (2, None), (3, 64), (3, 4096)])
def test_parse_round_trip(tmp_path, version, alignment):
    p, tensors, meta = model_file(tmp_path, version, alignment)
    g = B.Gguf(p)
    info = g.info()
    assert info["version"] == version
    assert info["n_tensors"] == len(tensors)
    assert info["n_kv"] == len(KVS) + (alignment is not None)
    assert info["alignment"] == (alignment or 32)
    assert info["data_offset"] == meta["data_offset"]
    assert info["data_offset"] % info["alignment"] == 0
    for i, (name, gtype, dims, data) in enumerate(tensors):
        t = g.tensor(i)
        assert t["name"] == name and t["type"] == gtype and t["dims"] == dims
        off, size = meta["offsets"][name]
        assert t["offset"] == off and t["size"] == size == len(data)
        assert t["n_elems"] == int(np.prod(dims))
        assert ctypes.string_at(t["data"], t["size"]) == bytes(data)
        assert g.find(name)["offset"] == off
    assert g.find("blk.0.no_such.weight") is None
    g.close()


def test_metadata_values(tmp_path):
    p, _, _ = model_file(tmp_path)
    g = B.Gguf(p)
    assert g.kv_str("general.architecture") == "qwen3moe"
    assert g.kv_str("general.name") == "tiny synthetic"
    assert g.kv_int("qwen3moe.expert_used_count") == 4
    assert g.kv_float("qwen3moe.attention.layer_norm_rms_epsilon") == pytest.approx(1e-5, rel=1e-7)
    assert g.kv_int("t.u8") == 200
    assert g.kv_int("t.i8") == -100
    assert g.kv_int("t.u16") == 60000
    assert g.kv_int("t.i16") == -30000
    assert g.kv_int("t.i32") == -2_000_000_000
    assert g.kv_int("t.u64") & (2**64 - 1) == 2**63 + 5
    assert g.kv_int("t.i64") == -(2**62)
    assert g.kv_float("t.f64") == 3.141592653589793
    assert g.kv_int("t.bool") == 1
    # wrong kind or absent: no value
    assert g.kv_int("general.name") is None
    assert g.kv_float("t.i32") is None
    assert g.kv_str("t.arr_str") is None
    assert g.kv_int("absent.key") is None


def test_kv_str_truncates_to_buffer(tmp_path):
    p, _, _ = model_file(tmp_path)
    g = B.Gguf(p)
    buf = ctypes.create_string_buffer(5)
    assert _lib.lib.bread_gguf_kv_str(g._h, b"general.name", buf, 5) == 0
    assert buf.value == b"tiny"


def test_moe_shape_from_tensors_and_metadata(tmp_path):
    p, _, _ = model_file(tmp_path)
    s = B.Gguf(p).moe_shape(1)
    assert (s.hidden, s.expert_inter, s.shared_inter, s.n_experts) == (H, I, ISH, E)
    assert s.top_k == 4
    assert s.rms_eps == pytest.approx(1e-5, rel=1e-7)
    with pytest.raises(B.BreadError):
        B.Gguf(p).moe_shape(2)


def test_moe_shape_defaults_without_metadata(tmp_path):
    p = str(tmp_path / "nometa.gguf")
    W.write_gguf(p, [], W.moe_layer_tensors(0, H, I, ISH, E, seed=5))
    s = B.Gguf(p).moe_shape(0)
    d = _lib.default_shape()
    assert (s.top_k, s.rms_eps) == (d.top_k, d.rms_eps)


def test_type_sizes():
    ts = _lib.lib.bread_ggml_type_size
    # block sizes of the GGUF block layouts
    assert ts(0, 10) == 40 and ts(1, 10) == 20 and ts(30, 10) == 20
    assert ts(8, 64) == 68  # Q8_0: 32 elements in 34 bytes
    assert ts(12, 512) == 288  # Q4_K: 256 in 144
    assert ts(14, 512) == 420  # Q6_K: 256 in 210
    assert ts(22, 256) == 82  # IQ2_S: d + qs[64] + qh[8] + scales[8]
    assert ts(12, 100) == 0  # not a whole number of blocks
    assert ts(99, 256) == 0  # unknown type


# ---- the reference's parser -------------------------------------------------


class RefTensor(ctypes.Structure):
    # gguf.h:82-90
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("size", ctypes.c_uint64),
                ("n_elems", ctypes.c_uint64)]


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_GGUF):
        pytest.skip("oracle/_ref/libref_gguf.so not built (reference tree absent)")
    r = ctypes.CDLL(REF_GGUF)
    r.gguf_open.restype = ctypes.c_void_p
    r.gguf_open.argtypes = [ctypes.c_char_p]
    r.gguf_close.argtypes = [ctypes.c_void_p]
    r.gguf_version.restype = ctypes.c_uint32
    r.gguf_version.argtypes = [ctypes.c_void_p]
    r.gguf_num_tensors.restype = ctypes.c_uint64
    r.gguf_num_tensors.argtypes = [ctypes.c_void_p]
    r.gguf_data_offset.restype = ctypes.c_uint64
    r.gguf_data_offset.argtypes = [ctypes.c_void_p]
    r.gguf_tensor_by_idx.restype = ctypes.POINTER(RefTensor)
    r.gguf_tensor_by_idx.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    r.gguf_find_tensor.restype = ctypes.POINTER(RefTensor)
    r.gguf_find_tensor.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
    r.ggml_tensor_nbytes.restype = ctypes.c_uint64
    r.ggml_tensor_nbytes.argtypes = [ctypes.c_uint64, ctypes.c_uint32]
    return r


@pytest.mark.parametrize("version,alignment", [(3, None), (2, None), (3, 128)])
def test_matches_reference_parser(tmp_path, ref, version, alignment):
    p, tensors, _ = model_file(tmp_path, version, alignment)
    rc = ref.gguf_open(p.encode())
    assert rc
    try:
        g = B.Gguf(p)
        info = g.info()
        assert info["version"] == ref.gguf_version(rc)
        assert info["n_tensors"] == ref.gguf_num_tensors(rc)
        assert info["data_offset"] == ref.gguf_data_offset(rc)
        for i in range(info["n_tensors"]):
            a = g.tensor(i)
            b = ref.gguf_tensor_by_idx(rc, i).contents
            assert a["name"] == b.name.decode()
            assert (a["type"], len(a["dims"])) == (b.type, b.n_dims)
            assert a["dims"] == list(b.dims[: b.n_dims])
            assert (a["offset"], a["size"], a["n_elems"]) == (b.offset, b.size, b.n_elems)
            f = ref.gguf_find_tensor(rc, b.name).contents
            assert f.offset == b.offset
    finally:
        ref.gguf_close(rc)


def test_type_sizes_match_reference(ref):
    for t in [0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 23, 24, 25, 26, 27, 28, 29,
              30]:
        for n in (256, 4096, 256 * 257):
            assert _lib.lib.bread_ggml_type_size(t, n) == ref.ggml_tensor_nbytes(n, t), t
    # IQ2_S: ggml's block_iq2_s is 2 + 64 + 8 + 8 = 82 bytes per 256; the
    # reference's table says 84 (gguf.c:92), a deliberate difference
    assert _lib.lib.bread_ggml_type_size(22, 256) == 82 and ref.ggml_tensor_nbytes(256, 22) == 84


# ---- malformed files ----------------------------------------------------------


def _open_status(path):
    h = ctypes.c_void_p()
    return _lib.lib.bread_gguf_open(path.encode(), ctypes.byref(h)), h


def _patched(tmp_path, blob, name):
    p = str(tmp_path / name)
    with open(p, "wb") as f:
        f.write(blob)
    return p


def test_malformed_files_are_rejected(tmp_path):
    good, _, _ = model_file(tmp_path, layers=(0,))
    blob = open(good, "rb").read()
    head = 24
    cases = {
        "magic": b"GGUX" + blob[4:],
        "version1": blob[:4] + struct.pack("<I", 1) + blob[8:],
        "version4": blob[:4] + struct.pack("<I", 4) + blob[8:],
        "short_header": blob[:20],
        "truncated_meta": blob[:200],
        "huge_n_kv": blob[:16] + struct.pack("<Q", 2**60) + blob[head:],
        "huge_n_tensors": blob[:8] + struct.pack("<Q", 2**60) + blob[16:],
        "no_data": blob[: len(blob) - 1000],
        "empty": b"",
    }
    # a key whose length runs past the end of the file
    cases["key_len"] = blob[:head] + struct.pack("<Q", 2**40) + blob[head + 8:]
    for name, b in cases.items():
        rc, h = _open_status(_patched(tmp_path, b, name + ".gguf"))
        assert rc == _lib.ERR_FORMAT, (name, rc)
        assert not h.value


def test_malformed_tensor_records(tmp_path):
    def one(dims, gtype=W.GGML_F32, n_dims=None, offset=None):
        p = str(tmp_path / "t.gguf")
        W.write_gguf(p, [], [("x", gtype, dims, np.zeros(4 * 16, np.uint8))])
        blob = bytearray(open(p, "rb").read())
        rec = 24 + 8 + 1  # header, name length, name
        if n_dims is not None:
            blob[rec:rec + 4] = struct.pack("<I", n_dims)
        if offset is not None:
            at = rec + 4 + 8 * len(dims) + 4
            blob[at:at + 8] = struct.pack("<Q", offset)
        open(p, "wb").write(bytes(blob))
        return _open_status(p)[0]

    assert one([16]) == 0
    assert one([16], n_dims=5) == _lib.ERR_FORMAT
    assert one([16], offset=2**62) == _lib.ERR_FORMAT  # data beyond the file
    assert one([2**40, 2**40]) == _lib.ERR_FORMAT  # 2^80 elements: data beyond the file
    assert one([2**32, 2**32, 2**32]) == _lib.ERR_FORMAT  # element count overflows u64


def test_missing_file_and_bad_args(tmp_path):
    rc, h = _open_status(str(tmp_path / "absent.gguf"))
    assert rc == _lib.ERR_ARG and not h.value
    with pytest.raises(B.BreadError):
        B.Gguf(str(tmp_path / "absent.gguf"))
    p, _, _ = model_file(tmp_path, layers=(0,))
    g = B.Gguf(p)
    t = _lib.GgufTensor()
    assert _lib.lib.bread_gguf_tensor(g._h, 10**6, ctypes.byref(t)) == _lib.ERR_ARG
