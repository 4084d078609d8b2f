"""ctypes wrapper of oracle/liboracle.so — the CPU restatement of the
reference's MoE path.  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product package.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_uint8, c_uint16, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# BREAD_ORACLE_LIB: another build of the oracle (the sanitizer build of tests/sanitize.sh)
LIB_PATH = os.environ.get("BREAD_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_dequant.so")

QTYPE_F32, QTYPE_F16, QTYPE_Q8_0, QTYPE_Q4_K, QTYPE_Q6_K = 0, 1, 8, 12, 14


class OShape(ctypes.Structure):
    _fields_ = [("hidden", c_int), ("expert_inter", c_int), ("shared_inter", c_int),
                ("n_experts", c_int), ("top_k", c_int)]


class OLayer(ctypes.Structure):
    _fields_ = [
        ("gate_exps", c_void_p), ("up_exps", c_void_p), ("down_exps", c_void_p),
        ("gate_expert_bytes", c_uint64), ("up_expert_bytes", c_uint64), ("down_expert_bytes", c_uint64),
        ("gate_type", c_int), ("up_type", c_int), ("down_type", c_int),
        ("gate_shexp", c_void_p), ("up_shexp", c_void_p), ("down_shexp", c_void_p),
        ("gate_shexp_type", c_int), ("up_shexp_type", c_int), ("down_shexp_type", c_int),
        ("router", c_void_p), ("shexp_gate", c_void_p),
    ]


_lib = ctypes.CDLL(LIB_PATH)
_lib.oracle_h2f.restype = c_float
_lib.oracle_h2f.argtypes = [c_uint16]
_lib.oracle_f2h.restype = c_uint16
_lib.oracle_f2h.argtypes = [c_float]
_lib.oracle_get_scale_min_k4.argtypes = [c_int, c_void_p, POINTER(c_uint8), POINTER(c_uint8)]
for _n in ("oracle_dequant_q4k_block", "oracle_dequant_q6k_block", "oracle_dequant_q8_0_block"):
    getattr(_lib, _n).argtypes = [c_void_p, c_void_p]
_lib.oracle_row_bytes.restype = c_uint64
_lib.oracle_row_bytes.argtypes = [c_int, c_int]
_lib.oracle_dequant_rows.argtypes = [c_void_p, c_int, c_int, c_int, c_void_p]
_lib.oracle_matvec.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_int, c_int]
_lib.oracle_matvec_mt.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int]
_lib.oracle_matvec_f16io.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_int, c_int]
_lib.oracle_rms_norm_weighted.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_float]
_lib.oracle_swiglu.argtypes = [c_void_p, c_void_p, c_void_p, c_int]
_lib.oracle_softmax.argtypes = [c_void_p, c_int]
_lib.oracle_topk.argtypes = [c_void_p, c_int, c_int, c_void_p, c_void_p]
_lib.oracle_sigmoid.restype = c_float
_lib.oracle_sigmoid.argtypes = [c_float]
_lib.oracle_route.restype = c_float
_lib.oracle_route.argtypes = [POINTER(OShape), POINTER(OLayer), c_void_p, c_void_p, c_void_p, c_void_p]
_lib.oracle_route_batch.argtypes = [POINTER(OShape), POINTER(OLayer), c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_int]
_lib.oracle_expf.restype = c_float
_lib.oracle_expf.argtypes = [c_float]
_lib.oracle_expf_array.argtypes = [c_void_p, c_void_p, c_uint64]
_lib.oracle_moe_token.argtypes = [POINTER(OShape), POINTER(OLayer), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
_lib.oracle_moe_token_mt.argtypes = [POINTER(OShape), POINTER(OLayer), c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_int]
_lib.oracle_moe_forward.argtypes = [POINTER(OShape), POINTER(OLayer), c_void_p, c_void_p, c_int, c_void_p,
                                    c_void_p, c_void_p, c_int]
_lib.oracle_greedy_f16.restype = c_int
_lib.oracle_greedy_f16.argtypes = [c_void_p, c_int]
_lib.oracle_spec_round.restype = c_int
_lib.oracle_spec_round.argtypes = [c_void_p, c_void_p, c_int, ctypes.c_int32, c_int, c_int, c_void_p, c_void_p]
_lib.oracle_online_cores.restype = c_int
_lib.oracle_affinity_cores.restype = c_int


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return c_void_p(a.ctypes.data)


def h2f(h: int) -> float:
    return _lib.oracle_h2f(h)


def f2h(f: float) -> int:
    return _lib.oracle_f2h(f)


def get_scale_min_k4(j: int, scales: np.ndarray):
    d, m = c_uint8(), c_uint8()
    _lib.oracle_get_scale_min_k4(j, _ptr(scales), ctypes.byref(d), ctypes.byref(m))
    return d.value, m.value


def dequant_block(qtype: int, block: np.ndarray) -> np.ndarray:
    n = 32 if qtype == QTYPE_Q8_0 else 256
    out = np.empty(n, np.float32)
    fn = {QTYPE_Q4_K: _lib.oracle_dequant_q4k_block, QTYPE_Q6_K: _lib.oracle_dequant_q6k_block,
          QTYPE_Q8_0: _lib.oracle_dequant_q8_0_block}[qtype]
    fn(_ptr(np.ascontiguousarray(block, np.uint8)), _ptr(out))
    return out


def row_bytes(qtype: int, cols: int) -> int:
    return int(_lib.oracle_row_bytes(qtype, cols))


def dequant_rows(w: np.ndarray, qtype: int, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows * cols, np.float32)
    assert _lib.oracle_dequant_rows(_ptr(w), qtype, rows, cols, _ptr(out)) == 0
    return out.reshape(rows, cols)


def matvec(w: np.ndarray, qtype: int, x: np.ndarray, rows: int, cols: int, nthreads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    if nthreads > 1:
        rc = _lib.oracle_matvec_mt(_ptr(w), qtype, _ptr(x), _ptr(y), rows, cols, nthreads)
    else:
        rc = _lib.oracle_matvec(_ptr(w), qtype, _ptr(x), _ptr(y), rows, cols)
    assert rc == 0
    return y


def matvec_f16io(w: np.ndarray, qtype: int, x16: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x16 = np.ascontiguousarray(x16, np.uint16)
    y = np.empty(rows, np.uint16)
    assert _lib.oracle_matvec_f16io(_ptr(w), qtype, _ptr(x16), _ptr(y), rows, cols) == 0
    return y


def rms_norm_weighted(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _lib.oracle_rms_norm_weighted(_ptr(x), _ptr(np.ascontiguousarray(w, np.float32)), _ptr(out), x.size, eps)
    return out


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    out = np.empty(g.size, np.float32)
    _lib.oracle_swiglu(_ptr(np.ascontiguousarray(g, np.float32)), _ptr(np.ascontiguousarray(u, np.float32)),
                       _ptr(out), g.size)
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    _lib.oracle_softmax(_ptr(y), y.size)
    return y


def topk(p: np.ndarray, k: int):
    p = np.ascontiguousarray(p, np.float32)
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    _lib.oracle_topk(_ptr(p), p.size, k, _ptr(idx), _ptr(w))
    return idx, w


def sigmoid(x: float) -> float:
    return _lib.oracle_sigmoid(x)


class HostLayer:
    """A layer's weights on the host (numpy), native GGUF layout."""

    def __init__(self, shape: OShape, gate_exps, up_exps, down_exps, gate_sh, up_sh, down_sh, router, shgate,
                 types=(QTYPE_Q4_K, QTYPE_Q4_K, QTYPE_Q6_K, QTYPE_Q4_K, QTYPE_Q4_K, QTYPE_Q6_K)):
        """types: gate, up, down, gate_shexp, up_shexp, down_shexp (each Q4_K
        or Q6_K), as the reference records per tensor (loader.c:191-193)."""
        self.shape = shape
        self.types = tuple(int(t) for t in types)
        self.arrays = [np.ascontiguousarray(a) for a in (gate_exps, up_exps, down_exps, gate_sh, up_sh, down_sh)]
        self.router = np.ascontiguousarray(router, np.float32)
        self.shgate = None if shgate is None else np.ascontiguousarray(shgate, np.uint16)
        H, I = shape.hidden, shape.expert_inter
        tg, tu, td, tgs, tus, tds = self.types
        g, u, d, gs, us, ds = self.arrays
        self.desc = OLayer(g.ctypes.data, u.ctypes.data, d.ctypes.data,
                           I * row_bytes(tg, H), I * row_bytes(tu, H), H * row_bytes(td, I),
                           tg, tu, td,
                           gs.ctypes.data, us.ctypes.data, ds.ctypes.data,
                           tgs, tus, tds,
                           self.router.ctypes.data, None if self.shgate is None else self.shgate.ctypes.data)


def route(layer: HostLayer, x: np.ndarray, want_logits: bool = False):
    K, E = layer.shape.top_k, layer.shape.n_experts
    idx = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    logits = np.empty(E, np.float32) if want_logits else None
    g = _lib.oracle_route(ctypes.byref(layer.shape), ctypes.byref(layer.desc),
                          _ptr(np.ascontiguousarray(x, np.float32)), _ptr(idx), _ptr(w), _ptr(logits))
    return (idx, w, g, logits) if want_logits else (idx, w, g)


def route_batch(layer: HostLayer, x: np.ndarray, nthreads: int = 16, want_logits: bool = False):
    """oracle_route for every row of x [T][H]: (idx [T][K], w [T][K], gsh [T]
    [, logits [T][E]])."""
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    K, E = layer.shape.top_k, layer.shape.n_experts
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    g = np.empty(T, np.float32)
    lg = np.empty((T, E), np.float32) if want_logits else None
    _lib.oracle_route_batch(ctypes.byref(layer.shape), ctypes.byref(layer.desc), _ptr(x), T, _ptr(idx), _ptr(w),
                            _ptr(g), _ptr(lg), nthreads)
    return (idx, w, g, lg) if want_logits else (idx, w, g)


def expf(x: np.ndarray) -> np.ndarray:
    """The C library's expf (the one cpu_softmax calls), elementwise."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _lib.oracle_expf_array(_ptr(x), _ptr(out), x.size)
    return out


def expert_block(layer: HostLayer, x: np.ndarray, hidden: np.ndarray, idx: np.ndarray, w: np.ndarray,
                 nthreads: int = 1) -> None:
    """hidden[t] += sum_k w[t][k] * expert_{idx[t][k]}(x[t]) in rank order, the
    routed experts alone with given routing: the CPU side of the reference's
    expert benchmark (expert_bench.cu:127-144: gate/up matvecs, SwiGLU, down,
    scaled by the weight and summed in k order) and the routed loop of
    one_layer.cu:1455-1470.  Each term is rounded before it is added."""
    s = layer.shape
    H, I = s.hidden, s.expert_inter
    tg, tu, td = layer.types[:3]
    g, u, d = layer.arrays[:3]
    gb, ub, db = I * row_bytes(tg, H), I * row_bytes(tu, H), H * row_bytes(td, I)
    for t in range(x.shape[0]):
        xt = np.ascontiguousarray(x[t], np.float32)
        for k in range(idx.shape[1]):
            e = int(idx[t, k])
            eg = matvec(g[e * gb:(e + 1) * gb], tg, xt, I, H, nthreads)
            eu = matvec(u[e * ub:(e + 1) * ub], tu, xt, I, H, nthreads)
            eo = matvec(d[e * db:(e + 1) * db], td, swiglu(eg, eu), H, I, nthreads)
            hidden[t] += np.float32(w[t, k]) * eo


def moe_forward(layer: HostLayer, x: np.ndarray, hidden: np.ndarray, n_tokens: int, nthreads: int = 1):
    """hidden (float32 [T][H]) is updated in place; returns (idx, w, gsh)."""
    K = layer.shape.top_k
    x = np.ascontiguousarray(x, np.float32)
    assert hidden.dtype == np.float32 and hidden.flags["C_CONTIGUOUS"]
    idx = np.empty((n_tokens, K), np.int32)
    w = np.empty((n_tokens, K), np.float32)
    g = np.empty(n_tokens, np.float32)
    _lib.oracle_moe_forward(ctypes.byref(layer.shape), ctypes.byref(layer.desc), _ptr(x), _ptr(hidden), n_tokens,
                            _ptr(idx), _ptr(w), _ptr(g), nthreads)
    return idx, w, g


def moe_token_mt(layer: HostLayer, x: np.ndarray, hidden: np.ndarray, nthreads: int):
    K = layer.shape.top_k
    idx = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    g = np.empty(1, np.float32)
    _lib.oracle_moe_token_mt(ctypes.byref(layer.shape), ctypes.byref(layer.desc),
                             _ptr(np.ascontiguousarray(x, np.float32)), _ptr(hidden), _ptr(idx), _ptr(w), _ptr(g),
                             nthreads)
    return idx, w, g[0]


def moe_token(layer: HostLayer, x: np.ndarray, hidden: np.ndarray):
    K = layer.shape.top_k
    idx = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    g = np.empty(1, np.float32)
    _lib.oracle_moe_token(ctypes.byref(layer.shape), ctypes.byref(layer.desc),
                          _ptr(np.ascontiguousarray(x, np.float32)), _ptr(hidden), _ptr(idx), _ptr(w), _ptr(g))
    return idx, w, g[0]


def online_cores() -> int:
    return int(_lib.oracle_online_cores())


def affinity_cores() -> int:
    return int(_lib.oracle_affinity_cores())


def ref_dequant_lib():
    """The reference's own dequant_q4k_cpu.c compiled into oracle/_ref, or None."""
    if not os.path.exists(REF_PATH):
        return None
    lib = ctypes.CDLL(REF_PATH)
    lib.dequant_q4k_block_cpu.argtypes = [c_void_p, c_void_p]
    lib.dequant_q6k_block_cpu.argtypes = [c_void_p, c_void_p]
    return lib


def greedy_f16(logits16: np.ndarray) -> int:
    """greedy_sample (main.cu:326-335) over one row of fp16 logits."""
    a = np.ascontiguousarray(logits16, np.float16)
    return int(_lib.oracle_greedy_f16(_ptr(a.view(np.uint16)), a.size))


def spec_round(pred, draft, eos: int, total_gen: int, max_tokens: int):
    """One verification round (main_speculative.cu:474-510): returns
    (n_accept, next confirmed token, total_gen after the round)."""
    p = np.ascontiguousarray(pred, np.int32)
    d = np.ascontiguousarray(draft if len(draft) else [0], np.int32)
    nx = np.zeros(1, np.int32)
    g = np.zeros(1, np.int32)
    a = _lib.oracle_spec_round(_ptr(p), _ptr(d), len(draft), eos, total_gen, max_tokens, _ptr(nx), _ptr(g))
    return int(a), int(nx[0]), int(g[0])
