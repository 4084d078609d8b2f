"""ctypes binding of libbread_moe.so (the C ABI declared in include/bread_moe.h).

The library is the product: every compute call goes to the HIP kernels in it.
There is no CPU fallback; if the shared object is missing, importing this
module raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_longlong, c_uint16, c_uint64, c_void_p

# PyTorch ships its own libamdhip64/libhsa-runtime64 (same soname as the
# system ROCm).  Loading torch first makes libbread_moe bind to that one
# runtime; loading it second would bring a second HIP/HSA runtime into the
# process, and the one that initialises last finds no device.
try:
    import torch  # noqa: F401
except ImportError:  # plain C/ctypes users without torch: the system runtime is the only one
    pass

HERE = os.path.dirname(os.path.abspath(__file__))
# BREAD_MOE_LIB: another build of the library (the sanitizer build of tests/sanitize.sh)
LIB_PATH = os.environ.get("BREAD_MOE_LIB") or os.path.join(HERE, "libbread_moe.so")

QTYPE_F32 = 0
QTYPE_F16 = 1
QTYPE_Q8_0 = 8
QTYPE_Q4_K = 12
QTYPE_Q6_K = 14

# bread_moe_path_t
PATH_AUTO = 0
PATH_DECODE = 1
PATH_GROUPED = 2
PATH_PER_TOKEN = 3
PATH_SMALL = 4

QK_K = 256
Q4K_BLOCK_BYTES = 144
Q6K_BLOCK_BYTES = 210
Q8_0_BLOCK_ELEMS = 32
Q8_0_BLOCK_BYTES = 34

OK = 0
ERR_ARG = -1
ERR_QTYPE = -2
ERR_SHAPE = -3
ERR_ALIGN = -4
ERR_HIP = -5
ERR_NOMEM = -6
ERR_CAPACITY = -7
ERR_DEVICE = -8
ERR_FORMAT = -9


class BreadError(RuntimeError):
    def __init__(self, status: int, where: str, device_error: int = 0):
        self.status = status
        self.device_error = device_error  # bread_moe_ctx_check's error word
        detail = lib.bread_last_error().decode(errors="replace")
        super().__init__(f"{where}: {status_str(status)} ({status}): {detail}")


class MoeShape(ctypes.Structure):
    _fields_ = [
        ("hidden", c_int),
        ("expert_inter", c_int),
        ("shared_inter", c_int),
        ("n_experts", c_int),
        ("top_k", c_int),
        ("rms_eps", c_float),
    ]


class MoeLayer(ctypes.Structure):
    _fields_ = [
        ("gate_exps", c_void_p),
        ("up_exps", c_void_p),
        ("down_exps", c_void_p),
        ("gate_expert_bytes", c_uint64),
        ("up_expert_bytes", c_uint64),
        ("down_expert_bytes", c_uint64),
        ("gate_type", c_int),
        ("up_type", c_int),
        ("down_type", c_int),
        ("gate_shexp", c_void_p),
        ("up_shexp", c_void_p),
        ("down_shexp", c_void_p),
        ("gate_shexp_type", c_int),
        ("up_shexp_type", c_int),
        ("down_shexp_type", c_int),
        ("router", c_void_p),
        ("shexp_gate", c_void_p),
        ("post_norm_w", c_void_p),
    ]


class GgufTensor(ctypes.Structure):
    _fields_ = [
        ("name", c_char_p),
        ("type", ctypes.c_uint32),
        ("n_dims", ctypes.c_uint32),
        ("dims", c_uint64 * 4),
        ("offset", c_uint64),
        ("size", c_uint64),
        ("n_elems", c_uint64),
        ("data", c_void_p),
    ]


# name -> (restype, argtypes); mirrors include/bread_moe.h one to one.
SIGNATURES = {
    "bread_status_str": (c_char_p, [c_int]),
    "bread_last_error": (c_char_p, []),
    "bread_set_exit_on_error": (None, [c_int]),
    "bread_matvec": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "bread_matvec_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "bread_dequant_rows": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "bread_moe_shape_default": (None, [POINTER(MoeShape)]),
    "bread_moe_ctx_create": (c_int, [POINTER(MoeShape), c_int, POINTER(c_void_p)]),
    "bread_moe_ctx_destroy": (c_int, [c_void_p]),
    "bread_moe_ctx_check": (c_int, [c_void_p, POINTER(c_int)]),
    "bread_moe_expert_block": (c_int, [c_void_p, POINTER(MoeLayer), c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                       c_void_p]),
    "bread_route": (c_int, [c_void_p, POINTER(MoeLayer), c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "bread_route_noalloc": (
        c_int,
        [POINTER(MoeShape), POINTER(MoeLayer), c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "bread_route_layer": (
        c_int,
        [c_void_p, POINTER(MoeLayer), c_void_p, POINTER(c_int32), POINTER(c_float), POINTER(c_float), c_void_p],
    ),
    "bread_route_layer_f16": (
        c_int,
        [c_void_p, POINTER(MoeLayer), c_void_p, POINTER(c_int32), POINTER(c_float), POINTER(c_float), c_void_p],
    ),
    "bread_moe_forward": (
        c_int,
        [c_void_p, POINTER(MoeLayer), c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "bread_moe_forward_f16": (
        c_int,
        [c_void_p, POINTER(MoeLayer), c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "bread_moe_stack_forward": (
        c_int,
        [c_void_p, POINTER(MoeLayer), c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "bread_moe_greedy_head": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p],
    ),
    "bread_argmax_f16": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "bread_spec_accept": (
        c_int,
        [POINTER(c_int32), POINTER(c_int32), c_int, c_int32, c_int, POINTER(c_int), POINTER(c_int32)],
    ),
    "bread_moe_decode_layers": (
        c_int, [c_void_p, POINTER(MoeLayer), c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "bread_moe_ctx_set_trace": (c_int, [c_void_p, c_void_p, ctypes.c_size_t, POINTER(c_int)]),
    "bread_moe_ctx_set_path": (c_int, [c_void_p, c_int]),
    "bread_moe_ctx_set_spin_limit": (c_int, [c_void_p, c_longlong]),
    "bread_moe_ctx_route_stats": (c_int, [c_void_p, POINTER(c_uint64), c_int, c_int]),
    "bread_small_auto_tokens": (c_int, []),
    "bread_stack_loop_tokens": (c_int, []),
    "bread_rmsnorm_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "bread_arena_create": (c_int, [POINTER(MoeShape), c_int, POINTER(c_void_p)]),
    "bread_arena_destroy": (c_int, [c_void_p]),
    "bread_arena_layer": (c_int, [c_void_p, c_int, POINTER(MoeLayer)]),
    "bread_arena_layer_bytes": (c_uint64, [c_void_p]),
    "bread_synth_q4k": (c_int, [c_void_p, c_uint64, c_uint64, c_void_p]),
    "bread_synth_q6k": (c_int, [c_void_p, c_uint64, c_uint64, c_void_p]),
    "bread_synth_normal_f32": (c_int, [c_void_p, c_uint64, c_uint64, c_float, c_float, c_void_p]),
    "bread_synth_normal_f16": (c_int, [c_void_p, c_uint64, c_uint64, c_float, c_float, c_void_p]),
    "bread_gguf_open": (c_int, [c_char_p, POINTER(c_void_p)]),
    "bread_gguf_close": (c_int, [c_void_p]),
    "bread_gguf_info": (c_int, [c_void_p, POINTER(ctypes.c_uint32), POINTER(c_uint64), POINTER(c_uint64),
                                POINTER(c_uint64), POINTER(ctypes.c_uint32)]),
    "bread_gguf_tensor": (c_int, [c_void_p, c_uint64, POINTER(GgufTensor)]),
    "bread_gguf_find": (c_int, [c_void_p, c_char_p, POINTER(GgufTensor)]),
    "bread_gguf_kv_int": (c_int, [c_void_p, c_char_p, POINTER(ctypes.c_int64)]),
    "bread_gguf_kv_float": (c_int, [c_void_p, c_char_p, POINTER(ctypes.c_double)]),
    "bread_gguf_kv_str": (c_int, [c_void_p, c_char_p, c_char_p, ctypes.c_size_t]),
    "bread_ggml_type_size": (c_uint64, [ctypes.c_uint32, c_uint64]),
    "bread_gguf_moe_shape": (c_int, [c_void_p, c_int, POINTER(MoeShape)]),
    "bread_arena_load_gguf": (c_int, [c_void_p, c_int, c_void_p, c_int]),
    "bread_arena_set_layer_types": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()'). "
            "There is no CPU fallback for the MoE path."
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def status_str(status: int) -> str:
    return lib.bread_status_str(int(status)).decode()


def check(status: int, where: str) -> None:
    if status != OK:
        raise BreadError(int(status), where)


def default_shape() -> MoeShape:
    s = MoeShape()
    lib.bread_moe_shape_default(ctypes.byref(s))
    return s
