"""Python host layer over the C ABI: device memory and streams come from
PyTorch (plumbing); every computation is a call into libbread_moe.so.

Names mirror the reference's interface for this path (kernels.cu:289
bread_matvec, one_layer.cu:937 route_layer, the MoE block of
one_layer_forward one_layer.cu:1800-1986), with the reference's exit(1)
replaced by a raised BreadError carrying the status code.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import BreadError, MoeLayer, MoeShape, check, lib

QTYPE_Q8_0 = _lib.QTYPE_Q8_0
QTYPE_Q4_K = _lib.QTYPE_Q4_K
QTYPE_Q6_K = _lib.QTYPE_Q6_K
PATH_AUTO = _lib.PATH_AUTO
PATH_DECODE = _lib.PATH_DECODE
PATH_GROUPED = _lib.PATH_GROUPED
PATH_PER_TOKEN = _lib.PATH_PER_TOKEN
PATH_SMALL = _lib.PATH_SMALL


def _p(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _s(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


_HIP = None


def device_copy(dst: int, src: int, nbytes: int) -> None:
    """Synchronous device-to-device copy between raw device pointers (HIP
    runtime of the process, which torch has loaded)."""
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _HIP.hipMemcpy.restype = ctypes.c_int
    torch.cuda.synchronize()
    rc = _HIP.hipMemcpy(dst, src, nbytes, 3)  # hipMemcpyDeviceToDevice
    if rc != 0:
        raise RuntimeError(f"hipMemcpy failed: {rc}")


def row_bytes(qtype: int, cols: int) -> int:
    if qtype == QTYPE_Q4_K:
        return cols // 256 * 144
    if qtype == QTYPE_Q6_K:
        return cols // 256 * 210
    if qtype == QTYPE_Q8_0:
        return cols // 32 * 34
    raise ValueError(f"qtype {qtype}")


# ---------------------------------------------------------------- matvec


def bread_matvec(w, x, y, rows: int, cols: int, qtype: int, stream=None) -> None:
    """fp16 in / fp16 out (kernels.cu:289). x, y: torch.float16 device tensors."""
    check(lib.bread_matvec(_p(w), _p(x), _p(y), rows, cols, qtype, _s(stream)), "bread_matvec")


def bread_matvec_f32(w, x, y, rows: int, cols: int, qtype: int, stream=None) -> None:
    check(lib.bread_matvec_f32(_p(w), _p(x), _p(y), rows, cols, qtype, _s(stream)), "bread_matvec_f32")


def bread_dequant_rows(w, qtype: int, rows: int, cols: int, out=None, stream=None) -> torch.Tensor:
    if out is None:
        out = torch.empty(rows * cols, dtype=torch.float32, device=w.device)
    check(lib.bread_dequant_rows(_p(w), qtype, rows, cols, _p(out), _s(stream)), "bread_dequant_rows")
    return out


def bread_rmsnorm_f32(x, w, out, n: int, n_tokens: int, eps: float, stream=None) -> None:
    check(lib.bread_rmsnorm_f32(_p(x), _p(w), _p(out), n, n_tokens, eps, _s(stream)), "bread_rmsnorm_f32")


# ---------------------------------------------------------------- synth


def synth_q4k(dst, n_blocks: int, seed: int, stream=None) -> None:
    check(lib.bread_synth_q4k(_p(dst), n_blocks, seed, _s(stream)), "bread_synth_q4k")


def synth_q6k(dst, n_blocks: int, seed: int, stream=None) -> None:
    check(lib.bread_synth_q6k(_p(dst), n_blocks, seed, _s(stream)), "bread_synth_q6k")


def synth_normal_f32(dst, n: int, seed: int, mean: float, std: float, stream=None) -> None:
    check(lib.bread_synth_normal_f32(_p(dst), n, seed, mean, std, _s(stream)), "bread_synth_normal_f32")


def synth_normal_f16(dst, n: int, seed: int, mean: float, std: float, stream=None) -> None:
    check(lib.bread_synth_normal_f16(_p(dst), n, seed, mean, std, _s(stream)), "bread_synth_normal_f16")


# ---------------------------------------------------------------- shape / layers


def shape(hidden=2048, expert_inter=512, shared_inter=512, n_experts=256, top_k=8, rms_eps=1e-6) -> MoeShape:
    return MoeShape(hidden, expert_inter, shared_inter, n_experts, top_k, rms_eps)


# Expert tensor types of a layer: gate, up, down, gate_shexp, up_shexp,
# down_shexp.  STANDARD_TYPES is the mix the reference GPU path hardcodes and
# the specialised kernels take; each entry may be Q4_K or Q6_K.
STANDARD_TYPES = (QTYPE_Q4_K, QTYPE_Q4_K, QTYPE_Q6_K, QTYPE_Q4_K, QTYPE_Q4_K, QTYPE_Q6_K)
BLOCK_BYTES = {QTYPE_Q4_K: 144, QTYPE_Q6_K: 210}


def row_bytes(qtype: int, cols: int) -> int:
    """Bytes of one Q4_K or Q6_K row of cols columns."""
    return (cols // 256) * BLOCK_BYTES[qtype]


def layer_types(d: MoeLayer) -> tuple:
    return (d.gate_type, d.up_type, d.down_type, d.gate_shexp_type, d.up_shexp_type, d.down_shexp_type)


def shape_bytes(s: MoeShape, types=STANDARD_TYPES) -> dict:
    """Byte sizes of one layer's tensors (native GGUF layout)."""
    H, I, Ish, E = s.hidden, s.expert_inter, s.shared_inter, s.n_experts
    g, u, d, gs, us, ds = types
    return {
        "gate_expert": I * row_bytes(g, H),
        "up_expert": I * row_bytes(u, H),
        "down_expert": H * row_bytes(d, I),
        "gate_sh": Ish * row_bytes(gs, H),
        "up_sh": Ish * row_bytes(us, H),
        "down_sh": H * row_bytes(ds, Ish),
        "router": E * H * 4,
        "shgate": H * 2,
    }


def synth_quant(dst, qtype: int, nbytes: int, seed: int, stream=None) -> None:
    """Fill nbytes of Q4_K or Q6_K superblocks with the device generator."""
    fn = synth_q4k if qtype == QTYPE_Q4_K else synth_q6k
    fn(dst, nbytes // BLOCK_BYTES[qtype], seed, stream)


def route_noalloc(s: MoeShape, layer: MoeLayer, x: torch.Tensor, n_tokens: int, stream=None):
    """bread_route_noalloc: routing without a context (the library's static
    device workspace holds the logits; n_tokens * n_experts <= 1048576)."""
    K = s.top_k
    idx = torch.empty((n_tokens, K), dtype=torch.int32, device=x.device)
    w = torch.empty((n_tokens, K), dtype=torch.float32, device=x.device)
    gsh = torch.empty((n_tokens,), dtype=torch.float32, device=x.device)
    check(lib.bread_route_noalloc(ctypes.byref(s), ctypes.byref(layer), _p(x), n_tokens, _p(idx), _p(w), _p(gsh),
                                  _s(stream)), "bread_route_noalloc")
    return idx, w, gsh


@dataclass
class LayerTensors:
    """One layer's weights as device tensors (keeps them alive)."""

    shape: MoeShape
    gate_exps: torch.Tensor
    up_exps: torch.Tensor
    down_exps: torch.Tensor
    gate_sh: torch.Tensor
    up_sh: torch.Tensor
    down_sh: torch.Tensor
    router: torch.Tensor
    shgate: torch.Tensor | None
    types: tuple = STANDARD_TYPES

    def desc(self) -> MoeLayer:
        b = shape_bytes(self.shape, self.types)
        g, u, d, gs, us, ds = self.types
        return MoeLayer(
            self.gate_exps.data_ptr(), self.up_exps.data_ptr(), self.down_exps.data_ptr(),
            b["gate_expert"], b["up_expert"], b["down_expert"],
            g, u, d,
            self.gate_sh.data_ptr(), self.up_sh.data_ptr(), self.down_sh.data_ptr(),
            gs, us, ds,
            self.router.data_ptr(),
            self.shgate.data_ptr() if self.shgate is not None else None,
            None,
        )


def layer_seeds(seed: int, layer: int) -> dict:
    base = (seed * 1_000_003 + layer * 101) & ((1 << 63) - 1)
    names = ["gate_exps", "up_exps", "down_exps", "gate_sh", "up_sh", "down_sh", "router", "shgate"]
    return {n: base + i for i, n in enumerate(names)}


def synth_layer_tensors(s: MoeShape, seed: int, layer: int = 0, router_std: float = 0.02,
                        shgate_std: float = 0.02, device="cuda", stream=None, types=STANDARD_TYPES) -> LayerTensors:
    """Allocate one layer with torch and fill it with the device generator
    (types: the six expert tensor types, each Q4_K or Q6_K)."""
    types = tuple(types)
    b = shape_bytes(s, types)
    E = s.n_experts
    sd = layer_seeds(seed, layer)
    u8 = dict(dtype=torch.uint8, device=device)
    t = LayerTensors(
        s,
        torch.empty(E * b["gate_expert"], **u8),
        torch.empty(E * b["up_expert"], **u8),
        torch.empty(E * b["down_expert"], **u8),
        torch.empty(b["gate_sh"], **u8),
        torch.empty(b["up_sh"], **u8),
        torch.empty(b["down_sh"], **u8),
        torch.empty(E * s.hidden, dtype=torch.float32, device=device),
        torch.empty(s.hidden, dtype=torch.float16, device=device),
        types,
    )
    g, u, d, gs, us, ds = types
    synth_quant(t.gate_exps, g, E * b["gate_expert"], sd["gate_exps"], stream)
    synth_quant(t.up_exps, u, E * b["up_expert"], sd["up_exps"], stream)
    synth_quant(t.down_exps, d, E * b["down_expert"], sd["down_exps"], stream)
    synth_quant(t.gate_sh, gs, b["gate_sh"], sd["gate_sh"], stream)
    synth_quant(t.up_sh, us, b["up_sh"], sd["up_sh"], stream)
    synth_quant(t.down_sh, ds, b["down_sh"], sd["down_sh"], stream)
    synth_normal_f32(t.router, E * s.hidden, sd["router"], 0.0, router_std, stream)
    synth_normal_f16(t.shgate, s.hidden, sd["shgate"], 0.0, shgate_std, stream)
    return t


def argmax_f16(logits: torch.Tensor, stream=None) -> torch.Tensor:
    """bread_argmax_f16 over the rows of a 2-d fp16 device tensor."""
    assert logits.dtype == torch.float16 and logits.dim() == 2 and logits.is_contiguous()
    out = torch.empty((logits.shape[0],), dtype=torch.int32, device=logits.device)
    check(lib.bread_argmax_f16(_p(logits), logits.shape[1], logits.shape[0], _p(out), _s(stream)),
          "bread_argmax_f16")
    return out


def spec_accept(pred, draft, eos: int, max_accept: int):
    """bread_spec_accept on host lists: (n_accept, next token)."""
    pred = list(pred)
    draft = list(draft)
    assert len(pred) == len(draft) + 1
    pa = (ctypes.c_int32 * len(pred))(*pred)
    da = (ctypes.c_int32 * max(1, len(draft)))(*draft)
    na, nx = ctypes.c_int(), ctypes.c_int32()
    check(lib.bread_spec_accept(pa, da, len(draft), eos, max_accept, ctypes.byref(na), ctypes.byref(nx)),
          "bread_spec_accept")
    return na.value, nx.value


class Gguf:
    """A parsed GGUF v2/v3 file (bread_gguf_*): metadata and tensor index over
    a read-only mapping; weights are read when loaded into an Arena."""

    def __init__(self, path: str):
        self._h = ctypes.c_void_p()
        check(lib.bread_gguf_open(path.encode(), ctypes.byref(self._h)), "bread_gguf_open")

    def info(self) -> dict:
        v, a = ctypes.c_uint32(), ctypes.c_uint32()
        nt, nk, off = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        check(lib.bread_gguf_info(self._h, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nk), ctypes.byref(off),
                                  ctypes.byref(a)), "bread_gguf_info")
        return {"version": v.value, "n_tensors": nt.value, "n_kv": nk.value, "data_offset": off.value,
                "alignment": a.value}

    @staticmethod
    def _t(t: _lib.GgufTensor) -> dict:
        return {"name": t.name.decode(), "type": t.type, "dims": list(t.dims[: t.n_dims]), "offset": t.offset,
                "size": t.size, "n_elems": t.n_elems, "data": t.data}

    def tensor(self, i: int) -> dict:
        t = _lib.GgufTensor()
        check(lib.bread_gguf_tensor(self._h, i, ctypes.byref(t)), "bread_gguf_tensor")
        return self._t(t)

    def tensors(self) -> list:
        return [self.tensor(i) for i in range(self.info()["n_tensors"])]

    def find(self, name: str):
        t = _lib.GgufTensor()
        return self._t(t) if lib.bread_gguf_find(self._h, name.encode(), ctypes.byref(t)) == 0 else None

    def kv_int(self, key: str):
        v = ctypes.c_int64()
        return v.value if lib.bread_gguf_kv_int(self._h, key.encode(), ctypes.byref(v)) == 0 else None

    def kv_float(self, key: str):
        v = ctypes.c_double()
        return v.value if lib.bread_gguf_kv_float(self._h, key.encode(), ctypes.byref(v)) == 0 else None

    def kv_str(self, key: str):
        b = ctypes.create_string_buffer(4096)
        return b.value.decode() if lib.bread_gguf_kv_str(self._h, key.encode(), b, 4096) == 0 else None

    def moe_shape(self, layer: int) -> MoeShape:
        sh = MoeShape()
        check(lib.bread_gguf_moe_shape(self._h, layer, ctypes.byref(sh)), "bread_gguf_moe_shape")
        return sh

    def close(self) -> None:
        if self._h:
            lib.bread_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Arena:
    """All experts of n_layers layers resident in HBM (bread_arena_*)."""

    def __init__(self, s: MoeShape, n_layers: int):
        self.shape = s
        self.n_layers = n_layers
        self._h = ctypes.c_void_p()
        check(lib.bread_arena_create(ctypes.byref(s), n_layers, ctypes.byref(self._h)), "bread_arena_create")

    @property
    def layer_bytes(self) -> int:
        return int(lib.bread_arena_layer_bytes(self._h))

    def layer(self, l: int) -> MoeLayer:
        d = MoeLayer()
        check(lib.bread_arena_layer(self._h, l, ctypes.byref(d)), "bread_arena_layer")
        return d

    def set_layer_types(self, l: int, types) -> None:
        """bread_arena_set_layer_types: the six expert tensor types of layer l
        (gate, up, down, gate_shexp, up_shexp, down_shexp; Q4_K or Q6_K)."""
        check(lib.bread_arena_set_layer_types(self._h, l, *[int(t) for t in types]), "bread_arena_set_layer_types")

    def synth_layer(self, l: int, seed: int, router_std=0.02, shgate_std=0.02, stream=None) -> None:
        d = self.layer(l)
        s = self.shape
        types = layer_types(d)
        b = shape_bytes(s, types)
        E = s.n_experts
        sd = layer_seeds(seed, l)
        st = _s(stream)

        def q(qtype, ptr, nbytes, sv):
            fn = lib.bread_synth_q4k if qtype == QTYPE_Q4_K else lib.bread_synth_q6k
            check(fn(ctypes.c_void_p(ptr), nbytes // BLOCK_BYTES[qtype], sv, st), fn.__name__)

        g, u, dn, gs, us, ds = types
        q(g, d.gate_exps, E * b["gate_expert"], sd["gate_exps"])
        q(u, d.up_exps, E * b["up_expert"], sd["up_exps"])
        q(dn, d.down_exps, E * b["down_expert"], sd["down_exps"])
        q(gs, d.gate_shexp, b["gate_sh"], sd["gate_sh"])
        q(us, d.up_shexp, b["up_sh"], sd["up_sh"])
        q(ds, d.down_shexp, b["down_sh"], sd["down_sh"])
        check(lib.bread_synth_normal_f32(ctypes.c_void_p(d.router), E * s.hidden, sd["router"], 0.0, router_std, st),
              "bread_synth_normal_f32")
        if d.shexp_gate:
            check(lib.bread_synth_normal_f16(ctypes.c_void_p(d.shexp_gate), s.hidden, sd["shgate"], 0.0, shgate_std,
                                             st), "bread_synth_normal_f16")

    def load_gguf(self, l: int, g: "Gguf", gguf_layer: int) -> None:
        """bread_arena_load_gguf: block gguf_layer's MoE tensors into layer l."""
        check(lib.bread_arena_load_gguf(self._h, l, g._h, gguf_layer), "bread_arena_load_gguf")

    def set_router_column(self, l: int, col: int, values) -> None:
        """Overwrite column col of layer l's fp32 router [E][H] with values[E]
        (e.g. a routing bias carried by a constant activation feature)."""
        d = self.layer(l)
        E, H = self.shape.n_experts, self.shape.hidden
        r = torch.empty(E * H, dtype=torch.float32, device=torch.device("cuda", torch.cuda.current_device()))
        device_copy(r.data_ptr(), d.router, E * H * 4)
        r.view(E, H)[:, col] = torch.as_tensor(values, dtype=torch.float32).to(r.device)
        device_copy(d.router, r.data_ptr(), E * H * 4)

    def close(self) -> None:
        if self._h:
            lib.bread_arena_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoeContext:
    """bread_moe_ctx_t: scratch for MoE calls on one stream."""

    def __init__(self, s: MoeShape, max_tokens: int = 1):
        self.shape = s
        self.max_tokens = max_tokens
        self._h = ctypes.c_void_p()
        check(lib.bread_moe_ctx_create(ctypes.byref(s), max_tokens, ctypes.byref(self._h)), "bread_moe_ctx_create")

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def set_path(self, path: int) -> None:
        """bread_moe_ctx_set_path: PATH_AUTO, PATH_DECODE, PATH_GROUPED, PATH_PER_TOKEN or PATH_SMALL."""
        check(lib.bread_moe_ctx_set_path(self._h, path), "bread_moe_ctx_set_path")

    def set_spin_limit(self, n_sleeps: int) -> None:
        """bread_moe_ctx_set_spin_limit: bound every wait of the decode and
        small-batch kernels at n_sleeps sleeps after the first look (< 0: the
        kernels' defaults).  A small bound forces the time-out error paths."""
        check(lib.bread_moe_ctx_set_spin_limit(self._h, n_sleeps), "bread_moe_ctx_set_spin_limit")

    def route(self, layer: MoeLayer, x: torch.Tensor, n_tokens: int, stream=None):
        K = self.shape.top_k
        idx = torch.empty((n_tokens, K), dtype=torch.int32, device=x.device)
        w = torch.empty((n_tokens, K), dtype=torch.float32, device=x.device)
        gsh = torch.empty((n_tokens,), dtype=torch.float32, device=x.device)
        check(lib.bread_route(self._h, ctypes.byref(layer), _p(x), n_tokens, _p(idx), _p(w), _p(gsh), _s(stream)),
              "bread_route")
        return idx, w, gsh

    def route_layer(self, layer: MoeLayer, x: torch.Tensor, stream=None):
        """route_layer shim (one_layer.cu:937): host lists and the raw gate logit."""
        K = self.shape.top_k
        idx = (ctypes.c_int32 * K)()
        w = (ctypes.c_float * K)()
        g = ctypes.c_float()
        check(lib.bread_route_layer(self._h, ctypes.byref(layer), _p(x), idx, w, ctypes.byref(g), _s(stream)),
              "bread_route_layer")
        return list(idx), list(w), g.value

    def route_layer_f16(self, layer: MoeLayer, normed16: torch.Tensor, stream=None):
        """route_layer on the reference's own input (one_layer.cu:937-939):
        fp16 d_normed2 [H], widened on the device; host lists and the raw
        shared-gate logit."""
        assert normed16.dtype == torch.float16 and normed16.is_contiguous()
        K = self.shape.top_k
        idx = (ctypes.c_int32 * K)()
        w = (ctypes.c_float * K)()
        g = ctypes.c_float()
        check(lib.bread_route_layer_f16(self._h, ctypes.byref(layer), _p(normed16), idx, w, ctypes.byref(g),
                                        _s(stream)), "bread_route_layer_f16")
        return list(idx), list(w), g.value

    def forward(self, layer: MoeLayer, x: torch.Tensor, hidden: torch.Tensor, n_tokens: int,
                want_routing: bool = False, stream=None):
        K = self.shape.top_k
        idx = w = gsh = None
        if want_routing:
            idx = torch.empty((n_tokens, K), dtype=torch.int32, device=x.device)
            w = torch.empty((n_tokens, K), dtype=torch.float32, device=x.device)
            gsh = torch.empty((n_tokens,), dtype=torch.float32, device=x.device)
        check(lib.bread_moe_forward(self._h, ctypes.byref(layer), _p(x), _p(hidden), n_tokens, _p(idx), _p(w),
                                    _p(gsh), _s(stream)), "bread_moe_forward")
        return idx, w, gsh

    def expert_block(self, layer: MoeLayer, x: torch.Tensor, hidden: torch.Tensor, n_tokens: int,
                     idx: torch.Tensor, w: torch.Tensor, stream=None) -> None:
        """bread_moe_expert_block: hidden += sum_k w[t][k] * expert_{idx[t][k]}(x_t),
        routed experts only, with the caller's routing (device int32 / fp32 [n_tokens][K])."""
        assert idx.dtype == torch.int32 and w.dtype == torch.float32
        check(lib.bread_moe_expert_block(self._h, ctypes.byref(layer), _p(x), _p(hidden), n_tokens, _p(idx),
                                         _p(w), _s(stream)), "bread_moe_expert_block")

    def forward_f16(self, layer: MoeLayer, hidden: torch.Tensor, normed: torch.Tensor, n_tokens: int,
                    norm_w=None, want_routing: bool = False, stream=None):
        """bread_moe_forward_f16: the MoE block on fp16 hidden / normed
        [n_tokens][H] (one_layer.cu:1800-1986).  norm_w: a float32 device
        tensor or raw device pointer (e.g. layer.post_norm_w); None takes
        `normed` as the input instead of computing it."""
        assert hidden.dtype == torch.float16 and normed.dtype == torch.float16
        K = self.shape.top_k
        idx = w = gsh = None
        if want_routing:
            idx = torch.empty((n_tokens, K), dtype=torch.int32, device=hidden.device)
            w = torch.empty((n_tokens, K), dtype=torch.float32, device=hidden.device)
            gsh = torch.empty((n_tokens,), dtype=torch.float32, device=hidden.device)
        nw = norm_w if isinstance(norm_w, int) or norm_w is None else norm_w.data_ptr()
        check(lib.bread_moe_forward_f16(self._h, ctypes.byref(layer), nw, _p(hidden), _p(normed), n_tokens, _p(idx),
                                        _p(w), _p(gsh), _s(stream)), "bread_moe_forward_f16")
        return idx, w, gsh

    def decode_layers(self, layers, hidden: torch.Tensor, want_routing: bool = False, stream=None):
        """bread_moe_decode_layers: one token through len(layers) layers,
        h <- h + MoE_l(RMSNorm(h) * w_l), in one launch."""
        n = len(layers)
        arr = (MoeLayer * n)(*layers)
        K = self.shape.top_k
        idx = w = gsh = None
        if want_routing:
            idx = torch.empty((n, K), dtype=torch.int32, device=hidden.device)
            w = torch.empty((n, K), dtype=torch.float32, device=hidden.device)
            gsh = torch.empty((n,), dtype=torch.float32, device=hidden.device)
        check(lib.bread_moe_decode_layers(self._h, arr, n, _p(hidden), _p(idx), _p(w), _p(gsh), _s(stream)),
              "bread_moe_decode_layers")
        return idx, w, gsh

    def decode_launcher(self, layers, hidden: torch.Tensor, stream=None):
        """A callable f(i) that runs bread_moe_decode_layers on the single
        layer layers[i % len(layers)] with every ctypes argument built once:
        a launch costs one foreign call (for loops that time the kernel)."""
        arrs = [(MoeLayer * 1)(l) for l in layers]
        n = len(arrs)
        fn = lib.bread_moe_decode_layers
        h, hp, sp = self._h, _p(hidden), _s(stream)

        def launch(i: int) -> None:
            rc = fn(h, arrs[i % n], 1, hp, None, None, None, sp)
            if rc:
                check(rc, "bread_moe_decode_layers")

        return launch

    def stack_forward(self, layers, hidden: torch.Tensor, n_tokens: int, want_routing: bool = False, stream=None):
        """bread_moe_stack_forward: n_tokens tokens through len(layers) MoE
        layers, h <- h + MoE_l(RMSNorm(h) * w_l): one batched call per layer,
        or one decode-stack launch per token for up to
        bread_stack_loop_tokens() tokens (automatic choice)."""
        n = len(layers)
        arr = (MoeLayer * n)(*layers)
        K = self.shape.top_k
        idx = w = gsh = None
        if want_routing:
            idx = torch.empty((n, n_tokens, K), dtype=torch.int32, device=hidden.device)
            w = torch.empty((n, n_tokens, K), dtype=torch.float32, device=hidden.device)
            gsh = torch.empty((n, n_tokens), dtype=torch.float32, device=hidden.device)
        check(lib.bread_moe_stack_forward(self._h, arr, n, _p(hidden), n_tokens, _p(idx), _p(w), _p(gsh),
                                          _s(stream)), "bread_moe_stack_forward")
        return idx, w, gsh

    def greedy_head(self, hidden: torch.Tensor, norm_w: torch.Tensor | None, w_out: torch.Tensor, qtype: int,
                    vocab: int, n_tokens: int, stream=None):
        """bread_moe_greedy_head: (tokens int32 [n_tokens], fp16 logits
        [n_tokens][vocab]) of the output norm + lm_head + greedy argmax."""
        logits = torch.empty((n_tokens, vocab), dtype=torch.float16, device=hidden.device)
        tokens = torch.empty((n_tokens,), dtype=torch.int32, device=hidden.device)
        check(lib.bread_moe_greedy_head(self._h, _p(hidden), _p(norm_w), _p(w_out), qtype, vocab, n_tokens,
                                        _p(logits), _p(tokens), _s(stream)), "bread_moe_greedy_head")
        return tokens, logits

    def set_trace(self, buf: torch.Tensor | None) -> int:
        """Record the decode kernel's timeline into buf (int64 device tensor)."""
        g = ctypes.c_int(0)
        n = 0 if buf is None else buf.numel()
        check(lib.bread_moe_ctx_set_trace(self._h, _p(buf), n, ctypes.byref(g)), "bread_moe_ctx_set_trace")
        self._trace = buf
        return g.value

    ROUTE_STAT_NAMES = ("decode_radius", "decode_per_expert", "decode_pair", "decode_exact",
                        "multi_certified", "multi_candidates", "multi_exact")

    def route_stats(self, reset: bool = False) -> dict:
        """bread_moe_ctx_route_stats: how often exact routing took each path
        (decode layers by certificate outcome, multi-token tokens certified
        or recomputed), since creation or the last reset."""
        n = len(self.ROUTE_STAT_NAMES)
        out = (ctypes.c_uint64 * n)()
        check(lib.bread_moe_ctx_route_stats(self._h, out, n, 1 if reset else 0), "bread_moe_ctx_route_stats")
        return dict(zip(self.ROUTE_STAT_NAMES, (int(v) for v in out)))

    def check_device(self) -> int:
        """bread_moe_ctx_check: 0, or BreadError carrying the kernels' error
        word in .device_error (the call clears it and resets the context)."""
        e = ctypes.c_int(0)
        rc = lib.bread_moe_ctx_check(self._h, ctypes.byref(e))
        if rc != _lib.OK:
            raise BreadError(int(rc), "bread_moe_ctx_check", e.value)
        return e.value

    def close(self) -> None:
        if self._h:
            lib.bread_moe_ctx_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
