"""Shared test helpers: seeded layers on the device, their host copies for the
oracle, and error metrics."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def oshape(s) -> "O.OShape":
    return O.OShape(s.hidden, s.expert_inter, s.shared_inter, s.n_experts, s.top_k)


def host_layer(t, drop_shgate: bool = False) -> "O.HostLayer":
    """Copy a breadv2_amd.LayerTensors to the host for the oracle."""
    sh = None if (drop_shgate or t.shgate is None) else t.shgate.cpu().numpy().view(np.uint16)
    return O.HostLayer(
        oshape(t.shape),
        t.gate_exps.cpu().numpy(), t.up_exps.cpu().numpy(), t.down_exps.cpu().numpy(),
        t.gate_sh.cpu().numpy(), t.up_sh.cpu().numpy(), t.down_sh.cpu().numpy(),
        t.router.cpu().numpy(), sh,
    )


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


# MoE-layer output tolerance of the north star: 1e-3 relative L2 and 1e-2
# max-abs against the fp32 reference computation on the same inputs.
REL_L2_TOL = 1e-3
MAX_ABS_TOL = 1e-2


def d2h(ptr: int, nbytes: int) -> np.ndarray:
    """Copy nbytes of device memory at a raw pointer to a new host array."""
    import ctypes

    import torch

    torch.cuda.synchronize()
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    out = np.empty(nbytes, np.uint8)
    rc = hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2)  # hipMemcpyDeviceToHost
    assert rc == 0, f"hipMemcpy failed: {rc}"
    return out


def arena_host_layer(s, d) -> "O.HostLayer":
    """Host copy (for the oracle) of one arena layer descriptor."""
    from breadv2_amd import api

    b = api.shape_bytes(s)
    E = s.n_experts
    return O.HostLayer(
        oshape(s),
        d2h(d.gate_exps, E * b["gate_expert"]), d2h(d.up_exps, E * b["up_expert"]),
        d2h(d.down_exps, E * b["down_expert"]), d2h(d.gate_shexp, b["gate_sh"]),
        d2h(d.up_shexp, b["up_sh"]), d2h(d.down_shexp, b["down_sh"]),
        d2h(d.router, b["router"]).view(np.float32), d2h(d.shexp_gate, b["shgate"]).view(np.uint16),
    )
