"""GPU: the compiled C++ caller of the library (tests/abi_caller.cpp, built by
tests/Makefile) against the CPU oracle.  It calls bread_matvec through the
reference's own C++ prototype (one_layer.cu:46-47) with the arguments of
one_layer.cu:1966-1977, and the MoE block through bread_moe_forward_f16 on
fp16 d_hidden / d_normed2 buffers (one_layer.cu:1800-1986), in a process of
its own that links libbread_moe.so directly.

- bread_matvec (Q4_K gate shape 512 x 2048, Q6_K down shape 2048 x 512): the
  oracle's fp16-rounded result within one fp16 ulp plus the fp32
  summation-order bound (as tests/test_gpu_quant.py);
- the MoE block at the decode kernel's shape (H 2048, I 512, 32 experts,
  top 8, unit-scale superblocks): normed input within one fp16 ulp of the
  oracle's RMSNorm, routing bit-exact against the oracle on that input, and
  the block's contribution to the fp16 residual within the north-star
  tolerance (1e-3 relative L2, 1e-2 max-abs of its RMS) of the oracle's fp32
  block, plus the one rounding of the result to fp16.
"""
import os
import subprocess

import numpy as np
import pytest
import torch

from breadv2_amd import api
from oracle import oracle as O

from helpers import host_layer, scale_layer_d
from test_gpu_quant import abs_bound, weights

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLER = os.path.join(ROOT, "tests", "_build", "abi_caller")


def run_caller(mode, d):
    assert os.access(CALLER, os.X_OK), f"{CALLER} missing: build it with make -C tests"
    print(f"abi_caller {mode} {d}", flush=True)
    r = subprocess.run([CALLER, mode, str(d)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]


def ulp16(a):
    a = np.abs(np.asarray(a, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(a, 2.0 ** -14))) - 10)


@pytest.mark.parametrize("qtype,rows,cols", [(O.QTYPE_Q4_K, 512, 2048), (O.QTYPE_Q6_K, 2048, 512)])
def test_caller_matvec_through_reference_prototype(tmp_path, qtype, rows, cols):
    w = weights(qtype, rows, cols, seed=41 + rows)
    x16 = np.random.default_rng(42).standard_normal(cols).astype(np.float16)
    (tmp_path / "meta.txt").write_text(f"{rows} {cols} {qtype}\n")
    w.tofile(tmp_path / "w.bin")
    x16.tofile(tmp_path / "x.bin")
    run_caller("matvec", tmp_path)
    got = np.fromfile(tmp_path / "y.bin", np.float16).astype(np.float32)
    ref = O.matvec_f16io(w, qtype, x16.view(np.uint16), rows, cols).view(np.float16).astype(np.float32)
    order = 2 * cols * 2.0 ** -24 * abs_bound(w, qtype, x16.astype(np.float32), rows, cols)
    assert np.all(np.abs(got - ref) <= np.spacing(np.abs(ref)) + order + 1e-6)


def test_caller_moe_block_f16(tmp_path):
    s = api.shape(n_experts=32)
    t = api.synth_layer_tensors(s, seed=4242, router_std=1.0 / np.sqrt(s.hidden))
    scale_layer_d(t, 6)
    torch.cuda.synchronize()
    hl = host_layer(t)
    rng = np.random.default_rng(43)
    h16 = (2.0 * rng.standard_normal(s.hidden)).astype(np.float16)
    nw = (1.0 + 0.1 * rng.standard_normal(s.hidden)).astype(np.float32)
    (tmp_path / "meta.txt").write_text(
        f"{s.hidden} {s.expert_inter} {s.shared_inter} {s.n_experts} {s.top_k} {s.rms_eps!r}\n")
    for name in ("gate_exps", "up_exps", "down_exps"):
        getattr(t, name).cpu().numpy().tofile(tmp_path / f"{name}.bin")
    for name, fn in (("gate_sh", "gate_sh"), ("up_sh", "up_sh"), ("down_sh", "down_sh")):
        getattr(t, name).cpu().numpy().tofile(tmp_path / f"{fn}.bin")
    t.router.cpu().numpy().tofile(tmp_path / "router.bin")
    t.shgate.cpu().numpy().tofile(tmp_path / "shgate.bin")
    nw.tofile(tmp_path / "norm_w.bin")
    h16.tofile(tmp_path / "hidden.bin")
    run_caller("moe", tmp_path)
    got_h = np.fromfile(tmp_path / "hidden_out.bin", np.float16)
    got_n = np.fromfile(tmp_path / "normed.bin", np.float16)
    gi = np.fromfile(tmp_path / "idx.bin", np.int32)
    # the normalised input: the oracle's RMSNorm rounded to fp16, within one ulp
    ref_n = O.rms_norm_weighted(h16.astype(np.float32), nw, s.rms_eps)
    assert np.all(np.abs(got_n.astype(np.float64) - ref_n.astype(np.float16).astype(np.float64)) <= ulp16(ref_n))
    # routing and the block on that input
    x = got_n.astype(np.float32)[None]
    ref = h16.astype(np.float32)[None].copy()
    ri, _, _ = O.moe_forward(hl, x, ref, 1, nthreads=16)
    assert np.array_equal(gi, np.asarray(ri).reshape(-1)), f"{gi} vs oracle {ri}"
    # the block's contribution within the north-star tolerance of the
    # oracle's fp32 block, plus the one rounding of the result to fp16
    base = h16.astype(np.float64)
    got_c, ref_c = got_h.astype(np.float64) - base, ref[0].astype(np.float64) - base
    rms = float(np.sqrt(np.mean(ref_c ** 2)))
    assert 0.1 < rms < 1e3
    half_ulp = 0.5 * ulp16(ref[0])
    rel = float(np.linalg.norm(got_c - ref_c) / np.linalg.norm(ref_c))
    assert rel < 1e-3 + float(np.linalg.norm(half_ulp) / np.linalg.norm(ref_c)), rel
    assert np.all(np.abs(got_c - ref_c) <= 1e-2 * rms + half_ulp)
