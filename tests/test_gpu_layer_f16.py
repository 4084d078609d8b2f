"""GPU: bread_moe_forward_f16, the MoE block of one_layer_forward on the
reference's fp16 residual stream (one_layer.cu:1800-1986, d_hidden and
d_normed2 as fp16, :1812-1815).

The checks chain to the oracle, on a unit-scale layer (superblock scales /
64, outputs of order one and inside fp16's range):
- the normalised input it writes matches the oracle's RMSNorm rounded to
  fp16 within one fp16 ulp (summation order and sqrt may differ in the last
  fp32 bit, which moves a rounding boundary at most one ulp);
- routing on that input is bit-exact against the oracle;
- the fp16 residual is bit-identical to bread_moe_forward on the fp32
  widening of the same fp16 inputs, rounded to fp16 once (the entry adds
  only the conversions);
- that fp32 result is within the layer tolerance of the oracle (1e-3
  relative L2, 1e-2 max-abs, on the block's contribution);
- with norm_w NULL the given `normed` is the input and is left unchanged.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

from helpers import assert_moe_close, host_layer, scale_layer_d

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def unit_layer():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=777)
    scale_layer_d(t, 6)
    torch.cuda.synchronize()
    return s, t, host_layer(t)


def ulp16(a: np.ndarray) -> np.ndarray:
    """Spacing of fp16 at |a| (subnormal spacing 2^-24 below 2^-14)."""
    a = np.abs(np.asarray(a, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def inputs(T, H, seed):
    rng = np.random.default_rng(seed)
    h16 = (2.0 * rng.standard_normal((T, H))).astype(np.float16)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    return h16, nw


def run_f16(ctx, t, h16, normed16, nw):
    hd = torch.from_numpy(h16.copy()).to(DEV)
    nd = torch.from_numpy(normed16.copy()).to(DEV)
    nwd = None if nw is None else torch.from_numpy(nw).to(DEV)
    idx, w, _ = ctx.forward_f16(t.desc(), hd, nd, h16.shape[0], norm_w=nwd, want_routing=True)
    torch.cuda.synchronize()
    return hd.cpu().numpy(), nd.cpu().numpy(), idx.cpu().numpy()


def check_chain(ctx, s, t, hl, h16, got_h, normed16, gi):
    T = h16.shape[0]
    x = normed16.astype(np.float32)
    ref = h16.astype(np.float32)
    ri, _, _ = O.moe_forward(hl, x, ref, T, nthreads=16)
    assert np.array_equal(gi, np.asarray(ri).reshape(gi.shape))
    hd = torch.from_numpy(h16.astype(np.float32)).to(DEV)
    ctx.forward(t.desc(), torch.from_numpy(x).to(DEV), hd, T)
    torch.cuda.synchronize()
    dev32 = hd.cpu().numpy()
    assert np.array_equal(got_h.view(np.uint16), dev32.astype(np.float16).view(np.uint16))
    assert 0.1 < float(np.sqrt(np.mean((ref - h16.astype(np.float32)).astype(np.float64) ** 2))) < 1e3
    assert_moe_close(dev32, ref, base=h16.astype(np.float32))
    assert ctx.check_device() == 0


@pytest.mark.parametrize("T,path", [(1, api.PATH_AUTO), (16, api.PATH_AUTO), (5, api.PATH_PER_TOKEN)])
def test_f16_block_matches_oracle(unit_layer, T, path):
    s, t, hl = unit_layer
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    h16, nw = inputs(T, s.hidden, 90 + T)
    got_h, got_n, gi = run_f16(ctx, t, h16, np.zeros_like(h16), nw)
    assert ctx.check_device() == 0
    # the normalised input: oracle RMSNorm (fp32) rounded to fp16
    ref_n = np.stack([O.rms_norm_weighted(h16[i].astype(np.float32), nw, s.rms_eps) for i in range(T)])
    dn = np.abs(got_n.astype(np.float64) - ref_n.astype(np.float16).astype(np.float64))
    assert np.all(dn <= ulp16(ref_n)), float(np.max(dn / ulp16(ref_n)))
    check_chain(ctx, s, t, hl, h16, got_h, got_n, gi)


def test_f16_block_given_normed_input(unit_layer):
    """norm_w NULL: `normed` is the caller's d_normed2 and is not written."""
    s, t, hl = unit_layer
    T = 4
    ctx = B.MoeContext(s, max_tokens=T)
    h16, _ = inputs(T, s.hidden, 55)
    n16 = np.random.default_rng(56).standard_normal((T, s.hidden)).astype(np.float16)
    got_h, got_n, gi = run_f16(ctx, t, h16, n16, None)
    assert np.array_equal(got_n.view(np.uint16), n16.view(np.uint16))
    check_chain(ctx, s, t, hl, h16, got_h, n16, gi)


def test_f16_block_rejects_bad_arguments(unit_layer):
    s, t, _ = unit_layer
    ctx = B.MoeContext(s, max_tokens=2)
    h = torch.zeros((4, s.hidden), dtype=torch.float16, device=DEV)
    with pytest.raises(B.BreadError):
        ctx.forward_f16(t.desc(), h, h.clone(), 4)  # more tokens than the context holds
    odd = torch.zeros(2 * s.hidden + 8, dtype=torch.float16, device=DEV)[1:1 + 2 * s.hidden]
    with pytest.raises(B.BreadError):
        ctx.forward_f16(t.desc(), odd, h.clone(), 2)  # misaligned hidden
