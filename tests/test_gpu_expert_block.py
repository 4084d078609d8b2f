"""GPU parity of bread_moe_expert_block: the routed experts with the
caller's routing, no router and no shared expert, the block the reference's
expert benchmark times (bread_benchmark_expert_block, expert_bench.cu:60-239:
experts 0..7, weights 1/8, input x_i = 0.5 sin(0.013 i) + 0.5 cos(0.007 (i +
11)), :45-51).  Against the oracle (oracle.expert_block, the same matvecs,
SwiGLU and rank-order accumulation): 1e-3 relative L2 and 1e-2 max-abs.
Also: several tokens with repeated experts and a nonzero residual, a mixed
Q4_K / Q6_K layer, bit-identical repeats, and an out-of-range index, which is
clamped (no load leaves the tensor) and flagged in the error word.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

from helpers import assert_moe_close, host_layer

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bench_input(H):
    """fill_input of expert_bench.cu:45-51 (float arithmetic as there)."""
    i = np.arange(H, dtype=np.float32)
    return (np.float32(0.5) * np.sin(np.float32(0.013) * i) +
            np.float32(0.5) * np.cos(np.float32(0.007) * (i + np.float32(11)))).astype(np.float32)


@pytest.fixture(scope="module")
def layer():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=777, layer=0)
    torch.cuda.synchronize()
    return s, t, host_layer(t)


def run(s, t, x, hidden, idx, w):
    T = x.shape[0]
    ctx = B.MoeContext(s, max_tokens=T)
    hd = dev(hidden)
    ctx.expert_block(t.desc(), dev(x), hd, T, dev(idx), dev(w))
    torch.cuda.synchronize()
    assert ctx.check_device() == 0
    return hd.cpu().numpy()


def test_reference_benchmark_block(layer):
    s, t, hl = layer
    K = s.top_k
    x = bench_input(s.hidden)[None]
    idx = np.arange(K, dtype=np.int32)[None]
    w = np.full((1, K), 1.0 / K, np.float32)
    hidden = np.zeros((1, s.hidden), np.float32)
    got = run(s, t, x, hidden, idx, w)
    ref = hidden.copy()
    O.expert_block(hl, x, ref, idx, w, nthreads=16)
    assert_moe_close(got, ref)
    again = run(s, t, x, hidden, idx, w)
    assert np.array_equal(got, again)


def test_tokens_with_repeated_experts(layer):
    s, t, hl = layer
    K, T = s.top_k, 5
    rng = np.random.default_rng(3)
    x = rng.standard_normal((T, s.hidden)).astype(np.float32)
    idx = rng.integers(0, s.n_experts, (T, K)).astype(np.int32)
    idx[0, 1] = idx[0, 0]
    w = rng.uniform(-1, 1, (T, K)).astype(np.float32)
    hidden = rng.standard_normal((T, s.hidden)).astype(np.float32)
    got = run(s, t, x, hidden, idx, w)
    ref = hidden.copy()
    O.expert_block(hl, x, ref, idx, w, nthreads=16)
    assert_moe_close(got, ref, base=hidden)


def test_mixed_type_layer():
    s = api.shape(hidden=512, expert_inter=256, shared_inter=256, n_experts=16, top_k=4)
    types = (api.QTYPE_Q6_K, api.QTYPE_Q4_K, api.QTYPE_Q4_K, api.QTYPE_Q4_K, api.QTYPE_Q4_K, api.QTYPE_Q6_K)
    t = api.synth_layer_tensors(s, seed=778, layer=0, types=types)
    torch.cuda.synchronize()
    hl = host_layer(t)
    x = bench_input(s.hidden)[None]
    idx = np.array([[15, 3, 3, 0]], np.int32)
    w = np.full((1, 4), 0.25, np.float32)
    hidden = np.zeros((1, s.hidden), np.float32)
    got = run(s, t, x, hidden, idx, w)
    ref = hidden.copy()
    O.expert_block(hl, x, ref, idx, w)
    assert_moe_close(got, ref)


def test_out_of_range_index_is_flagged(layer):
    s, t, _ = layer
    K = s.top_k
    ctx = B.MoeContext(s, max_tokens=1)
    idx = np.arange(K, dtype=np.int32)[None]
    idx[0, 3] = s.n_experts + 5
    idx[0, 5] = -2
    hd = dev(np.zeros((1, s.hidden), np.float32))
    ctx.expert_block(t.desc(), dev(bench_input(s.hidden)[None]), hd, 1, dev(idx),
                     dev(np.full((1, K), 1.0 / K, np.float32)))
    torch.cuda.synchronize()
    with pytest.raises(B.BreadError) as e:
        ctx.check_device()
    assert e.value.status == api._lib.ERR_DEVICE and e.value.device_error == 32
    assert ctx.check_device() == 0
