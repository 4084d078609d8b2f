"""GPU parity of the grouped multi-token path (tokens bucketed by expert,
expert GEMMs on the matrix cores) against the CPU oracle.

The oracle is the per-token MoE block (one_layer.cu:1413-1471) applied to
every token, so each case checks routing bit-exactly (indices in rank order)
and the layer output within 1e-3 relative L2 and 1e-2 max-abs, for the
batch shapes of batched decode / speculative verify (B = 8, 16, 64 with
Zipf-skewed routing) and of a 512-token prefill chunk (uniform and Zipf),
plus ragged and skewed edge cases: experts spanning several 16-pair tiles,
every token on the same experts, a different shared-expert width, and a
residual that is not zero.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import _lib, api, synth
from oracle import oracle as O

from helpers import MAX_ABS_TOL, REL_L2_TOL, assert_moe_close, host_layer, max_abs, rel_l2, scale_layer_d

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture(scope="module")
def full_layer():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=4321, layer=0)
    torch.cuda.synchronize()
    return s, t, host_layer(t)


@pytest.fixture(scope="module")
def zipf_layer(full_layer):
    """The full layer with the router's last column set to a Zipf(1.1) bias
    (tokens carry a constant 1 in their last feature)."""
    s, t, _ = full_layer
    router = t.router.clone().view(s.n_experts, s.hidden)
    router[:, -1] = dev(synth.zipf_bias(s.n_experts, 1.1, seed=99))
    lt = api.LayerTensors(s, t.gate_exps, t.up_exps, t.down_exps, t.gate_sh, t.up_sh, t.down_sh,
                          router.contiguous().view(-1), t.shgate)
    torch.cuda.synchronize()
    return s, lt, host_layer(lt)


def tokens(T: int, H: int, seed: int, zipf: bool) -> np.ndarray:
    x = np.random.default_rng(seed).standard_normal((T, H)).astype(np.float32)
    if zipf:
        x[:, -1] = 1.0
    return x


def run(s, t, x, hidden, path=api.PATH_GROUPED):
    T = x.shape[0]
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    hd = dev(hidden)
    idx, w, g = ctx.forward(t.desc(), dev(x), hd, T, want_routing=True)
    torch.cuda.synchronize()
    return hd.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), g.cpu().numpy()


def check(hl, x, hidden, got):
    out, idx, w, g = got
    ref = np.array(hidden, np.float32, copy=True)
    ridx, rw, rg = O.moe_forward(hl, x, ref, x.shape[0], nthreads=16)
    ridx = np.asarray(ridx).reshape(idx.shape)
    bad = np.nonzero(np.any(idx != ridx, axis=1))[0]
    assert bad.size == 0, f"routing differs at tokens {bad[:8]}: {idx[bad[0]]} vs {ridx[bad[0]]}"
    np.testing.assert_allclose(w, np.asarray(rw).reshape(w.shape), rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose(g, np.asarray(rg).reshape(g.shape), rtol=1e-4, atol=1e-4)
    return assert_moe_close(out, ref, base=hidden)


def distinct_experts(idx) -> int:
    return int(np.unique(idx).size)


@pytest.mark.parametrize("T", [8, 16, 64, 128, 129])
def test_grouped_batched_decode_zipf(zipf_layer, T):
    """Config 4: B tokens, Zipf-skewed routing (expert reuse across tokens).
    64 and 128 tokens fill one and two 64-token router tiles; 129 starts a
    third."""
    s, t, hl = zipf_layer
    x = tokens(T, s.hidden, 100 + T, zipf=True)
    hidden = np.zeros_like(x)
    got = run(s, t, x, hidden)
    check(hl, x, hidden, got)
    assert distinct_experts(got[1]) < T * s.top_k  # reuse happened


@pytest.mark.parametrize("zipf", [False, True])
def test_grouped_prefill_chunk(full_layer, zipf_layer, zipf):
    """Config 5: a 512-token prefill chunk, uniform and Zipf routing; under
    Zipf the top experts take several hundred tokens (many 16-pair tiles)."""
    s, t, hl = zipf_layer if zipf else full_layer
    x = tokens(512, s.hidden, 7, zipf=zipf)
    hidden = np.random.default_rng(8).standard_normal(x.shape).astype(np.float32)
    got = run(s, t, x, hidden)
    check(hl, x, hidden, got)
    counts = np.bincount(got[1].reshape(-1), minlength=s.n_experts)
    if zipf:
        assert counts.max() > 4 * 16


@pytest.mark.parametrize("T", [80, 300])
def test_grouped_all_tokens_same_experts(full_layer, T):
    """Identical tokens: K experts take every token (T/32 tiles each; at 300
    tokens ten tiles, split into segments of four tiles on different XCDs'
    work lists)."""
    s, t, hl = full_layer
    x = np.repeat(tokens(1, s.hidden, 11, zipf=False), T, axis=0)
    hidden = np.zeros_like(x)
    got = run(s, t, x, hidden)
    assert distinct_experts(got[1]) == s.top_k
    check(hl, x, hidden, got)


def test_grouped_two_tokens_forced(full_layer):
    """n_tokens = 2 on the grouped path, forced (AUTO takes the small-batch
    path up to bread_small_auto_tokens() tokens)."""
    s, t, hl = full_layer
    x = tokens(2, s.hidden, 12, zipf=False)
    hidden = np.zeros_like(x)
    check(hl, x, hidden, run(s, t, x, hidden, path=api.PATH_GROUPED))


@pytest.mark.parametrize("T", [17, 18])
def test_auto_hands_off_to_grouped(full_layer, T):
    """Just above bread_small_auto_tokens() tokens PATH_AUTO takes the grouped
    path; the result still meets the oracle."""
    s, t, hl = full_layer
    assert T > B.lib.bread_small_auto_tokens()
    x = tokens(T, s.hidden, 40 + T, zipf=False)
    hidden = np.zeros_like(x)
    check(hl, x, hidden, run(s, t, x, hidden, path=api.PATH_AUTO))


def test_grouped_single_token_forced(full_layer):
    s, t, hl = full_layer
    x = tokens(1, s.hidden, 13, zipf=False)
    hidden = np.zeros_like(x)
    check(hl, x, hidden, run(s, t, x, hidden))


@pytest.mark.parametrize("dims", [(512, 256, 256, 16, 2, 37), (1024, 256, 512, 40, 4, 29),
                                  (768, 512, 256, 64, 8, 50)])
def test_grouped_small_shapes(dims):
    """Ragged token counts, other hidden / intermediate sizes (shared wider or
    narrower than the routed experts), fewer experts, smaller K."""
    H, I, Ish, E, K, T = dims
    s = api.shape(hidden=H, expert_inter=I, shared_inter=Ish, n_experts=E, top_k=K)
    t = api.synth_layer_tensors(s, seed=5 + E, layer=0)
    torch.cuda.synchronize()
    hl = host_layer(t)
    x = tokens(T, H, 21 + T, zipf=False)
    hidden = np.random.default_rng(3).standard_normal(x.shape).astype(np.float32)
    check(hl, x, hidden, run(s, t, x, hidden))


def test_grouped_matches_per_token_path(full_layer):
    """The grouped and per-token device paths agree to the same tolerance."""
    s, t, _ = full_layer
    x = tokens(24, s.hidden, 31, zipf=False)
    hidden = np.zeros_like(x)
    a = run(s, t, x, hidden, path=api.PATH_GROUPED)
    b = run(s, t, x, hidden, path=api.PATH_PER_TOKEN)
    assert np.array_equal(a[1], b[1])
    assert_moe_close(a[0], b[0])


def test_grouped_repeat_is_bitwise_stable(full_layer):
    """Pair order inside an expert's bucket comes from atomics; each pair's
    result does not depend on it, so repeated runs agree bit for bit."""
    s, t, _ = full_layer
    x = tokens(64, s.hidden, 41, zipf=False)
    hidden = np.zeros_like(x)
    a = run(s, t, x, hidden)[0]
    b = run(s, t, x, hidden)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_grouped_unit_scale_raw_bounds():
    """Superblock scales divided by 64: outputs of order one, where the raw
    bounds apply (rel L2 < 1e-3, max |err| < 1e-2) without normalisation."""
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=556)
    scale_layer_d(t, 6)
    torch.cuda.synchronize()
    hl = host_layer(t)
    x = tokens(64, s.hidden, 57, zipf=False)
    hidden = np.zeros_like(x)
    got = run(s, t, x, hidden)
    ref = np.array(hidden, copy=True)
    ridx, _, _ = O.moe_forward(hl, x, ref, 64, nthreads=16)
    assert np.array_equal(got[1], ridx)
    assert 0.1 < float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) < 1e3
    assert rel_l2(got[0], ref) < REL_L2_TOL
    assert max_abs(got[0], ref) < MAX_ABS_TOL


def test_grouped_null_shared_gate(full_layer):
    """No shared-gate tensor: logit 0, shared weight sigmoid(0) = 0.5."""
    s, t, _ = full_layer
    lt = api.LayerTensors(s, t.gate_exps, t.up_exps, t.down_exps, t.gate_sh, t.up_sh, t.down_sh, t.router, None)
    hl = host_layer(t, drop_shgate=True)
    x = tokens(8, s.hidden, 58, zipf=False)
    hidden = np.zeros_like(x)
    got = run(s, lt, x, hidden)
    assert np.all(got[3] == 0.0)
    check(hl, x, hidden, got)


def _gate_d(t, s, expert: int, d: float):
    """Set d of every Q4_K superblock of one expert's gate matrix."""
    g = t.gate_exps.cpu().numpy().reshape(s.n_experts, -1)
    blocks = g[expert].reshape(-1, 144)
    blocks[:, 0:2] = np.array([d], np.float16).view(np.uint8)
    g[expert] = blocks.reshape(-1)
    t.gate_exps.copy_(torch.from_numpy(g.reshape(-1)))
    torch.cuda.synchronize()


def test_grouped_large_scales_near_fp16_limit():
    """d = 32: dequantised gate weights up to 32 * 63 * 15 = 30240, inside
    fp16's range; the packed-fp16 dequant stays exact in sc * q."""
    s = api.shape(hidden=512, expert_inter=256, shared_inter=256, n_experts=16, top_k=2)
    t = api.synth_layer_tensors(s, seed=91, layer=0)
    _gate_d(t, s, 3, 32.0)
    hl = host_layer(t)
    x = tokens(64, s.hidden, 92, zipf=False)
    hidden = np.zeros_like(x)
    got = run(s, t, x, hidden)
    assert np.any(got[1] == 3), "expert 3 not routed; pick another seed"
    check(hl, x, hidden, got)


def test_grouped_weights_beyond_fp16_flag_device_error():
    """d = 100 puts dequantised weights beyond fp16's range (the grouped
    path's operand type): the call completes and bread_moe_ctx_check reports
    BREAD_ERR_DEVICE with the range bit (4) set."""
    s = api.shape(hidden=512, expert_inter=256, shared_inter=256, n_experts=16, top_k=2)
    t = api.synth_layer_tensors(s, seed=91, layer=0)
    _gate_d(t, s, 3, 100.0)
    x = tokens(64, s.hidden, 92, zipf=False)
    ctx = B.MoeContext(s, max_tokens=64)
    ctx.set_path(api.PATH_GROUPED)
    idx, _, _ = ctx.forward(t.desc(), dev(x), dev(np.zeros_like(x)), 64, want_routing=True)
    torch.cuda.synchronize()
    assert np.any(idx.cpu().numpy() == 3)
    with pytest.raises(B.BreadError) as ei:
        ctx.check_device()
    assert ei.value.status == _lib.ERR_DEVICE
    ctx.check_device()  # cleared
