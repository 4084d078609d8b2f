"""GPU parity of the small-batch path (2..32 tokens: selected experts' rows
streamed over the whole GPU; at the decode shape and up to 16 tokens the
workgroup-per-CU kernels with integer gate/up dots) against the CPU oracle.

The oracle is the per-token MoE block (one_layer.cu:1413-1471) applied to
every token: routing bit-exact (indices in rank order), renormalised weights
and shared-gate logits to the last bits, layer outputs within 1e-3 relative
L2 and 1e-2 max-abs.  Cases: batched decode with Zipf-skewed routing
(B = 8, 16), uniform routing at the path's largest batch (32), two tokens,
every token on the same experts (more tokens per expert than one LDS stage
holds), other hidden / intermediate sizes and expert counts (more than 256
experts takes the wide top-k), a null shared gate, unit-scale weights with
the raw bounds, bit-identical repeats, and its agreement with the per-token
path.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api, synth
from oracle import oracle as O

from helpers import MAX_ABS_TOL, REL_L2_TOL, assert_moe_close, host_layer, max_abs, rel_l2, scale_layer_d

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture(scope="module")
def full_layer():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=8642, layer=0)
    torch.cuda.synchronize()
    return s, t, host_layer(t)


@pytest.fixture(scope="module")
def zipf_layer(full_layer):
    s, t, _ = full_layer
    router = t.router.clone().view(s.n_experts, s.hidden)
    router[:, -1] = dev(synth.zipf_bias(s.n_experts, 1.1, seed=98))
    lt = api.LayerTensors(s, t.gate_exps, t.up_exps, t.down_exps, t.gate_sh, t.up_sh, t.down_sh,
                          router.contiguous().view(-1), t.shgate)
    torch.cuda.synchronize()
    return s, lt, host_layer(lt)


def tokens(T, H, seed, zipf):
    x = np.random.default_rng(seed).standard_normal((T, H)).astype(np.float32)
    if zipf:
        x[:, -1] = 1.0
    return x


def run(s, t, x, hidden, path=api.PATH_SMALL):
    T = x.shape[0]
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    hd = dev(hidden)
    idx, w, g = ctx.forward(t.desc(), dev(x), hd, T, want_routing=True)
    torch.cuda.synchronize()
    assert ctx.check_device() == 0
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


@pytest.mark.parametrize("T", [8, 16])
def test_small_zipf_batches(zipf_layer, T):
    s, t, hl = zipf_layer
    x = tokens(T, s.hidden, 100 + T, zipf=True)
    hidden = np.random.default_rng(T).standard_normal(x.shape).astype(np.float32)
    check(hl, x, hidden, run(s, t, x, hidden))


@pytest.mark.parametrize("T", [2, 7, 32])
def test_small_uniform(full_layer, T):
    s, t, hl = full_layer
    x = tokens(T, s.hidden, 200 + T, zipf=False)
    hidden = np.zeros_like(x)
    check(hl, x, hidden, run(s, t, x, hidden))


def test_small_all_tokens_same_experts(full_layer):
    """32 copies of one token: 8 experts with 32 pairs each (six LDS stages of
    activations in gate/up, two of SwiGLU rows in down)."""
    s, t, hl = full_layer
    x = np.repeat(tokens(1, s.hidden, 7, zipf=False), 32, axis=0)
    hidden = np.random.default_rng(8).standard_normal(x.shape).astype(np.float32)
    out = check(hl, x, hidden, run(s, t, x, hidden))
    del out


@pytest.mark.parametrize("dims", [(512, 256, 256, 16, 2, 5), (1024, 256, 512, 40, 4, 19),
                                  (768, 512, 256, 64, 8, 32), (2048, 512, 512, 300, 8, 12),
                                  (256, 512, 256, 1024, 16, 9), (2048, 256, 512, 1024, 16, 10),
                                  (1024, 512, 256, 96, 12, 3)])
def test_small_other_shapes(dims):
    """Hidden 256..2048 (lanes of superblocks beyond H idle), intermediate 256
    or 512 with the shared expert narrower or wider, E up to 1024 (the wide
    top-k), K up to 16.  Hidden 1024 and 2048 route by certified fast sums
    (1024 experts and top-16 included), the others in the reference's order."""
    H, I, Ish, E, K, T = dims
    s = api.shape(hidden=H, expert_inter=I, shared_inter=Ish, n_experts=E, top_k=K)
    t = api.synth_layer_tensors(s, seed=11 + E, layer=0)
    torch.cuda.synchronize()
    hl = host_layer(t)
    x = tokens(T, H, 31 + T, zipf=False)
    hidden = np.random.default_rng(5).standard_normal(x.shape).astype(np.float32)
    check(hl, x, hidden, run(s, t, x, hidden))


def test_small_wide_hot_experts(full_layer):
    """Decode-shape kernels: 16 copies of one token (every expert of the
    token chosen 16 times: four slots of four pairs each per expert, the
    shared expert too), and a single token."""
    s, t, hl = full_layer
    x = np.repeat(tokens(1, s.hidden, 71, zipf=False), 16, axis=0)
    hidden = np.random.default_rng(72).standard_normal(x.shape).astype(np.float32)
    check(hl, x, hidden, run(s, t, x, hidden))
    x1 = tokens(1, s.hidden, 73, zipf=False)
    check(hl, x1, np.zeros_like(x1), run(s, t, x1, np.zeros_like(x1)))


@pytest.mark.parametrize("E,K,T", [(256, 4, 16), (128, 8, 11), (64, 6, 5), (256, 1, 3)])
def test_small_wide_other_k_e(E, K, T):
    """Decode shape (H 2048, I 512) with other expert counts and top-k."""
    s = api.shape(n_experts=E, top_k=K)
    t = api.synth_layer_tensors(s, seed=500 + E + K, layer=0)
    torch.cuda.synchronize()
    hl = host_layer(t)
    x = tokens(T, s.hidden, 600 + T, zipf=False)
    hidden = np.random.default_rng(601).standard_normal(x.shape).astype(np.float32)
    check(hl, x, hidden, run(s, t, x, hidden))


def test_small_null_shared_gate(full_layer):
    s, t, _ = full_layer
    lt = api.LayerTensors(s, t.gate_exps, t.up_exps, t.down_exps, t.gate_sh, t.up_sh, t.down_sh, t.router, None)
    hl = host_layer(t, drop_shgate=True)
    x = tokens(6, s.hidden, 17, zipf=False)
    hidden = np.zeros_like(x)
    out, idx, w, g = run(s, lt, x, hidden)
    assert np.all(g == 0.0)
    check(hl, x, hidden, (out, idx, w, g))


def test_small_unit_scale_raw_bounds():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=4242)
    scale_layer_d(t, 6)
    hl = host_layer(t)
    x = tokens(12, s.hidden, 9, zipf=False)
    hidden = np.zeros_like(x)
    out, idx, w, g = run(s, t, x, hidden)
    ref = hidden.copy()
    ridx, _, _ = O.moe_forward(hl, x, ref, x.shape[0], nthreads=16)
    assert np.array_equal(idx, np.asarray(ridx).reshape(idx.shape))
    assert 0.1 < float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) < 1e3
    assert rel_l2(out, ref) < REL_L2_TOL
    assert max_abs(out, ref) < MAX_ABS_TOL


def test_small_repeat_is_bitwise_stable(zipf_layer):
    s, t, _ = zipf_layer
    x = tokens(16, s.hidden, 41, zipf=True)
    hidden = np.zeros_like(x)
    a = run(s, t, x, hidden)[0]
    b = run(s, t, x, hidden)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_small_matches_per_token_path(full_layer):
    """Same routing; outputs within ~4e-5 (the small-batch path's gate/up dots
    take 16-bit fixed-point activations at the decode shape; the per-token
    path is fp32)."""
    s, t, _ = full_layer
    x = tokens(24, s.hidden, 51, zipf=False)
    hidden = np.zeros_like(x)
    a = run(s, t, x, hidden, path=api.PATH_SMALL)
    b = run(s, t, x, hidden, path=api.PATH_PER_TOKEN)
    assert np.array_equal(a[1], b[1])
    assert rel_l2(a[0], b[0]) < 1e-4


def test_small_auto_choice(full_layer):
    """AUTO takes the small path for 2..bread_small_auto_tokens() tokens: the
    output equals the forced small path bit for bit."""
    s, t, _ = full_layer
    n = B.lib.bread_small_auto_tokens()
    assert 2 <= n <= 32
    x = tokens(n, s.hidden, 61, zipf=False)
    hidden = np.zeros_like(x)
    a = run(s, t, x, hidden, path=api.PATH_AUTO)[0]
    b = run(s, t, x, hidden, path=api.PATH_SMALL)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_small_rejects_large_batches(full_layer):
    s, t, _ = full_layer
    ctx = B.MoeContext(s, max_tokens=33)
    ctx.set_path(api.PATH_SMALL)
    x = torch.zeros((33, s.hidden), device=DEV)
    h = torch.zeros_like(x)
    with pytest.raises(B.BreadError):
        ctx.forward(t.desc(), x, h, 33)
