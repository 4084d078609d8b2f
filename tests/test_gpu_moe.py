"""GPU parity of routing and the MoE layer against the CPU oracle.

Tier 1: routed expert indices bit-exact (rank order), ties to the lower index.
Tier 2: layer output within 1e-3 relative L2 and 1e-2 max-abs of the oracle's
fp32 computation on the same seeded inputs.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

from helpers import (MAX_ABS_TOL, REL_L2_TOL, arena_host_layer, assert_moe_close, host_layer, max_abs,
                     rel_l2, scale_layer_d)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def full_layer():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=1234, layer=0)
    torch.cuda.synchronize()
    return s, t, host_layer(t)


def xs(n_tokens: int, H: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((n_tokens, H)).astype(np.float32)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def run_forward(ctx, t, x: np.ndarray, hidden: np.ndarray):
    T = x.shape[0]
    xd, hd = dev(x), dev(hidden)
    idx, w, g = ctx.forward(t.desc(), xd, hd, T, want_routing=True)
    torch.cuda.synchronize()
    return hd.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), g.cpu().numpy()


def oracle_forward(hl, x: np.ndarray, hidden: np.ndarray):
    h = np.array(hidden, np.float32, copy=True)
    idx, w, g = O.moe_forward(hl, x, h, x.shape[0], nthreads=8)
    return h, idx, w, g


# ------------------------------------------------------------------ routing


def test_route_matches_oracle(full_layer):
    s, t, hl = full_layer
    T = 48
    x = xs(T, s.hidden, 1)
    ctx = B.MoeContext(s, max_tokens=T)
    idx, w, g = ctx.route(t.desc(), dev(x), T)
    torch.cuda.synchronize()
    idx, w, g = idx.cpu().numpy(), w.cpu().numpy(), g.cpu().numpy()
    for i in range(T):
        ri, rw, rg = O.route(hl, x[i])
        assert np.array_equal(idx[i], ri), f"token {i}: {idx[i]} vs {ri}"
        np.testing.assert_allclose(w[i], rw, rtol=2e-5, atol=1e-7)
        np.testing.assert_allclose(g[i], rg, rtol=1e-4, atol=1e-5)
        assert abs(float(np.sum(w[i], dtype=np.float64)) - 1.0) < 1e-5


def test_route_ties_go_to_lower_index(full_layer):
    """Identical router rows give bit-identical logits; the lower index must
    rank first (layer_ops.cu:241 strict '>' scan).  Covers a tie inside the
    top-K and a tie straddling the K/K+1 boundary."""
    s, t, _ = full_layer
    router = t.router.clone().view(s.n_experts, s.hidden)
    x = xs(1, s.hidden, 2)[0]
    xd = dev(x)
    base = torch.from_numpy(x / np.linalg.norm(x)).to(DEV)
    # experts 200 and 7 share a strong row; 150 and 3 share a weaker one
    router[200] = 3.0 * base
    router[7] = 3.0 * base
    router[150] = 1.5 * base
    router[3] = 1.5 * base
    lt = api.LayerTensors(s, t.gate_exps, t.up_exps, t.down_exps, t.gate_sh, t.up_sh, t.down_sh,
                          router.contiguous().view(-1), t.shgate)
    ctx = B.MoeContext(s, max_tokens=1)
    idx, w, g = ctx.route(lt.desc(), xd, 1)
    torch.cuda.synchronize()
    idx = idx.cpu().numpy()[0]
    assert list(idx[:4]) == [7, 200, 3, 150]
    hl = O.HostLayer(O.OShape(s.hidden, s.expert_inter, s.shared_inter, s.n_experts, s.top_k),
                     np.zeros(1, np.uint8), np.zeros(1, np.uint8), np.zeros(1, np.uint8), np.zeros(1, np.uint8),
                     np.zeros(1, np.uint8), np.zeros(1, np.uint8), router.cpu().numpy(),
                     t.shgate.cpu().numpy().view(np.uint16))
    ri, rw, _ = O.route(hl, x)
    assert np.array_equal(idx, ri)


def test_route_boundary_tie_k():
    """A K=2 selection where ranks 2 and 3 tie exactly: the lower index is in."""
    s = api.shape(hidden=512, expert_inter=256, shared_inter=256, n_experts=16, top_k=2)
    t = api.synth_layer_tensors(s, seed=77)
    router = torch.zeros(16, 512, device=DEV)
    x = np.ones(512, np.float32)
    router[9, :] = 0.01
    router[12, :] = 0.005
    router[4, :] = 0.005  # ties with 12: 4 must win
    t.router.copy_(router.view(-1))
    ctx = B.MoeContext(s, max_tokens=1)
    idx, w, _ = ctx.route(t.desc(), dev(x[None]), 1)
    torch.cuda.synchronize()
    assert list(idx.cpu().numpy()[0]) == [9, 4]


def test_route_nan_rule(full_layer):
    """A NaN logit makes every probability NaN; the defined rule takes the
    lowest unused indices 0..K-1 in order (the oracle's rule)."""
    s, t, hl = full_layer
    x = xs(1, s.hidden, 3)
    x[0, 5] = np.nan
    ctx = B.MoeContext(s, max_tokens=1)
    idx, w, _ = ctx.route(t.desc(), dev(x), 1)
    torch.cuda.synchronize()
    ri, rw, _ = O.route(hl, x[0])
    assert list(ri) == list(range(s.top_k))
    assert np.array_equal(idx.cpu().numpy()[0], ri)
    assert np.all(np.isnan(w.cpu().numpy()))


def test_route_layer_shim(full_layer):
    s, t, hl = full_layer
    x = xs(1, s.hidden, 4)
    ctx = B.MoeContext(s, max_tokens=1)
    hi, hw, hg = ctx.route_layer(t.desc(), dev(x))
    ri, rw, rg = O.route(hl, x[0])
    assert hi == list(ri)
    np.testing.assert_allclose(hw, rw, rtol=2e-5)
    np.testing.assert_allclose(hg, rg, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("seed", [5, 6, 7])
def test_route_layer_f16_shim(full_layer, seed):
    """The reference's route_layer input is fp16 d_normed2 (one_layer.cu:937-961):
    the shim widens it on the device; routing must equal the oracle's on the
    widened (exact) fp32 values, and the raw shared-gate logit is returned."""
    s, t, hl = full_layer
    x16 = xs(1, s.hidden, seed)[0].astype(np.float16)
    ctx = B.MoeContext(s, max_tokens=1)
    hi, hw, hg = ctx.route_layer_f16(t.desc(), torch.from_numpy(x16).to(DEV))
    ri, rw, rg = O.route(hl, x16.astype(np.float32))
    assert hi == list(ri)
    np.testing.assert_allclose(hw, rw, rtol=2e-5)
    np.testing.assert_allclose(hg, rg, rtol=1e-4, atol=1e-5)
    assert ctx.check_device() == 0


def test_route_layer_f16_rejects_misaligned(full_layer):
    s, t, _ = full_layer
    ctx = B.MoeContext(s, max_tokens=1)
    buf = torch.zeros(s.hidden + 8, dtype=torch.float16, device=DEV)
    with pytest.raises(B.BreadError) as e:
        ctx.route_layer_f16(t.desc(), buf[1:s.hidden + 1])
    assert e.value.status == api._lib.ERR_ALIGN


# ------------------------------------------------------------------ MoE layer


def test_decode_layer_matches_oracle(full_layer):
    """Config 2: one decode token through the single-launch kernel."""
    s, t, hl = full_layer
    ctx = B.MoeContext(s, max_tokens=1)
    for seed in range(4):
        x = xs(1, s.hidden, 100 + seed)
        hidden = np.zeros((1, s.hidden), np.float32) if seed % 2 == 0 else xs(1, s.hidden, 200 + seed)
        got, gi, gw, gg = run_forward(ctx, t, x, hidden)
        ref, ri, rw, rg = oracle_forward(hl, x, hidden)
        assert np.array_equal(gi, ri)
        np.testing.assert_allclose(gw, rw, rtol=2e-5, atol=1e-7)
        rl2 = assert_moe_close(got, ref, base=hidden)
        # far tighter than the contract: fp32 except the gate/up dots, whose
        # activations are 16-bit block fixed point (~3e-5 of the layer output)
        assert rl2 < 1e-4
    assert ctx.check_device() == 0


def test_decode_back_to_back_launches(full_layer):
    """The decode kernel resets its own sync block: many launches in a row,
    alternating inputs, each equal to its single-launch result bit for bit."""
    s, t, _ = full_layer
    ctx = B.MoeContext(s, max_tokens=1)
    x0, x1 = dev(xs(1, s.hidden, 5)), dev(xs(1, s.hidden, 6))
    outs = []
    for x in (x0, x1):
        h = torch.zeros(1, s.hidden, device=DEV)
        ctx.forward(t.desc(), x, h, 1)
        outs.append(h.clone())
    hs = [torch.zeros(1, s.hidden, device=DEV) for _ in range(20)]
    for i, h in enumerate(hs):
        ctx.forward(t.desc(), x0 if i % 2 == 0 else x1, h, 1)
    torch.cuda.synchronize()
    for i, h in enumerate(hs):
        assert torch.equal(h, outs[i % 2]), f"launch {i}"
    assert ctx.check_device() == 0


def test_decode_vs_multi_kernel_path(full_layer):
    """The single-launch kernel (fp32 but for 16-bit fixed-point gate/up
    activations) and the per-token kernels (fp32) agree to ~3e-5; the grouped
    path (fp16 operands) to the layer tolerance."""
    s, t, _ = full_layer
    ctx = B.MoeContext(s, max_tokens=2)
    x = xs(1, s.hidden, 8)
    h1 = torch.zeros(1, s.hidden, device=DEV)
    ctx.forward(t.desc(), dev(x), h1, 1)
    ctx.set_path(api.PATH_PER_TOKEN)
    h2 = torch.zeros(2, s.hidden, device=DEV)
    ctx.forward(t.desc(), dev(np.repeat(x, 2, 0)), h2, 2)
    ctx.set_path(api.PATH_GROUPED)
    h3 = torch.zeros(2, s.hidden, device=DEV)
    ctx.forward(t.desc(), dev(np.repeat(x, 2, 0)), h3, 2)
    torch.cuda.synchronize()
    a, b, c = h1.cpu().numpy()[0], h2.cpu().numpy(), h3.cpu().numpy()
    assert np.array_equal(b[0], b[1])
    assert rel_l2(a, b[0]) < 1e-4
    assert np.array_equal(c[0], c[1])
    assert_moe_close(c[0], a)


@pytest.mark.parametrize("path", [api.PATH_AUTO, api.PATH_PER_TOKEN])
@pytest.mark.parametrize("T", [2, 8, 16])
def test_multi_token_matches_oracle(full_layer, T, path):
    """AUTO runs the small-batch path at these sizes (up to
    bread_small_auto_tokens() = 16 tokens); PER_TOKEN the GEMV kernels."""
    s, t, hl = full_layer
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    x = xs(T, s.hidden, 300 + T)
    hidden = xs(T, s.hidden, 400 + T)
    got, gi, gw, _ = run_forward(ctx, t, x, hidden)
    ref, ri, rw, _ = oracle_forward(hl, x, hidden)
    assert np.array_equal(gi, ri)
    assert_moe_close(got, ref, base=hidden)


@pytest.mark.parametrize("H,I,E,K,T", [(512, 256, 16, 2, 1), (512, 256, 16, 2, 3), (768, 512, 32, 1, 2),
                                       (2048, 512, 64, 4, 1)])
def test_other_shapes_match_oracle(H, I, E, K, T):
    """Shapes the single-launch kernel is not built for run the multi-kernel
    path; K = 1 reduces the combine to one routed expert."""
    s = api.shape(hidden=H, expert_inter=I, shared_inter=I, n_experts=E, top_k=K)
    t = api.synth_layer_tensors(s, seed=H + E + K)
    hl = host_layer(t)
    ctx = B.MoeContext(s, max_tokens=T)
    x = xs(T, H, E)
    hidden = np.zeros((T, H), np.float32)
    got, gi, _, _ = run_forward(ctx, t, x, hidden)
    ref, ri, _, _ = oracle_forward(hl, x, hidden)
    assert np.array_equal(gi, ri)
    assert_moe_close(got, ref)


def test_unit_scale_raw_max_abs():
    """With superblock scales divided by 64 the layer output is of order one
    and the raw bounds apply: rel L2 < 1e-3 and max |err| < 1e-2."""
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=555)
    scale_layer_d(t, 6)
    hl = host_layer(t)
    ctx = B.MoeContext(s, max_tokens=4)
    for T in (1, 4):
        x = xs(T, s.hidden, 600 + T)
        hidden = np.zeros((T, s.hidden), np.float32)
        got, gi, _, _ = run_forward(ctx, t, x, hidden)
        ref, ri, _, _ = oracle_forward(hl, x, hidden)
        assert np.array_equal(gi, ri)
        assert 0.1 < float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) < 1e3
        assert rel_l2(got, ref) < REL_L2_TOL
        assert max_abs(got, ref) < MAX_ABS_TOL


def test_null_shared_gate(full_layer):
    """No ffn_gate_inp_shexp tensor: logit 0, shared weight sigmoid(0) = 0.5
    (one_layer.cu:974-976)."""
    s, t, _ = full_layer
    lt = api.LayerTensors(s, t.gate_exps, t.up_exps, t.down_exps, t.gate_sh, t.up_sh, t.down_sh, t.router, None)
    hl = host_layer(t, drop_shgate=True)
    ctx = B.MoeContext(s, max_tokens=1)
    x = xs(1, s.hidden, 9)
    hidden = np.zeros((1, s.hidden), np.float32)
    hd = dev(hidden)
    _, _, g = ctx.forward(lt.desc(), dev(x), hd, 1, want_routing=True)
    torch.cuda.synchronize()
    ref, _, _, rg = oracle_forward(hl, x, hidden)
    assert g.item() == 0.0 and rg[0] == 0.0
    assert_moe_close(hd.cpu().numpy(), ref)


def test_rmsnorm_matches_oracle():
    H, T = 2048, 3
    x = xs(T, H, 10) * 3.0
    w = np.random.default_rng(11).uniform(0.5, 1.5, H).astype(np.float32)
    out = torch.empty(T, H, device=DEV)
    api.bread_rmsnorm_f32(dev(x), dev(w), out, H, T, 1e-6)
    torch.cuda.synchronize()
    for i in range(T):
        ref = O.rms_norm_weighted(x[i], w, 1e-6)
        np.testing.assert_allclose(out[i].cpu().numpy(), ref, rtol=2e-6, atol=1e-7)


def test_stack_small_matches_oracle():
    """Config 3 in miniature: h <- h + MoE_l(RMSNorm(h)) over 3 distinct
    layers of the HBM arena at the full layer shape, 2 steps."""
    s = api.shape()
    L = 3
    arena = B.Arena(s, L)
    for l in range(L):
        arena.synth_layer(l, seed=99, router_std=1.0 / np.sqrt(s.hidden))
    torch.cuda.synchronize()
    hls = [arena_host_layer(s, arena.layer(l)) for l in range(L)]
    ctx = B.MoeContext(s, max_tokens=1)
    h = xs(1, s.hidden, 12)
    hd = dev(h)
    xn = torch.empty_like(hd)
    href = h[0].copy()
    ones = np.ones(s.hidden, np.float32)
    for step in range(2):
        for l in range(L):
            api.bread_rmsnorm_f32(hd, None, xn, s.hidden, 1, 1e-6)
            ctx.forward(arena.layer(l), xn, hd, 1)
            xr = O.rms_norm_weighted(href, ones, 1e-6)
            hh = href[None].copy()
            O.moe_forward(hls[l], xr[None], hh, 1)
            href = hh[0]
    torch.cuda.synchronize()
    got = hd.cpu().numpy()[0]
    assert_moe_close(got, href, base=h[0])
    arena.close()


def test_decode_layers_stack_matches_oracle():
    """Config 3 in one launch per token: h <- h + MoE_l(RMSNorm(h) * w_l) over
    4 arena layers with non-unit norm weights, for 2 tokens; single-layer
    launches in between keep the context's counters in step (the kernel's
    counters and tags only grow, indexed by the context's layer epoch)."""
    s = api.shape()
    L = 4
    arena = B.Arena(s, L)
    for l in range(L):
        arena.synth_layer(l, seed=77, router_std=1.0 / np.sqrt(s.hidden))
    rng = np.random.default_rng(13)
    nws = [rng.uniform(0.5, 1.5, s.hidden).astype(np.float32) for _ in range(L)]
    nwd = [dev(w) for w in nws]
    descs = []
    for l in range(L):
        d = arena.layer(l)
        d.post_norm_w = nwd[l].data_ptr()
        descs.append(d)
    torch.cuda.synchronize()
    hls = [arena_host_layer(s, arena.layer(l)) for l in range(L)]
    ctx = B.MoeContext(s, max_tokens=1)
    h0 = xs(1, s.hidden, 14)[0]
    hd = dev(h0[None])
    href = h0.copy()
    for step in range(2):
        idx, w, _ = ctx.decode_layers(descs, hd, want_routing=True)
        torch.cuda.synchronize()
        ridx = []
        for l in range(L):
            xr = O.rms_norm_weighted(href, nws[l], s.rms_eps)
            hh = href[None].copy()
            ri, rw, _ = O.moe_forward(hls[l], xr[None], hh, 1)
            ridx.append(ri[0])
            href = hh[0]
        assert np.array_equal(idx.cpu().numpy(), np.stack(ridx)), f"step {step}"
        assert_moe_close(hd.cpu().numpy()[0], href, base=h0)
        # a single-layer launch on the same context between stack launches
        xo = dev(xs(1, s.hidden, 15))
        ho = torch.zeros(1, s.hidden, device=DEV)
        ctx.forward(descs[0], xo, ho, 1)
        torch.cuda.synchronize()
        ref1 = np.zeros((1, s.hidden), np.float32)
        O.moe_forward(hls[0], xo.cpu().numpy(), ref1, 1)
        assert_moe_close(ho.cpu().numpy(), ref1)
    assert ctx.check_device() == 0
    arena.close()


def _tie_router(s, t, x, groups):
    """Router with all rows zero except `groups`: (scale, [experts]) rows set
    to scale * x / |x| (identical rows give bit-identical logits)."""
    router = torch.zeros(s.n_experts, s.hidden, device=DEV)
    base = torch.from_numpy(x / np.linalg.norm(x)).to(DEV)
    for scale, experts in groups:
        for e in experts:
            router[e] = scale * base
    return api.LayerTensors(s, t.gate_exps, t.up_exps, t.down_exps, t.gate_sh, t.up_sh, t.down_sh,
                            router.contiguous().view(-1), t.shgate)


def _oracle_route_only(s, lt, x):
    hl = O.HostLayer(O.OShape(s.hidden, s.expert_inter, s.shared_inter, s.n_experts, s.top_k),
                     np.zeros(1, np.uint8), np.zeros(1, np.uint8), np.zeros(1, np.uint8), np.zeros(1, np.uint8),
                     np.zeros(1, np.uint8), np.zeros(1, np.uint8), lt.router.cpu().numpy(),
                     lt.shgate.cpu().numpy().view(np.uint16))
    return O.route(hl, x)


def test_decode_routing_ties(full_layer):
    """The decode kernel's own selection: ties inside the top-8 and a five-way
    tie across the rank-8 boundary go to the lower indices, in rank order."""
    s, t, _ = full_layer
    x = xs(1, s.hidden, 21)[0]
    lt = _tie_router(s, t, x, [(3.0, [200, 7]), (1.5, [150, 3]), (1.0, [250, 31, 90, 17, 5])])
    ctx = B.MoeContext(s, max_tokens=1)
    h = torch.zeros(1, s.hidden, device=DEV)
    idx, w, _ = ctx.forward(lt.desc(), dev(x[None]), h, 1, want_routing=True)
    torch.cuda.synchronize()
    got = list(idx.cpu().numpy()[0])
    assert got == [7, 200, 3, 150, 5, 17, 31, 90]
    ri, rw, _ = _oracle_route_only(s, lt, x)
    assert got == list(ri)
    np.testing.assert_allclose(w.cpu().numpy()[0], rw, rtol=2e-5, atol=1e-7)
    assert ctx.check_device() == 0


def test_decode_routing_nan_rule(full_layer):
    """A NaN input makes every probability NaN: indices 0..K-1 in order."""
    s, t, hl = full_layer
    x = xs(1, s.hidden, 22)
    x[0, 11] = np.nan
    ctx = B.MoeContext(s, max_tokens=1)
    h = torch.zeros(1, s.hidden, device=DEV)
    idx, w, _ = ctx.forward(t.desc(), dev(x), h, 1, want_routing=True)
    torch.cuda.synchronize()
    ri, _, _ = O.route(hl, x[0])
    assert list(idx.cpu().numpy()[0]) == list(ri) == list(range(s.top_k))
    assert np.all(np.isnan(w.cpu().numpy()))
    # the context keeps working after a NaN token
    h2 = torch.zeros(1, s.hidden, device=DEV)
    x2 = xs(1, s.hidden, 23)
    idx2, _, _ = ctx.forward(t.desc(), dev(x2), h2, 1, want_routing=True)
    torch.cuda.synchronize()
    ref = np.zeros((1, s.hidden), np.float32)
    ri2, _, _ = O.moe_forward(hl, x2, ref, 1, nthreads=8)
    assert np.array_equal(idx2.cpu().numpy(), ri2)
    assert_moe_close(h2.cpu().numpy(), ref)
    assert ctx.check_device() == 0


@pytest.mark.parametrize("E,K", [(16, 1), (16, 2), (256, 3), (40, 8)])
def test_decode_small_k_matches_oracle(E, K):
    """The decode kernel at H 2048 / I 512 with other expert counts and K."""
    s = api.shape(n_experts=E, top_k=K)
    t = api.synth_layer_tensors(s, seed=E * 10 + K)
    hl = host_layer(t)
    ctx = B.MoeContext(s, max_tokens=1)
    for seed in range(3):
        x = xs(1, s.hidden, 700 + seed)
        hidden = xs(1, s.hidden, 800 + seed)
        got, gi, gw, _ = run_forward(ctx, t, x, hidden)
        ref, ri, rw, _ = oracle_forward(hl, x, hidden)
        assert np.array_equal(gi, ri)
        np.testing.assert_allclose(gw, rw, rtol=2e-5, atol=1e-7)
        assert_moe_close(got, ref, base=hidden)
    assert ctx.check_device() == 0
