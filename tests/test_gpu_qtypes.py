"""GPU parity of per-tensor weight types: each of the six expert tensors
(routed and shared gate, up, down) is Q4_K or Q6_K, as the reference
records per tensor (loader.c:191-193) and dispatches on in its fp32 path
(one_layer.cu:1465-1468 -> layer_ops.cu:169-189, cpu_tensor_matvec).

Against the CPU oracle (which dispatches the same way): routing bit-exact,
outputs within 1e-3 relative L2 and 1e-2 max-abs.  Cases:
  - layouts other than the reference GPU path's (Q4_K gate/up, Q6_K down):
    Q4_K down (the ffn_down mix of Q4_K_M files), all Q6_K, and gate / up /
    down / shared each different, at one token, a small batch and a larger
    one under the automatic choice and pinned to the per-token kernels;
  - pinned decode, small-batch and grouped paths refuse those layouts with
    BREAD_ERR_QTYPE instead of computing them wrongly;
  - a 4-layer stack with mixed layers (arena layers re-laid out by
    bread_arena_set_layer_types) through bread_moe_decode_layers, which
    splits it into decode-kernel runs and per-token layers, and through
    bread_moe_stack_forward for 3 tokens;
  - a GGUF file whose expert tensors mix Q4_K and Q6_K, loaded into the
    arena (the layer takes the file's types) and checked on its tensors.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

import gguf_writer as W
from helpers import arena_host_layer, assert_moe_close, host_layer, oshape

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
Q4, Q6 = api.QTYPE_Q4_K, api.QTYPE_Q6_K
LAYOUTS = {
    "q4_down": (Q4, Q4, Q4, Q4, Q4, Q4),
    "all_q6": (Q6, Q6, Q6, Q6, Q6, Q6),
    "mixed": (Q6, Q4, Q6, Q4, Q6, Q4),
}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def xs(T, H, seed):
    return np.random.default_rng(seed).standard_normal((T, H)).astype(np.float32)


@pytest.fixture(scope="module", params=sorted(LAYOUTS))
def typed_layer(request):
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=500 + len(request.param), layer=0, types=LAYOUTS[request.param])
    torch.cuda.synchronize()
    return request.param, s, t, host_layer(t)


def run(s, d, x, hidden, path):
    T = x.shape[0]
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    hd = dev(hidden)
    idx, _, _ = ctx.forward(d, dev(x), hd, T, want_routing=True)
    torch.cuda.synchronize()
    assert ctx.check_device() == 0
    return hd.cpu().numpy(), idx.cpu().numpy()


@pytest.mark.parametrize("T,path", [(1, api.PATH_AUTO), (3, api.PATH_AUTO), (24, api.PATH_AUTO),
                                    (5, api.PATH_PER_TOKEN)])
def test_typed_layer_matches_oracle(typed_layer, T, path):
    name, s, t, hl = typed_layer
    print(f"layout {name} T={T} path={path}", flush=True)
    x, hidden = xs(T, s.hidden, 10 + T), xs(T, s.hidden, 20 + T)
    got, gi = run(s, t.desc(), x, hidden, path)
    ref = hidden.copy()
    ri, _, _ = O.moe_forward(hl, x, ref, T, nthreads=16)
    assert np.array_equal(gi, np.asarray(ri).reshape(gi.shape))
    assert_moe_close(got, ref, base=hidden)


@pytest.mark.parametrize("path", [api.PATH_DECODE, api.PATH_SMALL, api.PATH_GROUPED])
def test_specialised_paths_refuse_other_layouts(typed_layer, path):
    _, s, t, _ = typed_layer
    T = 1 if path == api.PATH_DECODE else 4
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    with pytest.raises(B.BreadError) as e:
        ctx.forward(t.desc(), dev(xs(T, s.hidden, 3)), dev(xs(T, s.hidden, 4)), T)
    assert e.value.status == api._lib.ERR_QTYPE


def mixed_stack(s, types):
    """Arena layers of the given types with seeded weights and non-unit norm
    weights; returns the arena, the descriptors, oracle_stack(h0), which runs
    the stack on the host (RMSNorm, then the layer) for every row, and the
    device norm weights the descriptors point at (the caller keeps them
    alive while it uses the descriptors)."""
    L = len(types)
    arena = B.Arena(s, L)
    for l in range(L):
        arena.set_layer_types(l, types[l])
        arena.synth_layer(l, seed=91, router_std=1.0 / np.sqrt(s.hidden))
    rng = np.random.default_rng(17)
    nws = [rng.uniform(0.5, 1.5, s.hidden).astype(np.float32) for _ in range(L)]
    nwd = [dev(w) for w in nws]
    descs = []
    for l in range(L):
        d = arena.layer(l)
        assert api.layer_types(d) == tuple(types[l])
        d.post_norm_w = nwd[l].data_ptr()
        descs.append(d)
    torch.cuda.synchronize()
    hls = [arena_host_layer(s, arena.layer(l)) for l in range(L)]

    def oracle_stack(h0):
        h = h0.copy()
        ridx = []
        for l in range(L):
            xr = np.stack([O.rms_norm_weighted(h[t], nws[l], s.rms_eps) for t in range(h.shape[0])])
            ri, _, _ = O.moe_forward(hls[l], xr, h, h.shape[0], nthreads=16)
            ridx.append(np.asarray(ri).reshape(h.shape[0], -1))
        return h, np.stack(ridx)

    return arena, descs, oracle_stack, nwd


def test_mixed_stack_matches_oracle():
    """Layers 0 and 2 have the decode kernel's types, 1 and 3 not: one
    bread_moe_decode_layers call runs layer 0, layer 1 (per-token), layer 2,
    layer 3 (per-token) on one token; then 3 tokens (one stack launch each)
    and bread_stack_loop_tokens() + 1 tokens (batched calls per layer)
    through bread_moe_stack_forward."""
    s = api.shape()
    types = [api.STANDARD_TYPES, LAYOUTS["q4_down"], api.STANDARD_TYPES, LAYOUTS["mixed"]]
    arena, descs, oracle_stack, nwd = mixed_stack(s, types)
    TB = B.lib.bread_stack_loop_tokens() + 1
    ctx = B.MoeContext(s, max_tokens=TB)
    h0 = xs(1, s.hidden, 18)
    hd = dev(h0)
    idx, _, _ = ctx.decode_layers(descs, hd, want_routing=True)
    torch.cuda.synchronize()
    href, ridx = oracle_stack(h0)
    assert np.array_equal(idx.cpu().numpy(), ridx[:, 0])
    assert_moe_close(hd.cpu().numpy(), href, base=h0)

    for T in (3, TB):
        h3 = xs(T, s.hidden, 19 + T)
        hd3 = dev(h3)
        idx3, _, _ = ctx.stack_forward(descs, hd3, T, want_routing=True)
        torch.cuda.synchronize()
        href3, ridx3 = oracle_stack(h3)
        assert np.array_equal(idx3.cpu().numpy().reshape(ridx3.shape), ridx3), T
        assert_moe_close(hd3.cpu().numpy(), href3, base=h3)
    assert ctx.check_device() == 0
    arena.close()
    del nwd


def test_mixed_stack_other_shape_applies_each_layer_once():
    """A stack the decode kernel does not take (hidden 1024) whose first
    layer has other weight types.  The decode-run launcher refuses the whole
    stack before running any layer, so bread_moe_stack_forward's fallback
    (one batched call per layer) starts from the caller's hidden and applies
    every layer once; bread_moe_decode_layers returns BREAD_ERR_SHAPE with
    hidden untouched."""
    s = api.shape(hidden=1024)
    types = [LAYOUTS["q4_down"], api.STANDARD_TYPES, LAYOUTS["mixed"], api.STANDARD_TYPES]
    arena, descs, oracle_stack, nwd = mixed_stack(s, types)
    ctx = B.MoeContext(s, max_tokens=3)
    for T in (1, 3):
        h0 = xs(T, s.hidden, 40 + T)
        hd = dev(h0)
        idx, _, _ = ctx.stack_forward(descs, hd, T, want_routing=True)
        torch.cuda.synchronize()
        href, ridx = oracle_stack(h0)
        assert np.array_equal(idx.cpu().numpy().reshape(ridx.shape), ridx), T
        assert_moe_close(hd.cpu().numpy(), href, base=h0)
    h1 = xs(1, s.hidden, 45)
    hd1 = dev(h1)
    with pytest.raises(B.BreadError) as e:
        ctx.decode_layers(descs, hd1)
    assert e.value.status == api._lib.ERR_SHAPE
    torch.cuda.synchronize()
    assert np.array_equal(hd1.cpu().numpy(), h1)
    assert ctx.check_device() == 0
    arena.close()
    del nwd


def test_gguf_mixed_types_load_and_match(tmp_path):
    """Block 2 of a file with Q4_K down and a Q6_K shared gate loads into an
    arena layer created with the standard types: the layer takes the file's
    types and matches the oracle on the written tensors."""
    H, I, Ish, E = 512, 256, 256, 16
    gt = (W.GGML_Q4_K, W.GGML_Q6_K, W.GGML_Q4_K, W.GGML_Q6_K, W.GGML_Q4_K, W.GGML_Q4_K)
    tensors = W.moe_layer_tensors(2, H, I, Ish, E, seed=33, types=gt)
    p = str(tmp_path / "mixed.gguf")
    W.write_gguf(p, [("general.architecture", W.STRING, "qwen3moe"), ("qwen3moe.expert_used_count", W.U32, 4)],
                 tensors)
    g = B.Gguf(p)
    s = g.moe_shape(2)
    arena = B.Arena(s, 1)
    arena.load_gguf(0, g, 2)
    d = arena.layer(0)
    assert api.layer_types(d) == gt
    by = {n: (ty, data) for n, ty, _, data in tensors}
    names = ["ffn_gate_exps", "ffn_up_exps", "ffn_down_exps", "ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp"]
    arrays = [by[f"blk.2.{n}.weight"][1] for n in names]
    hl = O.HostLayer(oshape(s), *arrays, np.asarray(by["blk.2.ffn_gate_inp.weight"][1]).view(np.float32),
                     np.asarray(by["blk.2.ffn_gate_inp_shexp.weight"][1]).view(np.uint16), types=gt)
    # the arena holds the file's bytes
    assert arena_host_layer(s, d).arrays[2].tobytes() == np.asarray(arrays[2]).tobytes()
    for T in (1, 6, 40):
        x, hidden = xs(T, H, 70 + T), xs(T, H, 80 + T)
        got, gi = run(s, d, x, hidden, api.PATH_AUTO)
        ref = hidden.copy()
        ri, _, _ = O.moe_forward(hl, x, ref, T, nthreads=16)
        assert np.array_equal(gi, np.asarray(ri).reshape(gi.shape)), T
        assert_moe_close(got, ref, base=hidden)
    # back to the standard types: the layer is re-laid out
    arena.set_layer_types(0, api.STANDARD_TYPES)
    assert api.layer_types(arena.layer(0)) == api.STANDARD_TYPES
    arena.close()
    g.close()
