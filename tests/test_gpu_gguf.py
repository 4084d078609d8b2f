"""GPU: MoE layers loaded from GGUF files into the HBM arena
(bread_arena_load_gguf) run through bread_moe_forward on every path and
match the CPU oracle computed from the tensors that were written to the file.

The files come from the independent writer in tests/gguf_writer.py with the
tensor names of the reference's loader (loader.c:162-164, :551-569,
one_layer.cu:964-975, :1413): routed experts as 3-d [H, I, E] / [I, H, E]
tensors, shared experts 2-d, the fp32 router, optional fp16 shared gate and
fp32 post-attention norm weight.
"""
import ctypes

import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

import gguf_writer as W
from helpers import assert_moe_close, d2h, oshape

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def host_from_tensors(s, tensors, layer):
    by = {n.split(".", 2)[2]: d for n, _, _, d in tensors if n.startswith(f"blk.{layer}.")}
    ty = {n.split(".", 2)[2]: t for n, t, _, _ in tensors if n.startswith(f"blk.{layer}.")}
    names = ["ffn_gate_exps", "ffn_up_exps", "ffn_down_exps", "ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp"]
    sg = by.get("ffn_gate_inp_shexp.weight")
    return O.HostLayer(oshape(s), *[by[f"{n}.weight"] for n in names],
                       np.asarray(by["ffn_gate_inp.weight"]).view(np.float32),
                       None if sg is None else np.asarray(sg).view(np.uint16),
                       types=[ty[f"{n}.weight"] for n in names])


def forward(s, d, x, hidden, path):
    ctx = B.MoeContext(s, max_tokens=x.shape[0])
    ctx.set_path(path)
    hd = torch.from_numpy(hidden.copy()).to(DEV)
    idx, w, _ = ctx.forward(d, torch.from_numpy(x).to(DEV), hd, x.shape[0], want_routing=True)
    torch.cuda.synchronize()
    assert ctx.check_device() == 0
    return hd.cpu().numpy(), idx.cpu().numpy()


def check_paths(s, d, hl, cases):
    for T, path in cases:
        print(f"gguf layer: T={T} path={path}", flush=True)
        rng = np.random.default_rng(T + 7)
        x = rng.standard_normal((T, s.hidden)).astype(np.float32)
        hidden = rng.standard_normal((T, s.hidden)).astype(np.float32)
        got, gi = forward(s, d, x, hidden, path)
        ref = hidden.copy()
        ri, _, _ = O.moe_forward(hl, x, ref, T, nthreads=16)
        assert np.array_equal(gi, np.asarray(ri).reshape(gi.shape)), (T, path)
        assert_moe_close(got, ref, base=hidden)


@pytest.fixture(scope="module")
def full_file(tmp_path_factory):
    """Two blocks at the reference model's MoE shape (H 2048, I 512, 256
    experts, top-8), with shared gate and norm weight."""
    s = api.shape()
    tensors = []
    for l in (0, 1):
        tensors += W.moe_layer_tensors(l, s.hidden, s.expert_inter, s.shared_inter, s.n_experts, seed=60 + l)
    p = str(tmp_path_factory.mktemp("gguf") / "full.gguf")
    W.write_gguf(p, [("general.architecture", W.STRING, "qwen3moe"), ("qwen3moe.expert_used_count", W.U32, 8)],
                 tensors)
    return p, tensors


def test_load_exposes_file_bytes(full_file):
    p, tensors = full_file
    g = B.Gguf(p)
    s = g.moe_shape(1)
    assert (s.hidden, s.expert_inter, s.shared_inter, s.n_experts, s.top_k) == (2048, 512, 512, 256, 8)
    arena = B.Arena(s, 2)
    arena.load_gguf(0, g, 1)  # block 1 of the file into arena layer 0
    d = arena.layer(0)
    by = {n: data for n, _, _, data in tensors}
    b = api.shape_bytes(s)
    E = s.n_experts
    assert d.gate_expert_bytes == len(by["blk.1.ffn_gate_exps.weight"]) // E
    assert d.down_expert_bytes == len(by["blk.1.ffn_down_exps.weight"]) // E
    pairs = [(d.gate_exps, "ffn_gate_exps", E * b["gate_expert"]), (d.up_exps, "ffn_up_exps", E * b["up_expert"]),
             (d.down_exps, "ffn_down_exps", E * b["down_expert"]), (d.gate_shexp, "ffn_gate_shexp", b["gate_sh"]),
             (d.up_shexp, "ffn_up_shexp", b["up_sh"]), (d.down_shexp, "ffn_down_shexp", b["down_sh"]),
             (d.router, "ffn_gate_inp", b["router"]), (d.shexp_gate, "ffn_gate_inp_shexp", b["shgate"]),
             (d.post_norm_w, "post_attention_norm", s.hidden * 4)]
    for ptr, name, nbytes in pairs:
        assert ptr, name
        want = np.asarray(by[f"blk.1.{name}.weight"]).view(np.uint8)
        assert want.size == nbytes, name
        assert np.array_equal(d2h(ptr, nbytes), want), name
    arena.close()
    g.close()


def test_loaded_layer_matches_oracle_on_every_path(full_file):
    p, tensors = full_file
    g = B.Gguf(p)
    s = g.moe_shape(0)
    arena = B.Arena(s, 2)
    for l in (0, 1):
        arena.load_gguf(l, g, l)
    for l in (0, 1):
        hl = host_from_tensors(s, tensors, l)
        check_paths(s, arena.layer(l), hl, [(1, api.PATH_AUTO), (1, api.PATH_PER_TOKEN), (16, api.PATH_GROUPED),
                                            (16, api.PATH_PER_TOKEN)])
    arena.close()


def test_small_layer_without_optional_tensors(tmp_path):
    """A block with no shared-expert gate and no norm weight: the arena layer
    exposes NULL for both and the shared expert enters ungated."""
    H, I, Ish, E = 512, 256, 256, 16
    tensors = W.moe_layer_tensors(3, H, I, Ish, E, seed=11, with_shgate=False, with_norm=False)
    p = str(tmp_path / "small.gguf")
    W.write_gguf(p, [("general.architecture", W.STRING, "qwen3moe"), ("qwen3moe.expert_used_count", W.U32, 2)],
                 tensors)
    g = B.Gguf(p)
    s = g.moe_shape(3)
    assert (s.hidden, s.expert_inter, s.shared_inter, s.n_experts, s.top_k) == (H, I, Ish, E, 2)
    arena = B.Arena(s, 1)
    arena.load_gguf(0, g, 3)
    d = arena.layer(0)
    assert not d.shexp_gate and not d.post_norm_w
    check_paths(s, d, host_from_tensors(s, tensors, 3), [(1, api.PATH_AUTO), (37, api.PATH_GROUPED),
                                                         (37, api.PATH_PER_TOKEN)])
    arena.close()


def test_mismatched_file_is_rejected(tmp_path):
    """Types and dimensions must match the arena's shape."""
    H, I, Ish, E = 512, 256, 256, 16
    tensors = W.moe_layer_tensors(0, H, I, Ish, E, seed=12)
    p = str(tmp_path / "m.gguf")
    W.write_gguf(p, [], tensors)
    g = B.Gguf(p)
    arena = B.Arena(api.shape(hidden=H, expert_inter=I, shared_inter=Ish, n_experts=2 * E, top_k=2), 1)
    with pytest.raises(B.BreadError):
        arena.load_gguf(0, g, 0)
    with pytest.raises(B.BreadError):
        arena.load_gguf(0, g, 1)  # no such block
    arena.close()
