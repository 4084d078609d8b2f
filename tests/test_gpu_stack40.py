"""Config 3 at full size: 40 resident layers of the Qwen3.5-35B-A3B MoE shape
in the HBM arena (~21 GB), 128 consecutive decode tokens, each through all 40
layers in one bread_moe_decode_layers launch, on one context.  This is the
reference's per-token, per-layer loop (main.cu:677-713 -> one_layer_forward,
whose MoE block's fp32 order is one_layer.cu:1413-1471) with the layer loop
inside the kernel.

Checked:
  - every token's stack launch against 40 chained single-layer launches on a
    second context, bit for bit: every layer's routing record (indices,
    weights, shared-gate logit) and the final hidden state.  The stack
    launch's 40-entry layer table and its epoch-tagged exchange state (5,120
    layer epochs on one context here) must not change a single bit;
  - every token's routing on all 40 layers (5,120 layer-tokens through the
    decode kernel's certified routing) against the route-only oracle, indices
    bit-exact, with the certificate's outcomes counted once per layer-token;
  - every 16th token against the oracle on all 40 layers: routed indices
    bit-exact, each layer's output within the north-star tolerance.  Routed
    experts are copied back from the arena only when a token selects them.
Router rows ~ N(0, 1/2048) so the logits on the unit-RMS normalised input are
~ N(0, 1), and seeded norm weights U(0.5, 1.5) between layers.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

from helpers import assert_moe_close, d2h, oshape

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
L = 40
TOKENS = 128
SAMPLE_EVERY = 16


class SparseHostLayer:
    """Host copy of one arena layer for the oracle in which only the routed
    experts a token uses are filled; the stacked expert arrays are
    zero-initialised (pages untouched until an expert is copied in)."""

    def __init__(self, s, gate, up, down):
        self.s = s
        self.b = api.shape_bytes(s)
        self.gate, self.up, self.down = gate, up, down

    def load(self, d, experts) -> "O.HostLayer":
        b = self.b
        for e in experts:
            e = int(e)
            for arr, base, n in ((self.gate, d.gate_exps, b["gate_expert"]), (self.up, d.up_exps, b["up_expert"]),
                                 (self.down, d.down_exps, b["down_expert"])):
                arr[e * n:(e + 1) * n] = d2h(base + e * n, n)
        return O.HostLayer(oshape(self.s), self.gate, self.up, self.down,
                           d2h(d.gate_shexp, b["gate_sh"]), d2h(d.up_shexp, b["up_sh"]), d2h(d.down_shexp, b["down_sh"]),
                           d2h(d.router, b["router"]).view(np.float32), d2h(d.shexp_gate, b["shgate"]).view(np.uint16))


@pytest.fixture(scope="module")
def stack40():
    s = api.shape()
    arena = B.Arena(s, L)
    for l in range(L):
        arena.synth_layer(l, seed=4040, router_std=1.0 / np.sqrt(s.hidden))
    rng = np.random.default_rng(40)
    nws = [rng.uniform(0.5, 1.5, s.hidden).astype(np.float32) for _ in range(L)]
    nwd = [torch.from_numpy(w).to(DEV) for w in nws]
    descs = []
    for l in range(L):
        d = arena.layer(l)
        d.post_norm_w = nwd[l].data_ptr()
        descs.append(d)
    torch.cuda.synchronize()
    yield s, arena, descs, nws
    arena.close()


def test_stack40_128_tokens(stack40):
    s, arena, descs, nws = stack40
    H, K, E = s.hidden, s.top_k, s.n_experts
    b = api.shape_bytes(s)
    ctx_stack = B.MoeContext(s, max_tokens=1)
    ctx_chain = B.MoeContext(s, max_tokens=1)
    sparse = SparseHostLayer(s, np.zeros(E * b["gate_expert"], np.uint8), np.zeros(E * b["up_expert"], np.uint8),
                             np.zeros(E * b["down_expert"], np.uint8))
    rng = np.random.default_rng(128)
    distinct = set()
    all_in, all_idx = [], []
    ctx_stack.route_stats(reset=True)
    for t in range(TOKENS):
        h0 = rng.standard_normal((1, H)).astype(np.float32)
        ha = torch.from_numpy(h0).to(DEV)
        hb = ha.clone()
        ia, wa, ga = ctx_stack.decode_layers(descs, ha, want_routing=True)
        ins, ib, wb, gb = [], [], [], []
        for l in range(L):
            ins.append(hb.clone())
            i1, w1, g1 = ctx_chain.decode_layers([descs[l]], hb, want_routing=True)
            ib.append(i1)
            wb.append(w1)
            gb.append(g1)
        torch.cuda.synchronize()
        ia, wa, ga = ia.cpu().numpy(), wa.cpu().numpy(), ga.cpu().numpy()
        ib = torch.cat(ib).cpu().numpy()
        wb = torch.cat(wb).cpu().numpy()
        gb = torch.cat(gb).cpu().numpy()
        assert np.array_equal(ia, ib), f"token {t}: stack and chained routing differ"
        assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), f"token {t}: routing weights differ"
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), f"token {t}: shared-gate logits differ"
        assert torch.equal(ha, hb), f"token {t}: stack and chained hidden differ"
        distinct.update(ia.reshape(-1).tolist())
        hin = torch.cat(ins).cpu().numpy()
        all_in.append(hin)
        all_idx.append(ia)
        if t % SAMPLE_EVERY:
            continue
        hout = np.concatenate([hin[1:], hb.cpu().numpy()])
        for l in range(L):
            xr = O.rms_norm_weighted(hin[l], nws[l], s.rms_eps)
            hl = sparse.load(descs[l], ia[l])
            ref = hin[l][None].copy()
            ri, rw, rg = O.moe_forward(hl, xr[None], ref, 1, nthreads=16)
            assert np.array_equal(ri[0], ia[l]), f"token {t} layer {l}: {ia[l]} vs oracle {ri[0]}"
            np.testing.assert_allclose(wa[l], rw[0], rtol=2e-5, atol=1e-7)
            assert_moe_close(hout[l], ref[0], base=hin[l])
    # every layer-token's routing against the route-only oracle
    st = ctx_stack.route_stats()
    print(f"stack routing outcomes: {st}", flush=True)
    assert sum(st.values()) == TOKENS * L
    hins, idxs = np.stack(all_in), np.stack(all_idx)    # [TOKENS][L][H], [TOKENS][L][K]
    bad = 0
    for l in range(L):
        xr = np.stack([O.rms_norm_weighted(hins[t, l], nws[l], s.rms_eps) for t in range(TOKENS)])
        ri, _, _ = O.route_batch(sparse.load(descs[l], []), xr, nthreads=16)
        bad += int(np.sum(np.any(ri != idxs[:, l], axis=1)))
    assert bad == 0, f"{bad} of {TOKENS * L} layer-tokens routed differently"
    assert ctx_stack.check_device() == 0 and ctx_chain.check_device() == 0
    # routing varies over layers and tokens (logits ~ N(0, 1))
    assert len(distinct) > E // 2
    ctx_stack.close()
    ctx_chain.close()
