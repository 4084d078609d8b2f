"""Routing parity campaign on a GPU: many more tokens than the test suite
through every routing path, each checked against the CPU oracle's restatement
of the reference's routing (route_layer, one_layer.cu:964-985; cpu_softmax and
cpu_topk, layer_ops.cu:222-250).  Not collected by pytest; run as

    python tests/campaign_routing.py [--tokens N] [--seeds S]

For every path, router scale and router seed it prints the tokens routed, the
tokens whose expert indices differ from the oracle's (the bar is 0), the
largest relative difference of the routing weights, and the routing outcome
counters (bread_moe_ctx_route_stats: how often the certificate vouched for
the fast logits, and how often logits were recomputed in the reference's
order).  Exits non-zero on any index mismatch or device error.
"""
import argparse
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import breadv2_amd as B  # noqa: E402
from breadv2_amd import api  # noqa: E402
from oracle import oracle as O  # noqa: E402

from helpers import host_layer  # noqa: E402

DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def layer_with_router(base_t, s, router):
    lt = api.LayerTensors(s, base_t.gate_exps, base_t.up_exps, base_t.down_exps, base_t.gate_sh, base_t.up_sh,
                          base_t.down_sh, dev(router.reshape(-1)), base_t.shgate)
    torch.cuda.synchronize()
    return lt


def run_path(ctx, lt, x, path, T):
    """Indices and weights of every token of x through `path`, T tokens a call."""
    n = x.shape[0] // T
    xd = dev(x[:n * T])
    gis, gws = [], []
    if path == "route":
        for c in range(n):
            idx, w, _ = ctx.route(lt.desc(), xd[c * T:(c + 1) * T], T)
            gis.append(idx)
            gws.append(w)
    else:
        ctx.set_path(path)
        hid = torch.zeros(T, lt.shape.hidden, device=DEV)
        for c in range(n):
            idx, w, _ = ctx.forward(lt.desc(), xd[c * T:(c + 1) * T], hid, T, want_routing=True)
            gis.append(idx)
            gws.append(w)
    torch.cuda.synchronize()
    return torch.cat(gis).cpu().numpy(), torch.cat(gws).cpu().numpy(), n * T


PATHS = [
    ("bread_route", "route", 1024),
    ("decode, one launch a token", api.PATH_DECODE, 1),
    ("small-batch, 1 token a call", api.PATH_SMALL, 1),
    ("small-batch, 4 tokens a call", api.PATH_SMALL, 4),
    ("small-batch, 8 tokens a call", api.PATH_SMALL, 8),
    ("small-batch, 16 tokens a call", api.PATH_SMALL, 16),
    ("small-batch, 32 tokens a call", api.PATH_SMALL, 32),
    ("grouped, 64 tokens a call", api.PATH_GROUPED, 64),
    ("grouped, 512 tokens a call", api.PATH_GROUPED, 512),
]


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--tokens", type=int, default=16384, help="tokens per path, router scale and seed")
    ap.add_argument("--seeds", type=int, default=2, help="router matrices per scale")
    args = ap.parse_args()
    assert torch.cuda.is_available(), "the campaign needs the GPU"
    s = api.shape()
    base = api.synth_layer_tensors(s, seed=777, layer=0)
    torch.cuda.synchronize()
    ctx = B.MoeContext(s, max_tokens=1024)
    failed = False
    total = 0
    t_start = time.time()
    # router scales: the bench's (logit spread ~0.9), a 4x narrower one
    # (more near-ties for the certificate) and a 5x wider one
    for std_name, std in (("N(0, 0.02)", 0.02), ("N(0, 0.005)", 0.005), ("N(0, 0.1)", 0.1)):
        for seed in range(args.seeds):
            router = (np.random.default_rng(1000 + seed).standard_normal((s.n_experts, s.hidden)) * std).astype(
                np.float32)
            lt = layer_with_router(base, s, router)
            hl = host_layer(lt)
            x = np.random.default_rng(2000 + seed).standard_normal((args.tokens, s.hidden)).astype(np.float32)
            ri, rw, _ = O.route_batch(hl, x, nthreads=16)
            for name, path, T in PATHS:
                ctx.route_stats(reset=True)
                gi, gw, n = run_path(ctx, lt, x, path, T)
                st = ctx.route_stats()
                bad = int(np.sum(np.any(gi != ri[:n], axis=1)))
                rel = float(np.max(np.abs(gw - rw[:n]) / np.maximum(np.abs(rw[:n]), 1e-30)))
                dev_err = ctx.check_device()
                counters = {k: v for k, v in st.items() if v}
                print(f"{std_name} seed {seed} | {name}: {n} tokens, {bad} mismatching, "
                      f"max rel weight diff {rel:.2e}, outcomes {counters}", flush=True)
                failed |= bad != 0 or dev_err != 0
                total += n
    print(f"{total} token routings in {time.time() - t_start:.0f} s: "
          f"{'FAILED' if failed else 'every index equal to the oracle'}", flush=True)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
