"""MoE-layer output campaign on a GPU: every path's layer output against the
CPU oracle's fp32 restatement of the reference's MoE block (one_layer.cu:
1413-1471 with layer_ops.cu:32-255), per token, over many tokens and several
layers.  Not collected by pytest; run as

    python tests/campaign_outputs.py [--tokens N] [--layers L]

For each path and weight scale it prints the tokens compared, the routing
mismatches (the bar is 0), the relative L2 error of each call's layer output
(the T tokens of one call: the north-star bar 1e-3) and its max-abs error over
the output's RMS (bar 1e-2), as maxima over the calls, and the same two
figures per token (median, 99th percentile, maximum; for information: a
token is one row of a call's output).  "Unit" divides every superblock scale
by 64, so outputs are of order one; "bench" keeps the benchmark's synthetic
scales (outputs up to ~1e6).  Exits non-zero if a call breaks a bar or a
token routes differently.
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

from helpers import MAX_ABS_TOL, REL_L2_TOL, host_layer, scale_layer_d  # noqa: E402

DEV = "cuda:0"

PATHS = [
    ("decode kernel, one launch a token", api.PATH_DECODE, 1),
    ("small-batch, 8 tokens a call", api.PATH_SMALL, 8),
    ("small-batch, 16 tokens a call", api.PATH_SMALL, 16),
    ("grouped, 64 tokens a call", api.PATH_GROUPED, 64),
    ("grouped, 512 tokens a call", api.PATH_GROUPED, 512),
    ("per-token kernels, 4 tokens a call", api.PATH_PER_TOKEN, 4),
]


def per_token_errors(got, ref):
    d = got.astype(np.float64) - ref.astype(np.float64)
    r = ref.astype(np.float64)
    rl2 = np.linalg.norm(d, axis=1) / np.maximum(np.linalg.norm(r, axis=1), 1e-300)
    rms = np.sqrt(np.mean(r * r, axis=1))
    mab = np.max(np.abs(d), axis=1) / np.maximum(rms, 1.0)
    return rl2, mab


def per_call_errors(got, ref, T):
    n = got.shape[0] // T
    d = (got.astype(np.float64) - ref.astype(np.float64)).reshape(n, -1)
    r = ref.astype(np.float64).reshape(n, -1)
    rl2 = np.linalg.norm(d, axis=1) / np.maximum(np.linalg.norm(r, axis=1), 1e-300)
    rms = np.sqrt(np.mean(r * r, axis=1))
    mab = np.max(np.abs(d), axis=1) / np.maximum(rms, 1.0)
    return rl2, mab


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--tokens", type=int, default=2048, help="tokens per path, layer and scale")
    ap.add_argument("--layers", type=int, default=2, help="synthetic layers (weight seeds)")
    args = ap.parse_args()
    assert torch.cuda.is_available(), "the campaign needs the GPU"
    s = api.shape()
    ctx = B.MoeContext(s, max_tokens=512)
    failed = False
    t_start = time.time()
    for scale in ("unit", "bench"):
        for layer in range(args.layers):
            t = api.synth_layer_tensors(s, seed=4100 + layer, layer=layer)
            if scale == "unit":
                scale_layer_d(t, 6)
            torch.cuda.synchronize()
            hl = host_layer(t)
            x = np.random.default_rng(4200 + layer).standard_normal((args.tokens, s.hidden)).astype(np.float32)
            ref = np.zeros((args.tokens, s.hidden), np.float32)
            ri, _, _ = O.moe_forward(hl, x, ref, args.tokens, nthreads=16)
            for name, path, T in PATHS:
                n = args.tokens // T * T
                ctx.set_path(path)
                xd = torch.from_numpy(x[:n]).to(DEV)
                hid = torch.zeros(n, s.hidden, device=DEV)
                gis = []
                for c in range(n // T):
                    idx, _, _ = ctx.forward(t.desc(), xd[c * T:(c + 1) * T], hid[c * T:(c + 1) * T], T,
                                            want_routing=True)
                    gis.append(idx)
                torch.cuda.synchronize()
                gi = torch.cat(gis).cpu().numpy()
                bad = int(np.sum(np.any(gi != ri[:n], axis=1)))
                got = hid.cpu().numpy()
                crl2, cmab = per_call_errors(got, ref[:n], T)
                rl2, mab = per_token_errors(got, ref[:n])
                ok = bad == 0 and float(crl2.max()) < REL_L2_TOL and float(cmab.max()) < MAX_ABS_TOL
                ok = ok and ctx.check_device() == 0
                failed |= not ok
                print(f"{scale} layer {layer} | {name}: {n} tokens, {bad} routed differently | per call: rel L2 "
                      f"max {crl2.max():.2e}, max-abs/RMS max {cmab.max():.2e} | per token: rel L2 median "
                      f"{np.median(rl2):.2e} p99 {np.percentile(rl2, 99):.2e} max {rl2.max():.2e}, max-abs/RMS "
                      f"median {np.median(mab):.2e} max {mab.max():.2e}{'' if ok else '  FAILED'}", flush=True)
            del t
    print(f"done in {time.time() - t_start:.0f} s: {'FAILED' if failed else 'every call within the bars'}",
          flush=True)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
