"""Timeline of the decode kernel from its trace points (bread_moe_ctx_set_trace).

    python -m breadv2_amd.decode_timeline [--layers 8] [--stack 4] [--launches 8]

Runs single-layer launches and one stack launch of --stack layers over a
synthetic resident arena, back to back, and prints for each traced point the
earliest and latest workgroup's time in microseconds from the launch's first
workgroup start (the kernel's wall clock runs at 100 MHz).  Needs a GPU.
"""
import argparse

import numpy as np
import torch

from . import api
from .api import Arena, MoeContext

# trace point names, in the order of the header's point numbers
POINTS = ["start", "x ready", "own logit", "logits seen", "rank 1", "ranks known", "own down dots",
          "down dots", "SwiGLU seen", "output stored", "last SwiGLU", "down bands in", "passes",
          "ranks final", "exact logit", "exact logits seen", "cert prep", "cert ready"]


def timelines(ctx: MoeContext, descs, h, n_layers: int, launches: int):
    grid = ctx.set_trace(None)
    npt = len(POINTS)
    buf = torch.zeros(grid * n_layers * npt, dtype=torch.int64, device=h.device)
    ctx.set_trace(buf)
    out = []
    try:
        for i in range(launches):
            buf.zero_()
            ctx.decode_layers(descs[:n_layers], h)
            torch.cuda.synchronize()
            out.append(buf.cpu().numpy().reshape(grid, n_layers, npt).astype(np.float64))
    finally:
        ctx.set_trace(None)
    return out


def describe(t: np.ndarray) -> list:
    """Lines 'L<layer> point: earliest/latest' in µs from the first start."""
    t0 = t[:, 0, 0].min()
    lines = []
    for l in range(t.shape[1]):
        parts = []
        for k, name in enumerate(POINTS):
            col = t[:, l, k]
            col = col[col > 0]
            if len(col):
                parts.append(f"{name} {(col.min() - t0) * 0.01:.2f}/{(col.max() - t0) * 0.01:.2f}")
        lines.append(f"L{l}: " + ", ".join(parts))
    return lines


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--layers", type=int, default=8, help="resident layers (synthetic)")
    ap.add_argument("--stack", type=int, default=4, help="layers in the stack launch")
    ap.add_argument("--launches", type=int, default=8, help="traced launches of each kind (the middle one is shown)")
    args = ap.parse_args()
    s = api.shape()
    arena = Arena(s, args.layers)
    for l in range(args.layers):
        arena.synth_layer(l, seed=7)
    ctx = MoeContext(s, 1)
    h = torch.randn(1, s.hidden, device="cuda:0")
    descs = [arena.layer(l) for l in range(args.layers)]
    for i in range(20):  # warm-up
        ctx.decode_layers([descs[i % args.layers]], h)
    torch.cuda.synchronize()
    for n in (1, args.stack):
        runs = timelines(ctx, descs, h, n, args.launches)
        t = runs[len(runs) // 2]
        span = (t[:, -1, 9].max() - t[:, 0, 0].min()) * 0.01
        print(f"--- {n}-layer launch: span {span:.2f} us")
        for line in describe(t):
            print(line, flush=True)
    if ctx.check_device():
        raise RuntimeError("the decode kernel flagged a device error")
    arena.close()


if __name__ == "__main__":
    main()
