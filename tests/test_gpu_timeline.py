"""The decode kernel's trace points (bread_moe_ctx_set_trace) through the
timeline tool's functions: every workgroup records every point a certified
layer reaches, and the points of one workgroup follow the kernel's phase
order (input, own logit, all logits, rank 1, all ranks, last SwiGLU out,
all SwiGLU in, output stored)."""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from breadv2_amd import decode_timeline as TL

pytestmark = pytest.mark.gpu

# point numbers (include/bread_moe.h)
START, XRDY, LOGIT, POLLED, RANK1, ROUTED, HREADY, OUT, HLAST = 0, 1, 2, 3, 4, 5, 8, 9, 10


def test_timeline_points_in_phase_order():
    s = api.shape()
    L = 3
    arena = B.Arena(s, L)
    for l in range(L):
        arena.synth_layer(l, seed=5)
    ctx = B.MoeContext(s, 1)
    h = torch.randn(1, s.hidden, device="cuda:0", generator=torch.Generator("cuda:0").manual_seed(3))
    descs = [arena.layer(l) for l in range(L)]
    for n in (1, L):
        t = TL.timelines(ctx, descs, h, n, 2)[-1]
        assert t.shape[2] == len(TL.POINTS)
        for l in range(n):
            for p in (START, XRDY, LOGIT, POLLED, RANK1, ROUTED, HREADY, OUT):
                assert np.all(t[:, l, p] > 0), (n, l, TL.POINTS[p])
            g = t[:, l]
            assert np.all(g[:, START] <= g[:, LOGIT])
            assert np.all(g[:, POLLED] <= g[:, RANK1])
            assert np.all(g[:, RANK1] <= g[:, ROUTED])
            assert np.all(g[:, HREADY] <= g[:, OUT])
            # a workgroup sees every SwiGLU value only after the last one is stored somewhere
            assert g[:, HREADY].min() >= g[g[:, HLAST] > 0, HLAST].min()
            if l:
                # a workgroup enters layer l after it entered layer l - 1
                assert np.all(t[:, l, START] > t[:, l - 1, START])
        lines = TL.describe(t)
        assert len(lines) == n and lines[0].startswith("L0: start")
    assert ctx.check_device() == 0
    arena.close()
