"""bread_route_noalloc (routing with the library's static device workspace,
no allocation on any call) against bread_route (context workspace): bit-
identical indices, weights and shared-gate logits on two calls in a row, the
second with fewer tokens, so that the workspace holds the first call's
values when the second one runs."""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_noalloc_matches_context_route_on_two_calls():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=31, layer=0, router_std=1.0 / np.sqrt(2048))
    desc = t.desc()
    ctx = B.MoeContext(s, max_tokens=1024)
    gen = torch.Generator(device="cpu").manual_seed(5)
    for T in (1024, 37):
        x = torch.randn(T, s.hidden, generator=gen).to(DEV)
        i0, w0, g0 = ctx.route(desc, x, T)
        i1, w1, g1 = api.route_noalloc(s, desc, x, T)
        torch.cuda.synchronize()
        assert torch.equal(i0, i1), f"T={T}: indices differ"
        assert torch.equal(w0.view(torch.int32), w1.view(torch.int32)), f"T={T}: weights differ"
        assert torch.equal(g0.view(torch.int32), g1.view(torch.int32)), f"T={T}: shared-gate logits differ"
    assert ctx.check_device() == 0
