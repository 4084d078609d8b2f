"""Bit-exact routing against the reference's own arithmetic.

The reference routes on the host (route_layer, one_layer.cu:964-985):
sequential fp32 router sums (products rounded, then added, in column
order), cpu_softmax with the C library's expf and a sequential sum,
cpu_topk with ties to the lower index (layer_ops.cu:222-250).  The oracle
restates exactly that.  Every path must select the same experts in the same
rank order; the multi-token paths compute the logits in the same order and
the softmax with the same expf, so their weights are bit-identical too.

Constructed near-ties: two router rows a, b built so that the reference's
sequential fp32 sums order them one way while their exact values (or any
other summation order) order them the other way, or tie them exactly while
the exact values differ.  The pair sits at the rank-K/K+1 boundary or inside
the top K.  Each case is checked to be what it claims (the oracle's choice
differs from the exact-order choice) before the GPU is asked.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

from helpers import host_layer

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def seq32(W, x):
    """The reference's sequential fp32 sum of each row of W with x."""
    p = (W.astype(np.float32) * x.astype(np.float32)[None, :]).astype(np.float32)
    return np.add.accumulate(p, axis=1, dtype=np.float32)[:, -1]


def exact(W, x):
    return (W.astype(np.float64) * x.astype(np.float64)[None, :]).sum(axis=1)


def find_pair(rng, x, want_tie: bool, target: float):
    """Rows a, b with seq32 order opposite to the exact order (or a seq32 tie
    with distinct exact values) and logits near `target`."""
    H = x.size
    for _ in range(200):
        a = (rng.standard_normal(H) * 0.02).astype(np.float32)
        a *= np.float32(target / exact(a[None], x)[0])
        # b = a with two weights moved a few ulps in opposite directions: the
        # exact difference is tiny and of either sign, while the sequential
        # sums round at different places
        n = 4096
        b = np.repeat(a[None], n, axis=0)
        for direction in (np.float32(np.inf), np.float32(-np.inf)):
            j = rng.integers(0, H, n)
            k = rng.integers(1, 9, n)
            v = b[np.arange(n), j].copy()
            for step in range(1, 9):
                v = np.where(k >= step, np.nextafter(v, direction), v).astype(np.float32)
            b[np.arange(n), j] = v
        sa, sb = seq32(a[None], x)[0], seq32(b, x)
        ea, eb = exact(a[None], x)[0], exact(b, x)
        if want_tie:
            ok = np.nonzero((sb == sa) & (eb != ea))[0]
        else:
            ok = np.nonzero((np.sign(sa - sb) * np.sign(ea - eb) < 0))[0]
        if ok.size:
            return a, b[ok[0]]
    raise AssertionError("no near-tie found")


def near_tie_layer(seed: int, boundary: bool, want_tie: bool, E=256, K=8):
    """A router [E][H] and x with the constructed pair at ranks K-1/K
    (boundary) or 2/3 (inside the top K).  Returns (router, x, ia, ib)."""
    H = 2048
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(H).astype(np.float32)
    router = (rng.standard_normal((E, H)) * 0.004).astype(np.float32)   # logits ~ N(0, 0.18)
    n_above = K - 1 if boundary else 2
    a, b = find_pair(rng, x, want_tie, 3.0)
    # n_above rows clearly above the pair, the rest clearly below
    above = rng.choice(E, n_above + 2, replace=False)
    ia, ib = int(above[-2]), int(above[-1])
    for r, i in enumerate(above[:n_above]):
        router[i] = np.sign(x) * np.float32(0.004 + 0.0005 * r)          # logits ~ 6.5 + 0.8 r
    # the sequential winner at the higher index: ties and index-order
    # shortcuts then pick the wrong one
    wa = seq32(a[None], x)[0] >= seq32(b[None], x)[0]
    lo, hi = min(ia, ib), max(ia, ib)
    if want_tie:
        # seq32 tie: the reference takes the lower index; the exact-order
        # winner goes to the higher index
        first, second = (b, a) if exact(a[None], x)[0] > exact(b[None], x)[0] else (a, b)
    else:
        first, second = (b, a) if wa else (a, b)
    router[lo], router[hi] = first, second
    return router, x, lo, hi


def layer_with_router(base_t, s, router):
    r = dev(router.reshape(-1))
    lt = api.LayerTensors(s, base_t.gate_exps, base_t.up_exps, base_t.down_exps, base_t.gate_sh, base_t.up_sh,
                          base_t.down_sh, r, base_t.shgate)
    torch.cuda.synchronize()
    return lt


@pytest.fixture(scope="module")
def base():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=777, layer=0)
    torch.cuda.synchronize()
    return s, t


CASES = [(11, True, False), (12, True, True), (13, False, False), (14, False, True)]


def check_case_is_meaningful(router, x, K):
    ex_order = np.lexsort((np.arange(router.shape[0]), -exact(router, x)))[:K]
    sq = seq32(router, x)
    sq_order = np.lexsort((np.arange(router.shape[0]), -sq.astype(np.float64)))[:K]
    assert not np.array_equal(ex_order, sq_order), "construction does not separate the orders"
    return sq_order


@pytest.mark.parametrize("seed,boundary,tie", CASES)
@pytest.mark.parametrize("path,T", [("route", 1), ("route", 3), (api.PATH_PER_TOKEN, 2), (api.PATH_SMALL, 2),
                                    (api.PATH_SMALL, 16), (api.PATH_GROUPED, 17), (api.PATH_GROUPED, 129),
                                    (api.PATH_DECODE, 1)])
def test_near_ties_follow_sequential_order(base, seed, boundary, tie, path, T):
    s, t = base
    router, x, lo, hi = near_tie_layer(seed, boundary, tie)
    lt = layer_with_router(t, s, router)
    hl = host_layer(lt)
    ridx, rw, rg = O.route(hl, x)
    sq = check_case_is_meaningful(router, x, s.top_k)
    assert np.array_equal(ridx, sq), "oracle must follow the sequential order"
    xs = np.repeat(x[None], T, axis=0)
    ctx = B.MoeContext(s, max_tokens=T)
    if path == "route":
        idx, w, g = ctx.route(lt.desc(), dev(xs), T)
    else:
        ctx.set_path(path)
        hid = torch.zeros(T, s.hidden, device=DEV)
        idx, w, g = ctx.forward(lt.desc(), dev(xs), hid, T, want_routing=True)
    torch.cuda.synchronize()
    gi = idx.cpu().numpy()
    for tt in range(T):
        assert np.array_equal(gi[tt], ridx), f"token {tt}: {gi[tt]} vs oracle {ridx}"
    assert ctx.check_device() == 0


def bulk_layer(base, router_std, seed):
    s, t = base
    E, H = s.n_experts, s.hidden
    router = (np.random.default_rng(seed).standard_normal((E, H)) * router_std).astype(np.float32)
    return layer_with_router(t, s, router)


@pytest.mark.parametrize("router_std", [0.02, 1.0 / np.sqrt(2048)])
def test_bulk_route_bit_exact(base, router_std):
    """16,384 tokens through bread_route: indices, weights and shared-gate
    scores bit-identical to the oracle's (mismatch count 0)."""
    s, _ = base
    lt = bulk_layer(base, router_std, 5)
    hl = host_layer(lt)
    T = 16384
    x = np.random.default_rng(6).standard_normal((T, s.hidden)).astype(np.float32)
    ctx = B.MoeContext(s, max_tokens=T)
    idx, w, g = ctx.route(lt.desc(), dev(x), T)
    torch.cuda.synchronize()
    ri, rw, rg = O.route_batch(hl, x, nthreads=16)
    gi, gw, gg = idx.cpu().numpy(), w.cpu().numpy(), g.cpu().numpy()
    bad_idx = int(np.sum(np.any(gi != ri, axis=1)))
    bad_w = int(np.sum(np.any(gw.view(np.uint32) != rw.view(np.uint32), axis=1)))
    bad_g = int(np.sum(gg.view(np.uint32) != rg.view(np.uint32)))
    assert (bad_idx, bad_w, bad_g) == (0, 0, 0), f"mismatching tokens: idx {bad_idx}, w {bad_w}, gsh {bad_g}"


@pytest.mark.parametrize("path,T,chunks", [(api.PATH_SMALL, 16, 64), (api.PATH_GROUPED, 512, 8),
                                           (api.PATH_GROUPED, 64, 16), (api.PATH_PER_TOKEN, 8, 8)])
def test_bulk_paths_route_bit_exact(base, path, T, chunks):
    """Thousands of tokens through each multi-token path: indices bit-identical
    to the oracle's; weights bit-identical on the paths that sum every logit in
    the reference's order, within the certified radius's effect on the
    small-batch path (its certified tokens keep their fast logits)."""
    s, t = base
    lt = bulk_layer(base, 1.0 / np.sqrt(2048), 8)
    hl = host_layer(lt)
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    rng = np.random.default_rng(9 + T)
    gis, gws, xs = [], [], []
    for _ in range(chunks):
        x = rng.standard_normal((T, s.hidden)).astype(np.float32)
        hid = torch.zeros(T, s.hidden, device=DEV)
        idx, w, _ = ctx.forward(lt.desc(), dev(x), hid, T, want_routing=True)
        gis.append(idx)
        gws.append(w)
        xs.append(x)
    torch.cuda.synchronize()
    x = np.concatenate(xs)
    gi = torch.cat(gis).cpu().numpy()
    gw = torch.cat(gws).cpu().numpy()
    ri, rw, _ = O.route_batch(hl, x, nthreads=16)
    assert int(np.sum(np.any(gi != ri, axis=1))) == 0
    if path == api.PATH_SMALL:
        assert np.all(np.abs(gw - rw) <= 1e-3 * np.abs(rw) + 1e-7)
    else:
        assert int(np.sum(np.any(gw.view(np.uint32) != rw.view(np.uint32), axis=1))) == 0
    assert ctx.check_device() == 0


@pytest.mark.parametrize("router_std", [0.02, 1.0 / np.sqrt(2048)])
@pytest.mark.parametrize("path,T", [(api.PATH_SMALL, 1), (api.PATH_SMALL, 5), (api.PATH_SMALL, 16),
                                    (api.PATH_SMALL, 17), (api.PATH_SMALL, 32)])
def test_certified_routing_bulk(base, router_std, path, T):
    """Certified fast routing (the small-batch path, 1 to 32 tokens a call)
    over 2,048 tokens: indices bit-identical to the oracle's for every token;
    weights and shared-gate scores of certified tokens from the fast sums,
    within 1e-3 relative of the oracle's (the radius bounds the logits'
    difference at ~1e-4); the outcome counters account for every token, and
    most tokens are certified."""
    s, _ = base
    lt = bulk_layer(base, router_std, 30 + T)
    hl = host_layer(lt)
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(path)
    ctx.route_stats(reset=True)
    rng = np.random.default_rng(31 + T)
    n = 2048 // T
    gis, gws, ggs, xs = [], [], [], []
    for _ in range(n):
        x = rng.standard_normal((T, s.hidden)).astype(np.float32)
        hid = torch.zeros(T, s.hidden, device=DEV)
        idx, w, g = ctx.forward(lt.desc(), dev(x), hid, T, want_routing=True)
        gis.append(idx)
        gws.append(w)
        ggs.append(g)
        xs.append(x)
    torch.cuda.synchronize()
    x = np.concatenate(xs)
    gi = torch.cat(gis).cpu().numpy()
    gw = torch.cat(gws).cpu().numpy()
    gg = torch.cat(ggs).cpu().numpy().reshape(-1)
    ri, rw, rg = O.route_batch(hl, x, nthreads=16)
    st = ctx.route_stats()
    print(f"path {path} T={T} router std {router_std:.4f}: {st}", flush=True)
    assert int(np.sum(np.any(gi != ri, axis=1))) == 0
    assert np.all(np.abs(gw - rw) <= 1e-3 * np.abs(rw) + 1e-7), float(np.max(np.abs(gw - rw) / np.abs(rw)))
    rg = np.asarray(rg).reshape(-1)
    assert np.all(np.abs(gg - rg) <= 1e-3 * np.maximum(1.0, np.abs(rg)))
    assert st["multi_certified"] + st["multi_candidates"] + st["multi_exact"] == n * T
    assert st["multi_certified"] > 0.5 * n * T
    assert ctx.check_device() == 0


@pytest.mark.parametrize("router_std", [0.02, 1.0 / np.sqrt(2048)])
def test_bulk_decode_route_bit_exact(base, router_std):
    """4,096 tokens, each through a single-layer launch of the decode kernel
    (fast logits, certified ranks, reference-order recomputation when the
    certificate fails): indices bit-identical to the oracle's for every
    token, and the certificate's outcomes counted once per launch."""
    s, _ = base
    lt = bulk_layer(base, router_std, 21)
    hl = host_layer(lt)
    T = 4096
    x = np.random.default_rng(22).standard_normal((T, s.hidden)).astype(np.float32)
    xd = dev(x)
    ctx = B.MoeContext(s, max_tokens=1)
    ctx.set_path(api.PATH_DECODE)
    ctx.route_stats(reset=True)
    hid = torch.zeros(1, s.hidden, device=DEV)
    gis = []
    for t in range(T):
        idx, _, _ = ctx.forward(lt.desc(), xd[t:t + 1], hid, 1, want_routing=True)
        gis.append(idx)
    torch.cuda.synchronize()
    gi = torch.cat(gis).cpu().numpy()
    ri, _, _ = O.route_batch(hl, x, nthreads=16)
    bad = int(np.sum(np.any(gi != ri, axis=1)))
    st = ctx.route_stats()
    print(f"router std {router_std:.4f}: {st}", flush=True)
    assert bad == 0, f"{bad} of {T} tokens routed differently"
    assert st["decode_radius"] + st["decode_per_expert"] + st["decode_pair"] + st["decode_exact"] == T
    assert ctx.check_device() == 0


def test_decode_wide_logit_spread_routes_exactly(base):
    """One logit at 60 and the others between -55 and -46, not in index
    order.  The reference's probabilities below the first underflow to 0 and
    tie, so cpu_topk takes the lowest indices; the fast logits order them
    otherwise.  The certificate must not vouch for ranks whose probabilities
    are not normal floats: the decode kernel recomputes every logit in the
    reference's order and selects what the reference selects."""
    s, t = base
    E, H, K = s.n_experts, s.hidden, s.top_k
    rng = np.random.default_rng(31)
    x = rng.standard_normal(H).astype(np.float32)
    xx = np.float32(np.dot(x.astype(np.float64), x.astype(np.float64)))
    target = (-46.0 - 9.0 * rng.random(E)).astype(np.float32)   # expf(l - 60) underflows to 0
    top = 100
    target[top] = 60.0
    router = (target[:, None] * (x / xx)[None, :]).astype(np.float32)
    lt = layer_with_router(t, s, router)
    hl = host_layer(lt)
    ri, _, _, lg = O.route(hl, x, want_logits=True)
    rest = [e for e in range(E) if e != top]
    assert ri[0] == top and list(ri[1:]) == rest[:K - 1], "reference ties the underflowed probabilities"
    by_logit = np.lexsort((np.arange(E), -lg.astype(np.float64)))[:K]
    assert not np.array_equal(by_logit, ri), "the logit order must differ from the reference's choice"
    assert lg.max() - np.sort(lg)[-K] > 104.0
    ctx = B.MoeContext(s, max_tokens=1)
    ctx.set_path(api.PATH_DECODE)
    hid = torch.zeros(1, H, device=DEV)
    idx, _, _ = ctx.forward(lt.desc(), dev(x[None]), hid, 1, want_routing=True)
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy()[0], ri), f"{idx.cpu().numpy()[0]} vs oracle {ri}"
    assert ctx.route_stats()["decode_exact"] == 1
    assert ctx.check_device() == 0


def small_route(s, lt, xs):
    T = xs.shape[0]
    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(api.PATH_SMALL)
    ctx.route_stats(reset=True)
    hid = torch.zeros(T, s.hidden, device=DEV)
    idx, w, _ = ctx.forward(lt.desc(), dev(xs), hid, T, want_routing=True)
    torch.cuda.synchronize()
    st = ctx.route_stats()
    assert ctx.check_device() == 0
    return idx.cpu().numpy(), w.cpu().numpy(), st


def test_small_wide_logit_spread_routes_exactly(base):
    """The decode kernel's wide-spread case on the small-batch path: the
    fast certificate and the candidates' exact ranks must both refuse the
    underflowed probabilities, so every logit is summed in the reference's
    order and the host's selection picks the lowest indices, as cpu_topk
    does; weights then bit-identical too."""
    s, t = base
    E, H, K = s.n_experts, s.hidden, s.top_k
    rng = np.random.default_rng(31)
    x = rng.standard_normal(H).astype(np.float32)
    xx = np.float32(np.dot(x.astype(np.float64), x.astype(np.float64)))
    target = (-46.0 - 9.0 * rng.random(E)).astype(np.float32)
    target[100] = 60.0
    router = (target[:, None] * (x / xx)[None, :]).astype(np.float32)
    lt = layer_with_router(t, s, router)
    ri, rw, _ = O.route(host_layer(lt), x)
    gi, gw, st = small_route(s, lt, np.repeat(x[None], 3, axis=0))
    for tt in range(3):
        assert np.array_equal(gi[tt], ri), f"{gi[tt]} vs oracle {ri}"
        assert np.array_equal(gw[tt].view(np.uint32), np.asarray(rw, np.float32).view(np.uint32))
    assert st["multi_exact"] == 3, st


def test_small_tied_rows_route_by_index(base):
    """24 identical router rows on top (identical reference sums, so the
    reference takes them by index): the fast certificate cannot separate
    them, the candidates (more than one batch of 16 rows) are summed in the
    reference's order, tie exactly and are ranked by index."""
    s, t = base
    E, H = s.n_experts, s.hidden
    rng = np.random.default_rng(41)
    x = rng.standard_normal((5, H)).astype(np.float32)
    router = (rng.standard_normal((E, H)) * 0.004).astype(np.float32)
    rows = np.sort(rng.choice(E, 24, replace=False))
    router[rows] = (np.sign(x[0]) * 0.01).astype(np.float32)[None, :]
    lt = layer_with_router(t, s, router)
    ri, _, _ = O.route_batch(host_layer(lt), x, nthreads=8)
    assert np.array_equal(ri[0], rows[:s.top_k]), "the oracle ranks the tied rows by index"
    gi, _, st = small_route(s, lt, x)
    assert np.array_equal(gi, ri), f"{gi} vs oracle {ri}"
    assert st["multi_certified"] + st["multi_candidates"] + st["multi_exact"] == 5
    assert st["multi_candidates"] >= 1, st


def test_small_large_logits_route_exactly(base):
    """Logits far beyond |64| (router std 2): the certificate does not apply,
    every logit is summed in the reference's order and the host's selection
    runs: indices and weights bit-identical to the oracle's."""
    s, _ = base
    lt = bulk_layer(base, 2.0, 51)
    T = 7
    x = np.random.default_rng(52).standard_normal((T, s.hidden)).astype(np.float32)
    ri, rw, _ = O.route_batch(host_layer(lt), x, nthreads=8)
    gi, gw, st = small_route(s, lt, x)
    assert np.array_equal(gi, ri)
    assert np.array_equal(gw.view(np.uint32), np.asarray(rw, np.float32).view(np.uint32))
    assert st["multi_exact"] == T, st
