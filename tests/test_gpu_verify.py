"""GPU: batched speculative verification at the MoE boundary.

- bread_argmax_f16 is bit-exact against the oracle's greedy_sample
  restatement (main.cu:326-335), ties, NaN and infinities included;
- bread_moe_stack_forward takes B tokens through a stack of MoE layers.
  One call equals the same layers called one at a time, bit for bit; on
  each layer's own input the oracle's block (RMSNorm, MoE) gives the same
  routing bit for bit and the output within the layer tolerance.  One token
  equals the decode stack launch bit for bit.  B tokens at once agree with
  B single-token stacks: first-layer routing exactly, final residuals within
  the tolerance (deeper layers see inputs that differ by the grouped path's
  fp16-weight rounding, ~4e-4 relative L2 per layer against ~2e-6 for the
  fp32 paths, so near-tied ranks may swap there);
- bread_moe_greedy_head: fp16 logits within the bread_matvec bound of the
  oracle's, tokens the argmax of those logits; the batched Q4_K head (one
  pass over the weights for up to 32 tokens) on inputs whose fp16
  normalisation is exact: every token's logits within one fp16 ulp plus the
  fp32 order bound of the oracle's matvec on the same input, each token's
  logits and token bit-equal to a one-token call's;
- a verification round: the batched predictions equal the token-by-token
  ones (main_speculative.cu:477-497 runs bread_step per token), and
  bread_spec_accept accepts exactly the drafts that match them.
"""

import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api, synth
from oracle import oracle as O

from helpers import arena_host_layer, assert_moe_close
from test_gpu_quant import abs_bound

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
Q4K, Q6K = O.QTYPE_Q4_K, O.QTYPE_Q6_K
L = 3


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture(scope="module")
def stack():
    """L arena layers at the full shape with per-layer norm weights."""
    s = api.shape()
    arena = B.Arena(s, L)
    for l in range(L):
        arena.synth_layer(l, seed=321, router_std=1.0 / np.sqrt(s.hidden))
    rng = np.random.default_rng(5)
    nws = [rng.uniform(0.5, 1.5, s.hidden).astype(np.float32) for _ in range(L)]
    nwd = [dev(w) for w in nws]
    descs = []
    for l in range(L):
        d = arena.layer(l)
        d.post_norm_w = nwd[l].data_ptr()
        descs.append(d)
    torch.cuda.synchronize()
    hls = [arena_host_layer(s, arena.layer(l)) for l in range(L)]
    yield s, descs, hls, nws
    arena.close()


def test_argmax_matches_greedy_sample():
    rng = np.random.default_rng(2)
    for n, T in [(248320, 3), (1001, 4), (8, 2), (1, 1)]:
        a = rng.integers(-30, 30, (T, n)).astype(np.float16)  # many exact ties
        a[0, 0] = np.nan                     # row 0: NaN first -> 0
        if n > 3:
            a[1, 1] = np.float16(np.inf)     # row 1: +inf wins
            a[1, 2] = np.float16(np.inf)
            a[T - 1, :: 3] = np.nan          # last row: NaNs skipped
        got = B.argmax_f16(dev(a)).cpu().numpy()
        want = [O.greedy_f16(a[t]) for t in range(T)]
        assert list(got) == want, (n, list(got), want)


def test_stack_forward_matches_oracle(stack):
    s, descs, hls, nws = stack
    T = 8
    h0 = np.random.default_rng(21).standard_normal((T, s.hidden)).astype(np.float32)
    ctx = B.MoeContext(s, max_tokens=T)
    whole = dev(h0)
    ctx.stack_forward(descs, whole, T)
    hd = dev(h0)
    for l in range(L):
        h_in = hd.cpu().numpy()
        idx, _, _ = ctx.stack_forward([descs[l]], hd, T, want_routing=True)
        torch.cuda.synchronize()
        ref = h_in.copy()
        ridx = np.zeros((T, s.top_k), np.int32)
        for t in range(T):
            x = O.rms_norm_weighted(h_in[t], nws[l], s.rms_eps)
            hh = ref[t][None].copy()
            ri, _, _ = O.moe_forward(hls[l], x[None], hh, 1, nthreads=16)
            ridx[t] = np.asarray(ri).reshape(-1)
            ref[t] = hh[0]
        assert np.array_equal(idx.cpu().numpy()[0], ridx), l
        assert_moe_close(hd.cpu().numpy(), ref, base=h_in)
    torch.cuda.synchronize()
    assert np.array_equal(whole.cpu().numpy().view(np.uint32), hd.cpu().numpy().view(np.uint32))
    assert ctx.check_device() == 0


def test_stack_forward_one_token_is_decode_stack(stack):
    s, descs, _, _ = stack
    h0 = np.random.default_rng(22).standard_normal((1, s.hidden)).astype(np.float32)
    ctx = B.MoeContext(s, max_tokens=1)
    a, b = dev(h0), dev(h0)
    ctx.stack_forward(descs, a, 1)
    ctx.decode_layers(descs, b)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))
    assert ctx.check_device() == 0


def test_stack_forward_batched_equals_single_tokens(stack):
    s, descs, _, _ = stack
    T = 16
    h0 = np.random.default_rng(23).standard_normal((T, s.hidden)).astype(np.float32)
    ctx = B.MoeContext(s, max_tokens=T)
    hb = dev(h0)
    ib, wb, _ = ctx.stack_forward(descs, hb, T, want_routing=True)
    singles, isingle, wsingle = [], [], []
    for t in range(T):
        ht = dev(h0[t:t + 1])
        it, wt, _ = ctx.stack_forward(descs, ht, 1, want_routing=True)
        singles.append(ht)
        isingle.append(it)
        wsingle.append(wt)
    torch.cuda.synchronize()
    ones = torch.cat(singles).cpu().numpy()
    ib, wb = ib.cpu().numpy(), wb.cpu().numpy()
    i1, w1 = torch.cat(isingle, dim=1).cpu().numpy(), torch.cat(wsingle, dim=1).cpu().numpy()
    assert np.array_equal(ib[0], i1[0])
    np.testing.assert_allclose(wb[0], w1[0], rtol=2e-5, atol=1e-7)
    assert_moe_close(hb.cpu().numpy(), ones, base=h0)
    assert ctx.check_device() == 0


def test_stack_forward_few_tokens_run_decode_stacks(stack):
    """Up to bread_stack_loop_tokens() tokens under the automatic choice: one
    decode-stack launch per token, the routing of token t in record t of each
    layer; equal to single-token stacks bit for bit."""
    s, descs, _, _ = stack
    T = B.lib.bread_stack_loop_tokens()
    assert T >= 2
    h0 = np.random.default_rng(24).standard_normal((T, s.hidden)).astype(np.float32)
    ctx = B.MoeContext(s, max_tokens=T)
    hb = dev(h0)
    ib, wb, gb = ctx.stack_forward(descs, hb, T, want_routing=True)
    ib, wb, gb = ib.cpu().numpy(), wb.cpu().numpy(), gb.cpu().numpy()
    for t in range(T):
        ht = dev(h0[t:t + 1])
        it, wt, gt = ctx.stack_forward(descs, ht, 1, want_routing=True)
        torch.cuda.synchronize()
        assert np.array_equal(hb[t].cpu().numpy().view(np.uint32), ht[0].cpu().numpy().view(np.uint32))
        assert np.array_equal(ib[:, t], it.cpu().numpy()[:, 0])
        assert np.array_equal(wb[:, t], wt.cpu().numpy()[:, 0])
        assert np.array_equal(gb[:, t], gt.cpu().numpy()[:, 0])
    assert ctx.check_device() == 0


def head_weights(qtype, vocab, H, seed):
    return synth.synth_q4k(vocab * H // 256, seed) if qtype == Q4K else synth.synth_q6k(vocab * H // 256, seed)


def oracle_head(s, h, nw, w, qtype, vocab):
    x16 = np.stack([O.rms_norm_weighted(h[t], nw, s.rms_eps) for t in range(h.shape[0])]).astype(np.float16)
    lg = np.stack([O.matvec_f16io(w, qtype, x16[t].view(np.uint16), vocab, s.hidden).view(np.float16)
                   for t in range(h.shape[0])])
    return x16, lg


@pytest.mark.parametrize("qtype,vocab", [(Q4K, 16384), (Q6K, 4096)])
def test_greedy_head(qtype, vocab):
    s = api.shape()
    T = 4
    rng = np.random.default_rng(vocab)
    h = rng.standard_normal((T, s.hidden)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, s.hidden).astype(np.float32)
    w = head_weights(qtype, vocab, s.hidden, seed=vocab + qtype)
    ctx = B.MoeContext(s, max_tokens=T)
    tok, lg = ctx.greedy_head(dev(h), dev(nw), dev(w), qtype, vocab, T)
    torch.cuda.synchronize()
    tok, lg = tok.cpu().numpy(), lg.cpu().numpy()
    # the tokens are greedy_sample over the returned logits, exactly
    assert list(tok) == [O.greedy_f16(lg[t]) for t in range(T)]
    # the logits: fp16 result within one ulp plus the fp32 order bound of the
    # matvec tests, on the oracle's input (itself within one fp16 ulp of the
    # device's normalised input, so the bound is widened by that ulp's effect)
    _, ref = oracle_head(s, h, nw, w, qtype, vocab)
    g, r = lg.astype(np.float64), ref.astype(np.float64)
    assert np.linalg.norm(g - r) <= 2e-3 * np.linalg.norm(r)
    assert np.max(np.abs(g - r)) < 0.05 * max(1.0, float(np.max(np.abs(r))))
    # where the oracle's top two logits are apart by more than the error, the
    # tokens agree with the oracle's greedy choice
    for t in range(T):
        srt = np.sort(r[t])
        if srt[-1] - srt[-2] > 4 * float(np.max(np.abs(g[t] - r[t]))):
            assert tok[t] == O.greedy_f16(ref[t])


@pytest.mark.parametrize("T", [1, 5, 16, 17, 32, 35])
def test_greedy_head_batched_q4k(T):
    s = api.shape()
    H, vocab = s.hidden, 4096 + 16 * T
    rng = np.random.default_rng(600 + T)
    # h = +-1 and fp16-exact norm weights: x = h inv_rms w rounds to +-w in
    # fp16 on any summation order (inv_rms = 1/sqrt(1 + eps) is within 5e-7
    # of 1), so device and oracle start from the same x16
    h = rng.choice([-1.0, 1.0], size=(T, H)).astype(np.float32)
    nw = rng.choice([0.5, 0.75, 1.0, 1.25, 1.5], size=H).astype(np.float32)
    w = head_weights(Q4K, vocab, H, seed=900 + T)
    x16 = (h * nw[None]).astype(np.float16)
    ctx = B.MoeContext(s, max_tokens=T)
    wd, nwd = dev(w), dev(nw)
    print(f"batched head T={T} vocab={vocab}", flush=True)
    tok, lg = ctx.greedy_head(dev(h), nwd, wd, Q4K, vocab, T)
    torch.cuda.synchronize()
    tok, lg = tok.cpu().numpy(), lg.cpu().numpy()
    assert ctx.check_device() == 0
    for t in range(T):
        ref = O.matvec_f16io(w, Q4K, x16[t].view(np.uint16), vocab, H).view(np.float16).astype(np.float64)
        order = 2 * H * 2.0 ** -24 * abs_bound(w, Q4K, x16[t].astype(np.float32), vocab, H)
        err = np.abs(lg[t].astype(np.float64) - ref)
        assert np.all(err <= np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) + order + 1e-6), \
            f"token {t}: max excess {float(np.max(err - order))}"
        assert tok[t] == O.greedy_f16(lg[t])
    # tokens are independent: the one-token call gives the same row and token
    for t in sorted({0, T // 2, T - 1}):
        t1, l1 = ctx.greedy_head(dev(h[t:t + 1]), nwd, wd, Q4K, vocab, 1)
        assert np.array_equal(l1.cpu().numpy()[0].view(np.uint16), lg[t].view(np.uint16))
        assert int(t1.cpu().numpy()[0]) == tok[t]


@pytest.mark.parametrize("T", [1, 17])
def test_greedy_head_full_vocab_q4k(T):
    """The batched head at the lm_head's real size (248,320 x 2048 Q4_K, about
    60 tiles a workgroup): every token's argmax is greedy_sample over its
    returned logits, and the first and last 512 rows plus 4,096 random ones
    are within one fp16 ulp plus the fp32 order bound of the oracle's (h =
    +-1 and fp16-exact norm weights give device and oracle the same x16)."""
    s = api.shape()
    H, vocab = s.hidden, 248_320
    rng = np.random.default_rng(700 + T)
    h = rng.choice([-1.0, 1.0], size=(T, H)).astype(np.float32)
    nw = rng.choice([0.5, 0.75, 1.0, 1.25, 1.5], size=H).astype(np.float32)
    rb = H // 256 * 144
    wd = torch.empty(vocab * rb, dtype=torch.uint8, device=DEV)
    api.synth_q4k(wd, vocab * H // 256, 710 + T)
    ctx = B.MoeContext(s, max_tokens=T)
    print(f"full-vocab head T={T}", flush=True)
    tok, lg = ctx.greedy_head(dev(h), dev(nw), wd, Q4K, vocab, T)
    torch.cuda.synchronize()
    tok, lg = tok.cpu().numpy(), lg.cpu().numpy()
    assert ctx.check_device() == 0
    w = wd.cpu().numpy()
    x16 = (h * nw[None]).astype(np.float16)
    pick = np.unique(np.concatenate([np.arange(512), np.arange(vocab - 512, vocab),
                                     rng.integers(0, vocab, 4096)]))
    wsel = w.reshape(vocab, rb)[pick].reshape(-1)
    for t in range(T):
        assert tok[t] == O.greedy_f16(lg[t])
        ref = O.matvec_f16io(wsel, Q4K, x16[t].view(np.uint16), pick.size, H).view(np.float16).astype(np.float64)
        order = 2 * H * 2.0 ** -24 * abs_bound(wsel, Q4K, x16[t].astype(np.float32), pick.size, H)
        err = np.abs(lg[t][pick].astype(np.float64) - ref)
        assert np.all(err <= np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) + order + 1e-6), \
            f"token {t}: max excess {float(np.max(err - order))}"


def test_greedy_head_batched_nan_row():
    """greedy_sample keeps index 0 when logits[0] is NaN: a NaN input token
    gives an all-NaN row and token 0; the other tokens are unaffected."""
    s = api.shape()
    H, vocab, T = s.hidden, 2048, 3
    rng = np.random.default_rng(77)
    h = rng.standard_normal((T, H)).astype(np.float32)
    h[1, 5] = np.nan
    w = head_weights(Q4K, vocab, H, seed=78)
    ctx = B.MoeContext(s, max_tokens=T)
    tok, lg = ctx.greedy_head(dev(h), None, dev(w), Q4K, vocab, T)
    torch.cuda.synchronize()
    tok, lg = tok.cpu().numpy(), lg.cpu().numpy()
    assert np.all(np.isnan(lg[1].astype(np.float32))) and tok[1] == 0
    for t in (0, 2):
        assert tok[t] == O.greedy_f16(lg[t]) and not np.any(np.isnan(lg[t].astype(np.float32)))


def test_verify_round_matches_token_by_token(stack):
    """One round with B = 5 (4 drafts): the batched predictions equal the
    per-token ones, and acceptance stops at the first wrong draft."""
    s, descs, _, _ = stack
    B_ = 5
    vocab = 16384
    rng = np.random.default_rng(31)
    h0 = rng.standard_normal((B_, s.hidden)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, s.hidden).astype(np.float32)
    w = dev(head_weights(Q4K, vocab, s.hidden, seed=77))
    nwd = dev(nw)
    ctx = B.MoeContext(s, max_tokens=B_)
    # token by token, as the reference's bread_step loop
    seq = []
    for t in range(B_):
        ht = dev(h0[t:t + 1])
        ctx.stack_forward(descs, ht, 1)
        tk, _ = ctx.greedy_head(ht, nwd, w, Q4K, vocab, 1)
        seq.append(int(tk.cpu().numpy()[0]))
    # the whole round at once
    hb = dev(h0)
    ctx.stack_forward(descs, hb, B_)
    tb, _ = ctx.greedy_head(hb, nwd, w, Q4K, vocab, B_)
    bat = [int(v) for v in tb.cpu().numpy()]
    assert bat == seq
    eos = vocab - 1
    drafts = [seq[0], seq[1], (seq[2] + 1) % (vocab - 1), seq[3]]
    assert B.spec_accept(bat, drafts, eos, 100) == (2, seq[2])
    assert B.spec_accept(bat, seq[:4], eos, 100) == (4, seq[4])
    assert ctx.check_device() == 0


def test_stack_forward_rejects_bad_arguments(stack):
    s, descs, _, _ = stack
    ctx = B.MoeContext(s, max_tokens=2)
    h = torch.zeros((4, s.hidden), dtype=torch.float32, device=DEV)
    with pytest.raises(B.BreadError):
        ctx.stack_forward(descs, h, 4)
    bad = B.MoeLayer.from_buffer_copy(descs[0])
    bad.post_norm_w = descs[0].post_norm_w + 4
    with pytest.raises(B.BreadError):
        ctx.stack_forward([bad], h, 2)
