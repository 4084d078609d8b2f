"""Error paths of the kernels' bounded waits, forced from the host.

bread_moe_ctx_set_spin_limit(ctx, 0) gives every wait of the decode and
small-batch kernels one look and no sleep.  Waits on other workgroups or on
other waves then give up; every kernel still exits normally, and
bread_moe_ctx_check reports BREAD_ERR_DEVICE with the waits' bits:
  1, 2, 16  the decode kernel (hidden / SwiGLU values, router logits or
            radii, another wave of the same workgroup),
  8         the small-batch down kernel (its partner wave).
The check resets the context.  With the default limit back, the next calls
on the same context equal a fresh context's results bit for bit and the
oracle's to the layer tolerance.  Small non-zero limits let some waits
succeed and others give up at varying points; those runs must end too, with
either no bit or only the waits' bits.
"""
import numpy as np
import pytest
import torch

import breadv2_amd as B
from breadv2_amd import api
from oracle import oracle as O

from helpers import assert_moe_close, host_layer

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DECODE_BITS = 1 | 2 | 16
SMALL_BITS = 8


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.fixture(scope="module")
def full_layer():
    s = api.shape()
    t = api.synth_layer_tensors(s, seed=4242, layer=0)
    torch.cuda.synchronize()
    return s, t, host_layer(t)


def xs(T, H, seed):
    return np.random.default_rng(seed).standard_normal((T, H)).astype(np.float32)


def device_error(ctx) -> int:
    """The error word bread_moe_ctx_check reports (0 when it returns OK)."""
    try:
        return ctx.check_device()
    except B.BreadError as e:
        assert e.status == api._lib.ERR_DEVICE, str(e)
        assert e.device_error != 0
        return e.device_error


def decode_calls(ctx, t, x, hidden):
    """One single-layer launch and one two-layer stack launch."""
    h1 = dev(hidden)
    idx, _, _ = ctx.forward(t.desc(), dev(x), h1, 1, want_routing=True)
    h2 = dev(hidden)
    ctx.decode_layers([t.desc(), t.desc()], h2)
    torch.cuda.synchronize()
    return h1.cpu().numpy(), idx.cpu().numpy(), h2.cpu().numpy()


def small_call(ctx, t, x, hidden):
    hd = dev(hidden)
    idx, _, _ = ctx.forward(t.desc(), dev(x), hd, x.shape[0], want_routing=True)
    torch.cuda.synchronize()
    return hd.cpu().numpy(), idx.cpu().numpy()


def test_decode_spin_limit_zero_flags_and_recovers(full_layer):
    s, t, hl = full_layer
    x, hidden = xs(1, s.hidden, 31), xs(1, s.hidden, 32)
    fresh = B.MoeContext(s, max_tokens=1)
    want = decode_calls(fresh, t, x, hidden)
    assert fresh.check_device() == 0

    ctx = B.MoeContext(s, max_tokens=1)
    ctx.set_spin_limit(0)
    decode_calls(ctx, t, x, hidden)
    err = device_error(ctx)
    assert err != 0, "no wait gave up with a zero spin limit"
    assert err & ~DECODE_BITS == 0, f"unexpected bits {err:#x}"
    # the check cleared the word and reset the exchange state
    assert ctx.check_device() == 0

    ctx.set_spin_limit(-1)
    for _ in range(2):
        got = decode_calls(ctx, t, x, hidden)
        assert ctx.check_device() == 0
        for g, w in zip(got, want):
            assert np.array_equal(g, w)
    ref = hidden.copy()
    ridx, _, _ = O.moe_forward(hl, x, ref, 1)
    assert np.array_equal(got[1], np.asarray(ridx).reshape(got[1].shape))
    assert_moe_close(got[0], ref, base=hidden)


def test_small_spin_limit_zero_flags_and_recovers(full_layer):
    s, t, hl = full_layer
    T = 16
    x, hidden = xs(T, s.hidden, 41), xs(T, s.hidden, 42)
    fresh = B.MoeContext(s, max_tokens=T)
    fresh.set_path(api.PATH_SMALL)
    want = small_call(fresh, t, x, hidden)
    assert fresh.check_device() == 0

    ctx = B.MoeContext(s, max_tokens=T)
    ctx.set_path(api.PATH_SMALL)
    ctx.set_spin_limit(0)
    out, _ = small_call(ctx, t, x, hidden)
    err = device_error(ctx)
    assert err == SMALL_BITS, f"error word {err:#x}"
    # a workgroup whose wait gave up left its rows of hidden untouched
    assert np.any(np.all(out.reshape(T, -1, 8) == hidden.reshape(T, -1, 8), axis=(0, 2)))

    ctx.set_spin_limit(-1)
    got = small_call(ctx, t, x, hidden)
    assert ctx.check_device() == 0
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    ref = hidden.copy()
    ridx, _, _ = O.moe_forward(hl, x, ref, T, nthreads=16)
    assert np.array_equal(got[1], np.asarray(ridx).reshape(got[1].shape))
    assert_moe_close(got[0], ref, base=hidden)


@pytest.mark.parametrize("spin", [1, 8, 64])
def test_small_spin_limits_end_and_recover(full_layer, spin):
    """Limits that let some waits through: every launch ends, and any bit
    set is a wait's; the default limit then restores exact results."""
    s, t, _ = full_layer
    x1, h1 = xs(1, s.hidden, 51), xs(1, s.hidden, 52)
    x16, h16 = xs(16, s.hidden, 53), xs(16, s.hidden, 54)
    ctx = B.MoeContext(s, max_tokens=16)
    want_dec = decode_calls(ctx, t, x1, h1)
    ctx.set_path(api.PATH_SMALL)
    want_small = small_call(ctx, t, x16, h16)
    assert ctx.check_device() == 0

    ctx.set_spin_limit(spin)
    ctx.set_path(api.PATH_AUTO)
    decode_calls(ctx, t, x1, h1)
    assert device_error(ctx) & ~DECODE_BITS == 0
    ctx.set_path(api.PATH_SMALL)
    small_call(ctx, t, x16, h16)
    assert device_error(ctx) & ~SMALL_BITS == 0

    ctx.set_spin_limit(-1)
    got_small = small_call(ctx, t, x16, h16)
    ctx.set_path(api.PATH_AUTO)
    got_dec = decode_calls(ctx, t, x1, h1)
    assert ctx.check_device() == 0
    for g, w in zip(got_dec + got_small, want_dec + want_small):
        assert np.array_equal(g, w)


def test_spin_limit_bounds_checked_on_host(full_layer):
    s, _, _ = full_layer
    ctx = B.MoeContext(s, max_tokens=1)
    with pytest.raises(B.BreadError) as e:
        ctx.set_spin_limit(1 << 25)
    assert e.value.status == api._lib.ERR_ARG
    ctx.set_spin_limit(1 << 24)
    ctx.set_spin_limit(-5)
