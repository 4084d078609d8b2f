"""Pins the CPU oracle (oracle/bread_oracle.c) before it is trusted as the
parity checker.  Every check is independent of the oracle's own code: the
reference's known-answer blocks and its compiled dequant (golden vectors),
exhaustive hardware/numpy conversions, an independent packer for the 6-bit
scales, closed forms, fp64 brute force and stable sorts.
"""
import json
import os
import struct

import numpy as np
import pytest

from breadv2_amd import synth
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


# ---------------------------------------------------------------- fp16


def test_h2f_exhaustive_matches_hardware_conversion():
    """All 65,536 half patterns: finite values (subnormals included) equal
    numpy's float16 -> float32 conversion bit for bit; Inf/NaN keep their
    payload unquieted, as bread_h2f does (bread_utils.h:39-41)."""
    h = np.arange(65536, dtype=np.uint32)
    # through memory (an F16 row), not a ctypes float return, which widens to
    # a Python double and would quiet signalling NaNs on the way
    got = O.dequant_rows(h.astype(np.uint16).view(np.uint8), O.QTYPE_F16, 1, 65536).reshape(-1).view(np.uint32)
    hv = h.astype(np.uint16).view(np.float16)
    finite = np.isfinite(hv)
    ref = hv.astype(np.float32).view(np.uint32)
    assert np.array_equal(got[finite], ref[finite])
    # Inf / NaN: sign | 0x7F800000 | mantissa << 13
    nf = ~finite
    exp = ((h[nf] >> 15) << 31) | 0x7F800000 | ((h[nf] & 0x3FF) << 13)
    assert np.array_equal(got[nf], exp.astype(np.uint32))
    # the subnormal range is the case the reference's flushing converter lost
    assert O.h2f(0x0001) == 2.0 ** -24 and O.h2f(0x83FF) == -(1023 * 2.0 ** -24)


def test_f2h_round_to_nearest_even():
    # every finite half round-trips
    h = np.arange(65536, dtype=np.uint16)
    fin = np.isfinite(h.view(np.float16))
    for v in h[fin][::7]:
        assert O.f2h(O.h2f(int(v))) == int(v)
    # random floats over the whole half range (incl. subnormals, overflow, ties)
    rng = np.random.default_rng(0)
    f = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(1e-6),
        rng.standard_normal(2000).astype(np.float32) * np.float32(100),
        np.float32([65504, 65519.99, 65520, 1e9, -1e9, 2.0 ** -25, 2.0 ** -24 * 1.5, 0.0, -0.0]),
        # exact ties between two halves: 1 + (2k+1) * 2^-11
        (1 + (2 * np.arange(50) + 1) * 2.0 ** -11).astype(np.float32),
    ])
    ref = f.astype(np.float16).view(np.uint16)
    got = np.array([O.f2h(float(v)) for v in f], np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- 6-bit scales


def pack_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Independent Q4_K scale packer: 8 (scale, min) pairs of 6 bits into 12
    bytes.  Bytes 0-3: low 6 bits = sc[j], top 2 bits = bits 4-5 of sc[j+4];
    bytes 4-7: m[j] and bits 4-5 of m[j+4]; bytes 8-11: low nibble = low 4
    bits of sc[j+4], high nibble = low 4 bits of m[j+4]."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return q


def test_scale_min_unpack_exhaustive():
    """For every sub-block j and every (scale, min) pair value, with the other
    pairs random, unpacking the independent packing gives the pair back."""
    rng = np.random.default_rng(1)
    grid = np.arange(64, dtype=np.uint8)
    for j in range(8):
        for s in grid:
            sc = rng.integers(0, 64, 8).astype(np.uint8)
            m = rng.integers(0, 64, 8).astype(np.uint8)
            sc[j] = s
            m[j] = grid[(int(s) * 37 + j) % 64]
            q = pack_scales(sc, m)
            for jj in range(8):
                assert O.get_scale_min_k4(jj, q) == (sc[jj], m[jj])


# ---------------------------------------------------------------- dequant


def test_known_answer_blocks():
    doc = json.load(open(os.path.join(GOLD, "known_answer_blocks.json")))
    q4 = np.frombuffer(bytes.fromhex(doc["q4k_block_hex"]), np.uint8)
    q6 = np.frombuffer(bytes.fromhex(doc["q6k_block_hex"]), np.uint8)
    d4 = O.dequant_block(O.QTYPE_Q4_K, q4)
    exp = np.tile(np.repeat(np.float32([9.0, 5.0]), 32), 4)
    assert np.array_equal(d4, exp)
    assert np.all(O.dequant_block(O.QTYPE_Q6_K, q6) == 8.0)
    ones = np.ones(256, np.float32)
    assert O.matvec(q4, O.QTYPE_Q4_K, ones, 1, 256)[0] == doc["q4k_row_dot_ones"]
    assert O.matvec(q6, O.QTYPE_Q6_K, ones, 1, 256)[0] == doc["q6k_row_dot_ones"]


def test_dequant_matches_reference_golden_vectors():
    """The reference's own compiled dequant_q4k_cpu.c on seeded blocks: equal
    bit for bit wherever the fp16 scales are normal numbers; in the 8
    subnormal-scale blocks the reference file flushes d to 0
    (dequant_q4k_cpu.c:44-45) while the oracle follows bread_h2f, the
    converter of the live CPU path (layer_ops.cu:51-52)."""
    g = np.load(os.path.join(GOLD, "ref_dequant_vectors.npz"))
    tail = int(g["n_subnormal_tail"])
    for key, qt in (("q4k", O.QTYPE_Q4_K), ("q6k", O.QTYPE_Q6_K)):
        blocks, outs = g[key], g[key + "_out"]
        n = blocks.shape[0]
        for b in range(n):
            got = O.dequant_block(qt, blocks[b])
            if b < n - tail:
                assert np.array_equal(got.view(np.uint32), outs[b].view(np.uint32)), (key, b)
        # the reference file decodes subnormal fp16 as zero: on the same block
        # with its subnormal scales zeroed the oracle reproduces it exactly,
        # and with them kept it differs wherever the scale is not zero
        for b in range(n - tail, n):
            blk = blocks[b].copy()
            fields = (0, 2) if qt == O.QTYPE_Q4_K else (208,)
            flushed = blk.copy()
            any_sub = False
            for pos in fields:
                hv = int(blk[pos:pos + 2].view(np.uint16)[0])
                if (hv & 0x7C00) == 0:
                    flushed[pos:pos + 2] = np.array([hv & 0x8000], np.uint16).view(np.uint8)
                    any_sub |= (hv & 0x3FF) != 0
            assert np.array_equal(O.dequant_block(qt, flushed).view(np.uint32), outs[b].view(np.uint32)), (key, b)
            if any_sub:
                assert not np.array_equal(O.dequant_block(qt, blk), outs[b])


def test_dequant_matches_live_reference_build():
    """When oracle/_ref is built (this container), compare on fresh blocks."""
    ref = O.ref_dequant_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built here")
    q4 = synth.synth_q4k(300, 99).reshape(300, 144)
    q6 = synth.synth_q6k(300, 98).reshape(300, 210)
    out = np.empty(256, np.float32)
    for b in range(300):
        blk = np.ascontiguousarray(q4[b])
        ref.dequant_q4k_block_cpu(blk.ctypes.data, out.ctypes.data)
        assert np.array_equal(O.dequant_block(O.QTYPE_Q4_K, blk).view(np.uint32), out.view(np.uint32))
        blk6 = np.ascontiguousarray(q6[b])
        ref.dequant_q6k_block_cpu(blk6.ctypes.data, out.ctypes.data)
        assert np.array_equal(O.dequant_block(O.QTYPE_Q6_K, blk6).view(np.uint32), out.view(np.uint32))


def test_q4k_dequant_independent_formula():
    """Blocks built from known (d, dmin, sc, m, nibble) values with the
    independent packer; the expected value is computed in numpy float32 with
    the reference's three roundings: (d*sc)*q - dmin*m."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        d16 = rng.integers(0, 0x7C00, dtype=np.uint16)
        dm16 = rng.integers(0, 0x7C00, dtype=np.uint16)
        sc = rng.integers(0, 64, 8).astype(np.uint8)
        m = rng.integers(0, 64, 8).astype(np.uint8)
        nib = rng.integers(0, 16, 256).astype(np.uint8)
        blk = np.zeros(144, np.uint8)
        blk[0:2] = np.array([d16], np.uint16).view(np.uint8)
        blk[2:4] = np.array([dm16], np.uint16).view(np.uint8)
        blk[4:16] = pack_scales(sc, m)
        # element 64g + t (t < 32) is the low nibble of byte 32g + t, element
        # 64g + 32 + t the high nibble of the same byte
        for g in range(4):
            lo = nib[64 * g: 64 * g + 32]
            hi = nib[64 * g + 32: 64 * g + 64]
            blk[16 + 32 * g: 16 + 32 * g + 32] = lo | (hi << 4)
        d = np.array([d16], np.uint16).view(np.float16).astype(np.float32)[0]
        dmin = np.array([dm16], np.uint16).view(np.float16).astype(np.float32)[0]
        sub = np.arange(256) // 32
        d1 = (np.float32(d) * sc[sub].astype(np.float32)).astype(np.float32)
        m1 = (np.float32(dmin) * m[sub].astype(np.float32)).astype(np.float32)
        exp = (d1 * nib.astype(np.float32)).astype(np.float32) - m1
        got = O.dequant_block(O.QTYPE_Q4_K, blk)
        assert np.array_equal(got.view(np.uint32), exp.astype(np.float32).view(np.uint32))


def test_q6k_dequant_independent_formula():
    """Q6_K blocks from known 6-bit values and int8 scales; element
    128n + 32s + l has low nibble in ql[64n + 32(s&1) + l] (high nibble when
    s >= 2), bits 2s..2s+1 of qh[32n + l], scale sc[8n + l/16 + 2s]."""
    rng = np.random.default_rng(4)
    for _ in range(50):
        q = rng.integers(0, 64, 256).astype(np.uint8)
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        d16 = rng.integers(0, 0x7C00, dtype=np.uint16)
        blk = np.zeros(210, np.uint8)
        for n in range(2):
            for s in range(4):
                for l in range(32):
                    e = 128 * n + 32 * s + l
                    ql_i = 64 * n + 32 * (s & 1) + l
                    if s < 2:
                        blk[ql_i] |= q[e] & 15
                    else:
                        blk[ql_i] |= (q[e] & 15) << 4
                    blk[128 + 32 * n + l] |= (q[e] >> 4) << (2 * s)
        blk[192:208] = sc.view(np.uint8)
        blk[208:210] = np.array([d16], np.uint16).view(np.uint8)
        d = np.array([d16], np.uint16).view(np.float16).astype(np.float32)[0]
        e = np.arange(256)
        n_, s_, l_ = e // 128, (e % 128) // 32, e % 32
        scale = sc[8 * n_ + l_ // 16 + 2 * s_].astype(np.float32)
        exp = ((np.float32(d) * scale).astype(np.float32) * (q.astype(np.float32) - 32)).astype(np.float32)
        got = O.dequant_block(O.QTYPE_Q6_K, blk)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_q80_dequant_closed_form():
    rng = np.random.default_rng(5)
    blk = rng.integers(0, 256, 34).astype(np.uint8)
    blk[0:2] = np.array([0x1A3C], np.uint16).view(np.uint8)
    d = np.array([0x1A3C], np.uint16).view(np.float16).astype(np.float32)[0]
    exp = (np.float32(d) * blk[2:].view(np.int8).astype(np.float32)).astype(np.float32)
    assert np.array_equal(O.dequant_block(O.QTYPE_Q8_0, blk), exp)


# ---------------------------------------------------------------- matvec


@pytest.mark.parametrize("qtype,rows,cols", [(O.QTYPE_Q4_K, 64, 2048), (O.QTYPE_Q6_K, 64, 512),
                                             (O.QTYPE_Q4_K, 3, 768)])
def test_matvec_vs_fp64_bruteforce(qtype, rows, cols):
    w = synth.synth_q4k(rows * cols // 256, 7) if qtype == O.QTYPE_Q4_K else synth.synth_q6k(rows * cols // 256, 7)
    x = np.random.default_rng(6).standard_normal(cols).astype(np.float32)
    deq = O.dequant_rows(w, qtype, rows, cols).astype(np.float64)
    exact = deq @ x.astype(np.float64)
    got = O.matvec(w, qtype, x, rows, cols)
    bound = cols * 2.0 ** -24 * (np.abs(deq) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)
    # the sequential sum is what the reference computes: a Python float32 loop agrees bit for bit
    r = 1
    acc = np.float32(0)
    for c in range(cols):
        acc = np.float32(acc + np.float32(deq[r, c].astype(np.float32) * x[c]))
    assert acc == got[r]
    assert np.array_equal(O.matvec(w, qtype, x, rows, cols, nthreads=4), got)


def test_matvec_f16io_rounds_output():
    w = synth.synth_q4k(8 * 2048 // 256, 8)
    x16 = np.random.default_rng(9).standard_normal(2048).astype(np.float16)
    y = O.matvec_f16io(w, O.QTYPE_Q4_K, x16.view(np.uint16), 8, 2048)
    y32 = O.matvec(w, O.QTYPE_Q4_K, x16.astype(np.float32), 8, 2048)
    assert np.array_equal(y, y32.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- softmax / top-k


def test_softmax_properties():
    rng = np.random.default_rng(10)
    x = rng.standard_normal(256).astype(np.float32) * 3
    p = O.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(p, e / e.sum(), rtol=2e-6, atol=1e-12)
    assert abs(p.astype(np.float64).sum() - 1) < 1e-5
    # a NaN anywhere poisons the sum, so every probability is NaN
    x[17] = np.nan
    assert np.all(np.isnan(O.softmax(x)))


def test_topk_matches_stable_sort_with_ties():
    rng = np.random.default_rng(12)
    for trial in range(200):
        n = int(rng.integers(8, 257))
        k = int(rng.integers(1, min(n, 16) + 1))
        p = (rng.integers(0, 12, n) / 11.0).astype(np.float32)  # many exact ties
        idx, w = O.topk(p, k)
        order = sorted(range(n), key=lambda i: (-float(p[i]), i))[:k]
        assert list(idx) == order
        raw = p[order].astype(np.float32)
        s = np.float32(0)
        for v in raw:
            s = np.float32(s + v)
        exp = raw / s if s > 0 else raw
        assert np.array_equal(w, exp.astype(np.float32))


def test_topk_nan_rule():
    p = np.full(32, np.nan, np.float32)
    idx, w = O.topk(p, 8)
    assert list(idx) == list(range(8)) and np.all(np.isnan(w))


# ---------------------------------------------------------------- routing and the MoE block


def small_layer(E=16, K=4, H=512, I=256, seed=0, shgate=True):
    s = O.OShape(H, I, I, E, K)
    ge = I * (H // 256) * 144
    de = H * (I // 256) * 210
    rng = np.random.default_rng(seed)
    return O.HostLayer(
        s,
        synth.synth_q4k(E * ge // 144, seed + 1), synth.synth_q4k(E * ge // 144, seed + 2),
        synth.synth_q6k(E * de // 210, seed + 3), synth.synth_q4k(ge // 144, seed + 4),
        synth.synth_q4k(ge // 144, seed + 5), synth.synth_q6k(de // 210, seed + 6),
        (rng.standard_normal((E, H)) * 0.02).astype(np.float32),
        (rng.standard_normal(H) * 0.02).astype(np.float16).view(np.uint16) if shgate else None,
    )


def test_route_sequential_logits_and_fp64():
    L = small_layer(E=16, K=4, H=512)
    x = np.random.default_rng(13).standard_normal(512).astype(np.float32)
    idx, w, g, logits = O.route(L, x, want_logits=True)
    # sequential fp32 (one_layer.cu:969-971): a Python loop in numpy float32
    for e in (0, 7, 15):
        acc = np.float32(0)
        for j in range(512):
            acc = np.float32(acc + np.float32(L.router[e, j] * x[j]))
        assert acc == logits[e]
    np.testing.assert_allclose(logits, L.router.astype(np.float64) @ x.astype(np.float64), rtol=1e-4, atol=1e-5)
    gexp = sum(np.float64(v) for v in L.shgate.view(np.float16).astype(np.float64) * x.astype(np.float64))
    assert abs(g - gexp) < 1e-4
    order = sorted(range(16), key=lambda i: (-float(O.softmax(logits)[i]), i))[:4]
    assert list(idx) == order


def moe_fp64(L, x):
    """numpy fp64 re-derivation of the MoE block from the exact dequantised
    weights: shared first, then routed experts in rank order."""
    s = L.shape
    H, I = s.hidden, s.expert_inter
    g, u, d, gs, us, ds = L.arrays
    ge, de = I * (H // 256) * 144, H * (I // 256) * 210

    def dq(a, qt, rows, cols):
        return O.dequant_rows(np.ascontiguousarray(a), qt, rows, cols).astype(np.float64)

    xd = x.astype(np.float64)

    def expert(gw, uw, dw):
        gg = dq(gw, O.QTYPE_Q4_K, I, H) @ xd
        uu = dq(uw, O.QTYPE_Q4_K, I, H) @ xd
        hh = gg / (1 + np.exp(-gg)) * uu
        return dq(dw, O.QTYPE_Q6_K, H, I) @ hh

    idx, w, glog = O.route(L, x)
    out = 1 / (1 + np.exp(-np.float64(glog))) * expert(gs, us, ds)
    for k, e in enumerate(idx):
        out += np.float64(w[k]) * expert(g[e * ge:(e + 1) * ge], u[e * ge:(e + 1) * ge], d[e * de:(e + 1) * de])
    return out, idx


def test_moe_token_vs_fp64_rederivation():
    L = small_layer(E=16, K=4, H=512, I=256, seed=20)
    x = np.random.default_rng(14).standard_normal(512).astype(np.float32)
    h = np.zeros(512, np.float32)
    idx, w, g = O.moe_token(L, x, h)
    ref, ridx = moe_fp64(L, x)
    assert list(idx) == list(ridx)
    assert np.linalg.norm(h - ref) / np.linalg.norm(ref) < 1e-5


def test_moe_k1_is_one_expert_plus_shared():
    """K = 1: the renormalised weight is exactly 1, so the layer output is
    sigmoid(g) * shared(x) + expert_idx0(x)."""
    L = small_layer(E=8, K=1, H=512, I=256, seed=30)
    x = np.random.default_rng(15).standard_normal(512).astype(np.float32)
    h = np.zeros(512, np.float32)
    idx, w, g = O.moe_token(L, x, h)
    assert w[0] == 1.0
    ref, _ = moe_fp64(L, x)
    assert np.linalg.norm(h - ref) / np.linalg.norm(ref) < 1e-5


def test_moe_null_shared_gate_uses_half():
    L = small_layer(E=8, K=2, seed=40, shgate=False)
    x = np.random.default_rng(16).standard_normal(512).astype(np.float32)
    h = np.zeros(512, np.float32)
    _, _, g = O.moe_token(L, x, h)
    assert g == 0.0


def test_expert_block_is_moe_without_the_shared_expert():
    """With the shared expert's down weights all zero (Q6_K d = 0), the MoE
    block adds exactly 0 for it, so its output must equal the routed-only
    block run with the same routing, bit for bit."""
    L = small_layer(E=16, K=4, seed=60)
    L.arrays[5][:] = 0
    x = np.random.default_rng(18).standard_normal(512).astype(np.float32)
    h = np.zeros(512, np.float32)
    idx, w, _ = O.moe_token(L, x, h)
    h2 = np.zeros((1, 512), np.float32)
    O.expert_block(L, x[None], h2, np.asarray(idx)[None], np.asarray(w)[None])
    assert np.array_equal(h, h2[0])


def test_expert_block_vs_fp64_with_given_routing():
    """The reference benchmark's block (experts 0..K-1, weight 1/K) and an
    arbitrary routing with repeats, against numpy fp64 on the dequantised
    weights; the residual accumulates."""
    L = small_layer(E=8, K=4, H=512, I=256, seed=61)
    s = L.shape
    H, I = s.hidden, s.expert_inter
    g, u, d = L.arrays[:3]
    ge, de = I * (H // 256) * 144, H * (I // 256) * 210

    def dq(a, qt, rows, cols):
        return O.dequant_rows(np.ascontiguousarray(a), qt, rows, cols).astype(np.float64)

    rng = np.random.default_rng(19)
    x = rng.standard_normal((2, H)).astype(np.float32)
    idx = np.array([[0, 1, 2, 3], [5, 5, 0, 7]], np.int32)
    w = np.array([[0.25] * 4, [0.5, -0.25, 1.0, 0.125]], np.float32)
    base = rng.standard_normal((2, H)).astype(np.float32)
    h = base.copy()
    O.expert_block(L, x, h, idx, w)
    for t in range(2):
        ref = base[t].astype(np.float64)
        xd = x[t].astype(np.float64)
        for k in range(4):
            e = idx[t, k]
            gg = dq(g[e * ge:(e + 1) * ge], O.QTYPE_Q4_K, I, H) @ xd
            uu = dq(u[e * ge:(e + 1) * ge], O.QTYPE_Q4_K, I, H) @ xd
            ref += np.float64(w[t, k]) * (dq(d[e * de:(e + 1) * de], O.QTYPE_Q6_K, H, I) @ (gg / (1 + np.exp(-gg)) * uu))
        assert np.linalg.norm(h[t] - ref) / np.linalg.norm(ref - base[t]) < 1e-5


def test_moe_threaded_is_bit_identical_and_residual_accumulates():
    L = small_layer(E=16, K=4, seed=50)
    rng = np.random.default_rng(17)
    x = rng.standard_normal(512).astype(np.float32)
    base = rng.standard_normal(512).astype(np.float32)
    h1 = base.copy()
    h2 = base.copy()
    O.moe_token(L, x, h1)
    O.moe_token_mt(L, x, h2, 4)
    assert np.array_equal(h1, h2)
    h0 = np.zeros(512, np.float32)
    O.moe_token(L, x, h0)
    np.testing.assert_allclose(h1 - base, h0, rtol=1e-5, atol=1e-3)


def test_rms_norm_closed_form():
    rng = np.random.default_rng(18)
    x = rng.standard_normal(2048).astype(np.float32) * 5
    w = rng.uniform(0.5, 2, 2048).astype(np.float32)
    got = O.rms_norm_weighted(x, w, 1e-6)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    np.testing.assert_allclose(got, ref, rtol=2e-6)


def test_host_synth_generator_is_stable():
    """The generator's bytes are a function of (seed, position): prefixes agree
    and a fixed digest pins the stream."""
    a = synth.synth_q4k(10, 42)
    b = synth.synth_q4k(20, 42)
    assert np.array_equal(a, b[: a.size])
    d = synth.synth_q4k(4, 1).reshape(4, 144)[:, 0:4].copy().view(np.float16).astype(np.float32)
    assert np.all((d >= 1e-3 - 1e-6) & (d <= 1e-2 + 1e-5))
    sc = synth.synth_q6k(64, 2).reshape(64, 210)[:, 192:208].view(np.int8)
    assert sc.min() >= -32 and sc.max() <= 31
    digest = struct.unpack("<Q", synth.rng_words(1, 0, 1).tobytes())[0]
    assert digest == synth.fmix64(np.array([(1 * synth.SEED_MUL + synth.GAMMA) & synth.M64], np.uint64))[0]
