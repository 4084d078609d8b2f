"""GPU parity of the standalone quantized kernels (bread_dequant_rows,
bread_matvec_f32, bread_matvec) against the CPU oracle.

Tier 1: dequantized weights bit-exact (including subnormal fp16 scales).
Matvec: fp32 within an error bound derived from the sum of |w*x| (the
summation order differs from the oracle's sequential one); fp16 I/O within
one fp16 ulp plus the reference self-test's 0.05 (kernels.cu:512-514).
"""
import numpy as np
import pytest
import torch

from breadv2_amd import api, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

Q4K, Q6K, Q80 = O.QTYPE_Q4_K, O.QTYPE_Q6_K, O.QTYPE_Q8_0


def rand_q80(n_blocks: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    blk = rng.integers(0, 256, size=(n_blocks, 34), dtype=np.uint8)
    d = (rng.uniform(1e-3, 1e-2, n_blocks).astype(np.float32).astype(np.float16)).view(np.uint16)
    blk[:, 0:2] = d.reshape(-1, 1).view(np.uint8)
    return blk.reshape(-1)


def weights(qtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    if qtype == Q4K:
        return synth.synth_q4k(rows * cols // 256, seed)
    if qtype == Q6K:
        return synth.synth_q6k(rows * cols // 256, seed)
    return rand_q80(rows * cols // 32, seed)


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def known_q4k_block() -> np.ndarray:
    """The reference's Q4_K known-answer block (dequant_q4k_cpu.c:181-225)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)  # d = 1.0, dmin = 0
    b[4:8] = 1
    b[12:16] = 1
    b[16:] = 0x59
    return b


def known_q6k_block() -> np.ndarray:
    """The reference's Q6_K known-answer block (dequant_q4k_cpu.c:257-262)."""
    b = np.zeros(210, np.uint8)
    b[0:128] = 0x88
    b[128:192] = 0xAA
    b[192:208] = 1
    b[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)
    return b


@pytest.mark.parametrize("qtype,rows,cols", [(Q4K, 64, 2048), (Q6K, 96, 512), (Q80, 40, 2080), (Q4K, 3, 256),
                                             (Q6K, 7, 4352)])
def test_dequant_bit_exact(qtype, rows, cols):
    w = weights(qtype, rows, cols, seed=11 + rows)
    got = api.bread_dequant_rows(dev(w), qtype, rows, cols).cpu().numpy()
    ref = O.dequant_rows(w, qtype, rows, cols).reshape(-1)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4K, Q6K, Q80])
def test_dequant_subnormal_and_signed_scales(qtype):
    """fp16 scales over every exponent, including subnormals, zero and
    negative values: the case the reference's flushing converter got wrong."""
    rows, cols = 16, 2048 if qtype != Q80 else 2048
    w = weights(qtype, rows, cols, seed=5).copy()
    rng = np.random.default_rng(7)
    if qtype == Q4K:
        blk = w.reshape(-1, 144)
        hv = rng.integers(0, 0x7C00, size=(blk.shape[0], 2), dtype=np.uint16)
        hv[::3] &= 0x03FF  # subnormal / zero
        hv[1::5] |= 0x8000  # negative
        blk[:, 0:4] = hv.view(np.uint8).reshape(-1, 4)
    elif qtype == Q6K:
        blk = w.reshape(-1, 210)
        hv = rng.integers(0, 0x7C00, size=blk.shape[0], dtype=np.uint16)
        hv[::2] &= 0x03FF
        hv[1::3] |= 0x8000
        blk[:, 208:210] = hv.reshape(-1, 1).view(np.uint8)
    else:
        blk = w.reshape(-1, 34)
        hv = rng.integers(0, 0x7C00, size=blk.shape[0], dtype=np.uint16)
        hv[::2] &= 0x03FF
        blk[:, 0:2] = hv.reshape(-1, 1).view(np.uint8)
    got = api.bread_dequant_rows(dev(w), qtype, rows, cols).cpu().numpy()
    ref = O.dequant_rows(w, qtype, rows, cols).reshape(-1)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_known_answer_blocks():
    """kernels.cu:411-446 / dequant_q4k_cpu.c:181-283: 9/5 pattern, all 8.0,
    and the row dots with x = 1 (1792 and 2048)."""
    q4 = np.tile(known_q4k_block(), 8)  # 8 rows x 256 cols
    q6 = np.tile(known_q6k_block(), 8)
    d4 = api.bread_dequant_rows(dev(q4), Q4K, 8, 256).cpu().numpy().reshape(8, 256)
    d6 = api.bread_dequant_rows(dev(q6), Q6K, 8, 256).cpu().numpy().reshape(8, 256)
    exp4 = np.tile(np.repeat(np.array([9.0, 5.0], np.float32), 32), 4)
    assert np.array_equal(d4, np.tile(exp4, (8, 1)))
    assert np.all(d6 == 8.0)
    ones32 = torch.ones(256, dtype=torch.float32, device=DEV)
    y = torch.empty(8, dtype=torch.float32, device=DEV)
    api.bread_matvec_f32(dev(q4), ones32, y, 8, 256, Q4K)
    assert np.all(y.cpu().numpy() == 1792.0)
    api.bread_matvec_f32(dev(q6), ones32, y, 8, 256, Q6K)
    assert np.all(y.cpu().numpy() == 2048.0)
    ones16 = torch.ones(256, dtype=torch.float16, device=DEV)
    y16 = torch.empty(8, dtype=torch.float16, device=DEV)
    api.bread_matvec(dev(q4), ones16, y16, 8, 256, Q4K)
    assert np.max(np.abs(y16.float().cpu().numpy() - 1792.0)) < 0.05
    api.bread_matvec(dev(q6), ones16, y16, 8, 256, Q6K)
    assert np.max(np.abs(y16.float().cpu().numpy() - 2048.0)) < 0.05


def abs_bound(w, qtype, x, rows, cols):
    """sum_c (|d*sc*q| + |dmin*m|) * |x[c]| per row (fp64): the magnitude of
    the terms the kernels sum, for a summation-order error bound.  For Q4_K
    the dequant of the block with dmin's sign flipped gives d*sc*q + dmin*m."""
    wm = np.array(w, copy=True)
    if qtype == Q4K:
        wm.reshape(-1, 144)[:, 3] |= 0x80
    deq = np.abs(O.dequant_rows(wm, qtype, rows, cols).astype(np.float64))
    return (deq * np.abs(x.astype(np.float64))[None, :]).sum(axis=1)


@pytest.mark.parametrize(
    "qtype,rows,cols",
    [(Q4K, 512, 2048), (Q4K, 1, 256), (Q4K, 37, 4352), (Q4K, 300, 16384), (Q6K, 2048, 512), (Q6K, 5, 256),
     (Q6K, 33, 2304), (Q80, 100, 2048), (Q80, 3, 32), (Q80, 17, 2080),
     (Q4K, 20001, 2048), (Q4K, 16385, 4096), (Q6K, 20001, 2048), (Q6K, 16385, 4096)],
)
def test_matvec_f32_parity(qtype, rows, cols):
    """Config 1 is the first case (512 x 2048 Q4_K, x ~ N(0,1)).  Row counts
    >= 16384 with 2048 or 4096 columns take the long-matvec kernel (x held in
    registers, two rows per iteration; odd counts exercise its tail)."""
    w = weights(qtype, rows, cols, seed=rows * 7 + cols)
    x = np.random.default_rng(rows + cols).standard_normal(cols).astype(np.float32)
    y = torch.empty(rows, dtype=torch.float32, device=DEV)
    api.bread_matvec_f32(dev(w), dev(x), y, rows, cols, qtype)
    got = y.cpu().numpy().astype(np.float64)
    ref = O.matvec(w, qtype, x, rows, cols, nthreads=8).astype(np.float64)
    bound = abs_bound(w, qtype, x, rows, cols)
    # two fp32 summation orders differ by at most ~2 n u sum|w x|; observed is far lower
    assert np.all(np.abs(got - ref) <= 2 * cols * 2.0**-24 * bound + 1e-30)
    assert np.linalg.norm(got - ref) <= 1e-5 * np.linalg.norm(ref)


@pytest.mark.parametrize("qtype,rows,cols", [(Q4K, 512, 2048), (Q6K, 2048, 512), (Q80, 64, 2048), (Q4K, 9, 768),
                                             (Q4K, 20001, 2048), (Q4K, 16385, 4096), (Q4K, 16384, 2048),
                                             (Q6K, 16385, 4096), (Q6K, 20001, 2048)])
def test_matvec_f16_io(qtype, rows, cols):
    """bread_matvec fp16 I/O: equal to the oracle's fp16-rounded result up to
    one ulp plus the fp32 summation-order bound of test_matvec_f32_parity
    (which dominates for results near zero, where the fp16 ulp is tiny)."""
    w = weights(qtype, rows, cols, seed=3 + rows)
    x16 = np.random.default_rng(9).standard_normal(cols).astype(np.float16)
    y = torch.empty(rows, dtype=torch.float16, device=DEV)
    api.bread_matvec(dev(w), dev(x16), y, rows, cols, qtype)
    got = y.cpu().numpy()
    ref = O.matvec_f16io(w, qtype, x16.view(np.uint16), rows, cols).view(np.float16)
    g32 = got.astype(np.float32)
    r32 = ref.astype(np.float32)
    ulp = np.spacing(np.abs(ref)).astype(np.float32)
    order = 2 * cols * 2.0**-24 * abs_bound(w, qtype, x16.astype(np.float32), rows, cols)
    assert np.all(np.abs(g32 - r32) <= ulp + order + 1e-6)
    assert np.max(np.abs(g32 - r32)) < 0.05 * max(1.0, float(np.max(np.abs(r32))))


@pytest.mark.parametrize("qtype", [Q4K, Q6K])
def test_lm_head_full_size_f16_io(qtype):
    """The lm_head at its benchmark shape (248,320 x 2048, fp16 I/O, the
    long-matvec kernels): every row computed on the device; the first and
    last 1,024 rows (the kernel's first and last slots, the range-checked
    loads past the matrix) and 4,096 random ones checked against the oracle
    to the bound of test_matvec_f16_io."""
    rows, cols = 248_320, 2048
    rb = cols // 256 * (144 if qtype == Q4K else 210)
    wd = torch.empty(rows * rb, dtype=torch.uint8, device=DEV)
    (api.synth_q4k if qtype == Q4K else api.synth_q6k)(wd, rows * cols // 256, 77 + qtype)
    x16 = np.random.default_rng(78).standard_normal(cols).astype(np.float16)
    y = torch.empty(rows, dtype=torch.float16, device=DEV)
    api.bread_matvec(wd, dev(x16), y, rows, cols, qtype)
    got = y.cpu().numpy().astype(np.float32)
    w = wd.cpu().numpy()
    pick = np.unique(np.concatenate([np.arange(1024), np.arange(rows - 1024, rows),
                                     np.random.default_rng(79).integers(0, rows, 4096)]))
    wsel = w.reshape(rows, rb)[pick].reshape(-1)
    n = pick.size
    ref = O.matvec_f16io(wsel, qtype, x16.view(np.uint16), n, cols).view(np.float16).astype(np.float32)
    ulp = np.spacing(np.abs(ref.astype(np.float16))).astype(np.float32)
    order = 2 * cols * 2.0**-24 * abs_bound(wsel, qtype, x16.astype(np.float32), n, cols)
    err = np.abs(got[pick] - ref)
    assert np.all(err <= ulp + order + 1e-6), f"max excess {float(np.max(err - ulp - order))}"
    assert np.all(np.isfinite(got))


def test_matvec_zero_rows_is_noop():
    w = torch.zeros(144, dtype=torch.uint8, device=DEV)
    x = torch.zeros(256, dtype=torch.float32, device=DEV)
    y = torch.full((1,), 7.0, device=DEV)
    api.bread_matvec_f32(w, x, y, 0, 256, Q4K)
    torch.cuda.synchronize()
    assert y.item() == 7.0
