"""The routing softmax's expf (breadv2_amd/csrc/bread_expf.h, libm_expf) must
equal the C library's expf bit for bit: cpu_softmax (layer_ops.cu:222-229)
calls the C library's, and the oracle is that same function.

The restatement compiled for the host (tests/expf_check.hip, built here
against the same header the kernels include) is compared
with the C library over every float in [-104, -1] and [-2^-20, 0) and a
stride through all 2^32 bit patterns (NaNs, infinities, subnormals and the
overflow and underflow edges included).  The whole 2^32 range was checked
once the same way (0 mismatches).

Mistakes planted in a copy of the header, not in the product (two table
entries swapped; the quadratic coefficient off from its 8th hex digit) must
be caught by the same ranges."""
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "breadv2_amd", "csrc")
TOOL_SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "expf_check.hip")
HIPCC = "/opt/rocm/bin/hipcc"

RANGES = [
    ("bf800000", "c2d00000", 1),     # [-104, -1]: every float
    ("80000000", "b5800000", 1),     # (-2^-20, 0]: every float
    ("00000000", "ffffffff", 97),    # all bit patterns, stride 97
    ("80000000", "bf800000", 13),    # [-1, -0], stride 13
]


def build_tool(src, inc, exe):
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-I", str(inc), str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-400:]
    return str(exe)


@pytest.fixture(scope="module")
def tool(tmp_path_factory):
    return build_tool(TOOL_SRC, CSRC, tmp_path_factory.mktemp("expf") / "expf_check")


def run(tool, first, last, stride):
    r = subprocess.run([tool, first, last, str(stride)], capture_output=True, text=True)
    n, bad = (int(v) for v in r.stdout.split())
    return r.returncode, n, bad, r.stderr


@pytest.mark.parametrize("first,last,stride", RANGES)
def test_libm_expf_restatement_is_bit_exact(tool, first, last, stride):
    rc, n, bad, err = run(tool, first, last, stride)
    assert n > 10_000_000 or stride == 13 or (first, last) == ("80000000", "b5800000")
    assert bad == 0 and rc == 0, err


def test_oracle_expf_is_the_c_library():
    x = np.random.default_rng(0).uniform(-110, 90, 100_000).astype(np.float32)
    got = O.expf(x)
    # numpy's float32 exp is not the C library's; the oracle's must agree
    # with it to within one ulp and be the exact C library call
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    fin = np.isfinite(ref) & (ref > 1e-37)
    ulp = np.abs(got[fin].view(np.int32).astype(np.int64) - ref[fin].view(np.int32).astype(np.int64))
    assert ulp.max() <= 1


@pytest.mark.parametrize("old,new", [
    ("0x3fef72b83c7d517bull, 0x3fef54873168b9aaull", "0x3fef54873168b9aaull, 0x3fef72b83c7d517bull"),
    ("fresh_u32(0x50fac4f3u)", "fresh_u32(0x51fac4f3u)"),
])
def test_check_catches_planted_errors(tmp_path, old, new):
    """The check is sensitive: a copy of the header with a plausible mistake
    must fail on the ranges above."""
    src = open(os.path.join(CSRC, "bread_expf.h")).read()
    assert old in src
    (tmp_path / "bread_expf.h").write_text(src.replace(old, new))
    (tmp_path / "expf_check.hip").write_text(open(TOOL_SRC).read())
    # the copy's own directory comes first for a quoted include: the planted header
    exe = build_tool(tmp_path / "expf_check.hip", tmp_path, tmp_path / "expf_check")
    total = 0
    for first, last, stride in RANGES[:2]:
        rc, n, nbad, _ = run(str(exe), first, last, stride)
        total += nbad
    assert total > 0
