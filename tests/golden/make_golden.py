"""Write tests/golden/ref_dequant_vectors.npz: seeded Q4_K and Q6_K blocks and
the fp32 values the reference's own dequant_q4k_cpu.c (compiled from its
source into oracle/_ref by oracle/Makefile) produces for them.

Also writes tests/golden/known_answer_blocks.json: the two known-answer blocks
of the reference's self-tests (dequant_q4k_cpu.c:181-283, kernels.cu:411-446)
with their expected values.

Run from the repository root after `make -C oracle`:
    python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from breadv2_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402


def main() -> int:
    ref = O.ref_dequant_lib()
    if ref is None:
        print("oracle/_ref/libref_dequant.so missing: build it with `make -C oracle` where /root/reference exists")
        return 1
    n = 48
    q4 = synth.synth_q4k(n, 0x5EED4).reshape(n, 144).copy()
    q6 = synth.synth_q6k(n, 0x5EED6).reshape(n, 210).copy()
    # the last 8 blocks of each carry subnormal / zero / negative fp16 scales
    rng = np.random.default_rng(11)
    sub = rng.integers(0, 0x400, size=8, dtype=np.uint16)
    sub[0] = 0
    sub[1] = 0x8001
    q4[-8:, 0:2] = sub.reshape(-1, 1).view(np.uint8)
    q4[-8:, 2:4] = rng.integers(0, 0x400, size=8, dtype=np.uint16).reshape(-1, 1).view(np.uint8)
    q6[-8:, 208:210] = sub.reshape(-1, 1).view(np.uint8)
    out4 = np.empty((n, 256), np.float32)
    out6 = np.empty((n, 256), np.float32)
    for b in range(n):
        blk = np.ascontiguousarray(q4[b])
        ref.dequant_q4k_block_cpu(blk.ctypes.data, out4[b].ctypes.data)
        blk6 = np.ascontiguousarray(q6[b])
        ref.dequant_q6k_block_cpu(blk6.ctypes.data, out6[b].ctypes.data)
    np.savez_compressed(os.path.join(HERE, "ref_dequant_vectors.npz"), q4k=q4, q4k_out=out4, q6k=q6, q6k_out=out6,
                        n_subnormal_tail=np.int32(8))

    k4 = np.zeros(144, np.uint8)
    k4[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    k4[4:8] = 1
    k4[12:16] = 1
    k4[16:] = 0x59
    k6 = np.zeros(210, np.uint8)
    k6[0:128] = 0x88
    k6[128:192] = 0xAA
    k6[192:208] = 1
    k6[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)
    doc = {
        "source": "dequant_q4k_cpu.c:181-283 and kernels.cu:411-446 of arahe-dev/breadv2",
        "q4k_block_hex": k4.tobytes().hex(),
        "q4k_expected": "elements 64j+[0,32) = 9.0, 64j+[32,64) = 5.0; row dot with x = 1 is 1792",
        "q4k_row_dot_ones": 1792.0,
        "q6k_block_hex": k6.tobytes().hex(),
        "q6k_expected": "all 256 elements 8.0; row dot with x = 1 is 2048",
        "q6k_row_dot_ones": 2048.0,
    }
    with open(os.path.join(HERE, "known_answer_blocks.json"), "w") as f:
        json.dump(doc, f, indent=1)
    print("wrote golden vectors")
    return 0


if __name__ == "__main__":
    sys.exit(main())
