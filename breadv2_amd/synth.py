"""Host twin of the device's seeded weight generator (breadv2_amd/csrc/synth.hip).

word(seed, i) = fmix64(seed * 0x632BE59BD9B4E019 + (i + 1) * 0x9E3779B97F4A7C15),
the SplitMix64 output function over a counter; every byte depends only on
(seed, byte position), so host and device produce identical bytes.

Q4_K superblock k = little-endian bytes of words 18k .. 18k+17 (144 B), with
bytes 0..3 replaced by d and dmin: fp16 of U(1e-3, 1e-2) drawn from the low
and high 16 bits of word 18k's low half.
Q6_K superblock k = the first 210 bytes of words 27k .. 27k+26, with the 16
scale bytes (offset 192) mapped to int8 (raw & 63) - 32 and the fp16 d
(offset 208) drawn from the low 16 bits of word 27k+26.
"""
from __future__ import annotations

import numpy as np

GAMMA = 0x9E3779B97F4A7C15
SEED_MUL = 0x632BE59BD9B4E019
M64 = (1 << 64) - 1


def fmix64(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def rng_words(seed: int, start: int, count: int) -> np.ndarray:
    base = (seed * SEED_MUL) & M64
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(base) + i * np.uint64(GAMMA)
    return fmix64(z)


def scale_f16(u16: np.ndarray) -> np.ndarray:
    """fp16 bits of 1e-3 + 9e-3 * (u16 / 65536), fp32 multiply then add, RNE."""
    u = u16.astype(np.float32) * np.float32(1.0 / 65536.0)
    v = np.float32(1e-3) + np.float32(9e-3) * u
    return v.astype(np.float16).view(np.uint16)


def synth_q4k(n_blocks: int, seed: int) -> np.ndarray:
    w = rng_words(seed, 0, n_blocks * 18).reshape(n_blocks, 18)
    out = w.view(np.uint8).reshape(n_blocks, 144).copy()
    lo = (w[:, 0] & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    d = scale_f16(lo & np.uint32(0xFFFF))
    dmin = scale_f16(lo >> np.uint32(16))
    out[:, 0:2] = d.reshape(-1, 1).view(np.uint8)
    out[:, 2:4] = dmin.reshape(-1, 1).view(np.uint8)
    return out.reshape(-1)


def synth_q6k(n_blocks: int, seed: int) -> np.ndarray:
    w = rng_words(seed, 0, n_blocks * 27).reshape(n_blocks, 27)
    out = w.view(np.uint8).reshape(n_blocks, 216)[:, :210].copy()
    raw = out[:, 192:208].astype(np.int32)
    out[:, 192:208] = ((raw & 63) - 32).astype(np.int8).view(np.uint8)
    d = scale_f16((w[:, 26] & np.uint64(0xFFFF)).astype(np.uint32))
    out[:, 208:210] = d.reshape(-1, 1).view(np.uint8)
    return out.reshape(-1)


def normal_f32(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """N(mean, std) via numpy's PCG64 (host-only inputs such as activations)."""
    rng = np.random.default_rng(seed)
    return (mean + std * rng.standard_normal(n)).astype(np.float32)


def zipf_bias(n_experts: int, s: float, seed: int) -> np.ndarray:
    """Router logit bias log p_rank(e) with p_r proportional to r**-s over a
    seeded permutation of the experts (expert perm[r-1] has rank r).  The
    bias enters through the router GEMV itself: the caller sets the last
    activation feature of every token to 1 and the router's last column to
    this bias, so logit_e = sum_{j<H-1} W[e][j] x[j] + bias_e."""
    perm = np.random.default_rng(seed).permutation(n_experts)
    r = np.arange(1, n_experts + 1, dtype=np.float64)
    p = r ** -s
    p /= p.sum()
    bias = np.empty(n_experts, np.float64)
    bias[perm] = np.log(p)
    return bias.astype(np.float32)
