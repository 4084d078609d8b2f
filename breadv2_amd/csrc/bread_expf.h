// bread_expf.h — expf exactly as the host C library computes it, for the
// routing softmax (cpu_softmax, layer_ops.cu:222-229, calls the C library's
// expf).  The algorithm is the one glibc 2.35 ships for x86-64 (ARM
// optimized-routines' expf, the build with fused multiply-adds that glibc
// selects on CPUs with FMA): with N = 32, k = round(x N / ln 2) by the
// 1.5 * 2^52 shift trick, r = x N / ln 2 - k, 2^(k/N) assembled from a
// 32-entry table of 2^(i/N), and a cubic in r, all in double with fused
// multiply-adds, rounded once to float.  Inputs beyond the main range follow
// the same special cases (NaN and +inf propagate, -inf and x < log(2^-150)
// give 0, x > log(2^128) gives +inf).
//
// The table holds the correctly rounded doubles of 2^(i/32) minus i << 47
// (so that adding k << 47 sets the exponent); the polynomial coefficients
// are the published minimax fit.  This restatement was compared with the
// host's expf on all 2^32 float inputs and agrees bit for bit;
// tests/test_expf.py re-checks it on the host build against the oracle's
// libm at every run.
#pragma once

#include <stdint.h>

#include <hip/hip_runtime.h>

// The value unchanged; in GPU code an empty asm makes it opaque, so a
// constant is materialised at its use rather than hoisted into a register
// held across the caller's loops (in the decode kernel, a spill).
__host__ __device__ inline uint32_t fresh_u32(uint32_t v)
{
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(v));
#endif
    return v;
}

// The 32 table entries (used through libm_expf_t; a caller may copy them
// to LDS once and pass that copy, so the lookup does not wait on memory).
__host__ __device__ inline uint64_t libm_expf_tab(int i)
{
    constexpr uint64_t tab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    return tab[i & 31];
}

// The computation, with entry i of the table from tab(i).
template <class Tab>
__host__ __device__ inline float libm_expf_g(float x, Tab tab)
{
#pragma clang fp contract(off)
    constexpr double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
    constexpr double shift = 0x1.8p+52;
    constexpr double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    // c1 = 0x1.ebfce50fac4f3p-3 / 32^2 (bits 0x3f2ebfce50fac4f3), below
    constexpr double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7FFu;
    if (abstop >= 0x42Bu) {                      // |x| >= 88 or not finite
        if (ux == 0xFF800000u) return 0.0f;      // -inf
        if (abstop >= 0x7F8u) return x + x;      // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = __builtin_bit_cast(double, tab((int)(ki % 32)) + (ki << 47));
    const double c1 = __builtin_bit_cast(double, ((uint64_t)fresh_u32(0x3f2ebfceu) << 32) | fresh_u32(0x50fac4f3u));
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

struct LibmExpfConstTab {
    __host__ __device__ uint64_t operator()(int i) const { return libm_expf_tab(i); }
};

struct LibmExpfPtrTab {
    const uint64_t *t;
    __host__ __device__ uint64_t operator()(int i) const { return t[i]; }
};

__host__ __device__ inline float libm_expf(float x)
{
    return libm_expf_g(x, LibmExpfConstTab{});
}

// libm_expf with a copy of the table at tab (libm_expf_tab's 32 entries,
// e.g. in LDS).
__host__ __device__ inline float libm_expf_t(float x, const uint64_t *tab)
{
    return libm_expf_g(x, LibmExpfPtrTab{tab});
}
