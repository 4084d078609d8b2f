// q4k_mfma.h — Q4_K weights on the fp16 MFMA (v_mfma_f32_16x16x32_f16) with
// exact operands: a lane unpacks its quarter of a superblock row into the
// sub-block scale times the 4-bit code, sc * q <= 63 * 15, exact in fp16; the
// superblock scale d and the min term dmin * m * sum(x) are applied to the
// fp32 partial sums afterwards.  K is relabelled so that lane group g holds
// qs bytes [32 g, 32 g + 32): sub-block 2 g in their low nibbles, 2 g + 1 in
// their high nibbles (dequant_q4k_cpu.c:111-121); MFMA i takes elements
// 64 g + 8 i .. + 7 of the superblock from every lane group.  Used by the
// batched greedy head (verify.hip) and the small-batch gate/up kernel.
#pragma once

#include "bread_device.h"

typedef _Float16 q4m_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 q4m_half2 __attribute__((ext_vector_type(2)));
typedef float q4m_f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t Q4M_MAGIC = 0x64646464u;  // fp16 0x64xx = 1024 + xx

// Four nibbles (bytes of v, each < 16) as two packed fp16 pairs of sc * q.
__device__ __forceinline__ void q4m_scq(uint32_t v, q4m_half2 sc, q4m_half2 nsc, uint32_t &p0, uint32_t &p1)
{
    const q4m_half2 a = __builtin_bit_cast(q4m_half2, __builtin_amdgcn_perm(Q4M_MAGIC, v, 0x07010700u));
    const q4m_half2 b = __builtin_bit_cast(q4m_half2, __builtin_amdgcn_perm(Q4M_MAGIC, v, 0x07030702u));
    p0 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(a, sc, nsc));  // (1024 + q) sc - 1024 sc
    p1 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(b, sc, nsc));
}

// Eight consecutive elements' sc * q: the low (hi = 0) or high nibbles of
// the bytes in (a, b).
__device__ __forceinline__ q4m_half8 q4m_b8(uint32_t a, uint32_t b, int hi, q4m_half2 sc, q4m_half2 nsc)
{
    uint4 r;
    q4m_scq((a >> (4 * hi)) & 0x0F0F0F0Fu, sc, nsc, r.x, r.y);
    q4m_scq((b >> (4 * hi)) & 0x0F0F0F0Fu, sc, nsc, r.z, r.w);
    return __builtin_bit_cast(q4m_half8, r);
}

// A workgroup barrier that publishes the waves' LDS writes but leaves their
// global loads in flight (__syncthreads would wait for every outstanding
// load, the ring's tiles ahead included).  The asm memory clobber and the
// scheduling barrier keep LDS accesses and the ring's loads on their side.
__device__ __forceinline__ void q4m_bar()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// A lane's head and qs quarters of one superblock (row c, quarter g).
struct Q4mRaw {
    uint4 head;  // d, dmin, scales
    uint4 q0;    // qs bytes [32 g, 32 g + 16)
    uint4 q1;    // qs bytes [32 g + 16, 32 g + 32)
};

__device__ __forceinline__ void q4m_load(Q4mRaw &r, const uint8_t *sb, int g)
{
    r.head = *reinterpret_cast<const uint4 *>(sb);
    r.q0 = *reinterpret_cast<const uint4 *>(sb + 16 + 32 * g);
    r.q1 = *reinterpret_cast<const uint4 *>(sb + 32 + 32 * g);
}
