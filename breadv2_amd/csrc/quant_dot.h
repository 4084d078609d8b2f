// quant_dot.h — per-lane partial dot products of one quantized row with an
// activation vector, for the generic (any rows/cols) matvec kernels.
//
// Lane layout (wave64): 8 lanes per superblock, 8 superblocks per step.
//   Q4_K: lane chunk c = lane%8 owns qs bytes [16c, 16c+16), i.e. sub-block
//         pair j = c/2, low nibbles -> elements 64j+16(c%2)+[0,16),
//         high nibbles -> elements 64j+32+16(c%2)+[0,16)
//         (element order of dequant_q4k_cpu.c:111-121).
//   Q6_K: lane unit u = lane%8 owns half n = u/4 and l in [8t, 8t+8),
//         t = u%4: ql bytes 64n+l and 64n+32+l, qh byte 32n+l
//         -> elements 128n + 32s + l, s = 0..3 (dequant_q4k_cpu.c:155-170).
// The caller reduces the lane partials over the wave.
#pragma once

#include "bread_device.h"

// ---- activation loads (x must be 16-byte aligned; offsets are multiples of 8)

__device__ __forceinline__ void load_x8(const float *x, int off, float (&v)[8])
{
    const float4 a = *reinterpret_cast<const float4 *>(x + off);
    const float4 b = *reinterpret_cast<const float4 *>(x + off + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void load_x8(const uint16_t *x, int off, float (&v)[8])
{
    const uint4 a = *reinterpret_cast<const uint4 *>(x + off);
    v[0] = h2f(a.x); v[1] = h2f(a.x >> 16); v[2] = h2f(a.y); v[3] = h2f(a.y >> 16);
    v[4] = h2f(a.z); v[5] = h2f(a.z >> 16); v[6] = h2f(a.w); v[7] = h2f(a.w >> 16);
}

template <typename XT>
__device__ __forceinline__ void load_x16(const XT *x, int off, float (&v)[16])
{
    float a[8], b[8];
    load_x8(x, off, a);
    load_x8(x, off + 8, b);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        v[i] = a[i];
        v[8 + i] = b[i];
    }
}

// ---- Q4_K: one lane's 32 weights of a superblock

// hd = bytes 0..15 of the superblock (d, dmin, scales), q = its 16-byte qs
// chunk c, j = c/2.  Returns d*sc0*sum(lo*xl) - dmin*m0*sum(xl)
//                           + d*sc1*sum(hi*xh) - dmin*m1*sum(xh).
__device__ __forceinline__ float q4k_chunk_dot(uint4 hd, uint4 q, uint32_t j, const float (&xl)[16],
                                               const float (&xh)[16])
{
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * j, hd.y, hd.z, hd.w, sc0, m0);
    scale_min_k4(2 * j + 1, hd.y, hd.z, hd.w, sc1, m1);
    const float d = h2f(hd.x);
    const float dmin = h2f(hd.x >> 16);
    float al = 0.f, ah = 0.f, sl = 0.f, sh = 0.f;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t lo = qw[t] & 0x0F0F0F0Fu;
        const uint32_t hi = (qw[t] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            al = fmaf((float)byte_of(lo, k), xl[4 * t + k], al);
            ah = fmaf((float)byte_of(hi, k), xh[4 * t + k], ah);
            sl += xl[4 * t + k];
            sh += xh[4 * t + k];
        }
    }
    return (d * (float)sc0) * al - (dmin * (float)m0) * sl + (d * (float)sc1) * ah -
           (dmin * (float)m1) * sh;
}

template <typename XT>
__device__ __forceinline__ float q4k_row_partial(const uint8_t *row, int nb, const XT *x, int lane)
{
    const int c = lane & 7;
    const uint32_t j = (uint32_t)c >> 1;
    const int hh = c & 1;
    float acc = 0.f;
    for (int b = lane >> 3; b < nb; b += 8) {
        const uint8_t *blk = row + (size_t)b * Q4K_BYTES;
        const uint4 hd = ld_b128(blk);
        const uint4 q = ld_b128(blk + 16 + 16 * c);
        float xl[16], xh[16];
        const int base = b * QK + 64 * (int)j + 16 * hh;
        load_x16(x, base, xl);
        load_x16(x, base + 32, xh);
        acc += q4k_chunk_dot(hd, q, j, xl, xh);
    }
    return acc;
}

// ---- Q6_K: one lane's 32 weights of a superblock

// Bytes l..l+3 of ql (low half a, high half b) and qh -> four dwords of
// 6-bit values, one byte per weight, for s = 0..3 (element 32s + l).
__device__ __forceinline__ void q6k_unpack(uint32_t a, uint32_t b, uint32_t h, uint32_t (&q)[4])
{
    q[0] = (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
    q[1] = (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
    q[2] = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
    q[3] = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
}

// Signed scale sc[8n + i + 2s] from the 8 scale bytes of half n.
__device__ __forceinline__ float q6k_scale(uint2 scw, uint32_t p)
{
    const uint32_t w = p < 4 ? scw.x : scw.y;
    return (float)(int8_t)byte_of(w, p & 3u);
}

// xs[s][k] = x at element 32s + l0 + k of the half.  Returns
// d * sum_s sc_s * sum_k (q - 32) * xs[s][k].
__device__ __forceinline__ float q6k_unit_dot(uint2 ql0, uint2 ql1, uint2 qh, uint2 scw, uint32_t i,
                                              float d, const float (&xs)[4][8])
{
    float A[4] = {0.f, 0.f, 0.f, 0.f}, X[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 2; w++) {
        uint32_t q[4];
        q6k_unpack(w ? ql0.y : ql0.x, w ? ql1.y : ql1.x, w ? qh.y : qh.x, q);
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                A[s] = fmaf((float)byte_of(q[s], k), xs[s][4 * w + k], A[s]);
                X[s] += xs[s][4 * w + k];
            }
    }
    float r = 0.f;
#pragma unroll
    for (int s = 0; s < 4; s++) r = fmaf(q6k_scale(scw, i + 2 * s), fmaf(-32.f, X[s], A[s]), r);
    return d * r;
}

// q6k_unit_dot with the activation sums X[s] = sum_k xs[s][k] precomputed.
__device__ __forceinline__ float q6k_unit_dot_sx(uint2 ql0, uint2 ql1, uint2 qh, uint2 scw, uint32_t i, float d,
                                                 const float (&xs)[4][8], const float (&X)[4])
{
    float A[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 2; w++) {
        uint32_t q[4];
        q6k_unpack(w ? ql0.y : ql0.x, w ? ql1.y : ql1.x, w ? qh.y : qh.x, q);
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int k = 0; k < 4; k++) A[s] = fmaf((float)byte_of(q[s], k), xs[s][4 * w + k], A[s]);
    }
    float r = 0.f;
#pragma unroll
    for (int s = 0; s < 4; s++) r = fmaf(q6k_scale(scw, i + 2 * s), fmaf(-32.f, X[s], A[s]), r);
    return d * r;
}

template <typename XT>
__device__ __forceinline__ float q6k_row_partial(const uint8_t *row, int nb, const XT *x, int lane)
{
    const int u = lane & 7;
    const int n = u >> 2, t = u & 3;
    const uint32_t i = (uint32_t)t >> 1;
    float acc = 0.f;
    for (int b = lane >> 3; b < nb; b += 8) {
        const uint8_t *blk = row + (size_t)b * Q6K_BYTES;
        const uint2 ql0 = ld8_a2(blk + 64 * n + 8 * t);
        const uint2 ql1 = ld8_a2(blk + 64 * n + 32 + 8 * t);
        const uint2 qh = ld8_a2(blk + 128 + 32 * n + 8 * t);
        const uint2 scw = ld8_a2(blk + 192 + 8 * n);
        const float d = h2f(ld16_a2(blk + 208));
        float xs[4][8];
#pragma unroll
        for (int s = 0; s < 4; s++) load_x8(x, b * QK + 128 * n + 32 * s + 8 * t, xs[s]);
        acc += q6k_unit_dot(ql0, ql1, qh, scw, i, d, xs);
    }
    return acc;
}

// ---- Q8_0: one lane per 34-byte block of 32 weights

template <typename XT>
__device__ __forceinline__ float q80_row_partial(const uint8_t *row, int nb32, const XT *x, int lane)
{
    float acc = 0.f;
    for (int b = lane; b < nb32; b += WAVE) {
        const uint8_t *blk = row + (size_t)b * Q80_BYTES;
        const float d = h2f(ld16_a2(blk));
        float s = 0.f;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint2 q = ld8_a2(blk + 2 + 8 * m);
            float xv[8];
            load_x8(x, b * Q80_ELEMS + 8 * m, xv);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s = fmaf((float)(int8_t)byte_of(q.x, k), xv[k], s);
                s = fmaf((float)(int8_t)byte_of(q.y, k), xv[4 + k], s);
            }
        }
        acc = fmaf(d, s, acc);
    }
    return acc;
}

// q4k_chunk_dot against x in 16-bit block fixed point: over a 32-element
// block, x_i ~= s * (256 * hi_i + lo_i) with hi, lo int8, packed four
// elements to a word in element order (lh / ll: the high / low bytes of the
// lane's low-nibble run, hh / hl: of its high-nibble run; s_lo, s_hi their
// block scales).  sl, sh are the fp32 sums of the two runs, so the min term
// is exact.  The nibble products accumulate in v_dot4_i32_i8 (q <= 15 fits a
// signed byte; |sum| < 2^23, so the integer sums are exact and convert to
// fp32 exactly): 7 instructions per 8 weights against 19 for the fp32 form.
// The (scale, min) pairs of sub-blocks 2j and 2j+1 of a Q4_K superblock as
// bytes [sc0, sc1, m0, m1], without branches on j: get_scale_min_k4
// (dequant_q4k_cpu.c:70-79) reads, for j < 2, the low six bits of bytes
// 2j, 2j+1, 2j+4, 2j+5 and, for j >= 2 (r = 2j - 4), the nibbles of bytes
// 8+r, 9+r with the top two bits of bytes r, r+1 (scales) and 4+r, 5+r
// (mins).  Both cases gather with v_perm_b32.
__device__ __forceinline__ uint32_t q4k_scale_pair(uint4 hd, uint32_t j)
{
    const uint32_t jj = (j & 1u) * 0x02020202u;
    const uint32_t h = __builtin_amdgcn_perm(hd.z, hd.y, 0x05040100u + jj);
    if (j < 2) return h & 0x3F3F3F3Fu;
    const uint32_t l = __builtin_amdgcn_perm(hd.w, hd.w, 0x01000100u + jj);
    return (l & 0x00000F0Fu) | ((l >> 4) & 0x0F0F0000u) | ((h >> 2) & 0x30303030u);
}

__device__ __forceinline__ float q4k_chunk_dot_q16(uint4 hd, uint4 q, uint32_t j, uint4 lh, uint4 ll, uint4 hh,
                                                   uint4 hl, float s_lo, float s_hi, float sl, float sh)
{
    const uint32_t scm = q4k_scale_pair(hd, j);
    const uint32_t sc0 = byte_of(scm, 0), sc1 = byte_of(scm, 1), m0 = byte_of(scm, 2), m1 = byte_of(scm, 3);
    const float d = h2f(hd.x);
    const float dmin = h2f(hd.x >> 16);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const uint32_t xlh[4] = {lh.x, lh.y, lh.z, lh.w}, xll[4] = {ll.x, ll.y, ll.z, ll.w};
    const uint32_t xhh[4] = {hh.x, hh.y, hh.z, hh.w}, xhl[4] = {hl.x, hl.y, hl.z, hl.w};
    // 256 sum(q hi) + sum(q lo) in one chain per nibble half (exact: below
    // 2^23), one zeroed accumulator each
    int a_l = 0, a_h = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        a_l = __builtin_amdgcn_sdot4((int)(qw[t] & 0x0F0F0F0Fu), (int)xlh[t], a_l, false);
        a_h = __builtin_amdgcn_sdot4((int)((qw[t] >> 4) & 0x0F0F0F0Fu), (int)xhh[t], a_h, false);
    }
    a_l *= 256;
    a_h *= 256;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        a_l = __builtin_amdgcn_sdot4((int)(qw[t] & 0x0F0F0F0Fu), (int)xll[t], a_l, false);
        a_h = __builtin_amdgcn_sdot4((int)((qw[t] >> 4) & 0x0F0F0F0Fu), (int)xhl[t], a_h, false);
    }
    const float al = (float)a_l * s_lo;
    const float ah = (float)a_h * s_hi;
    return (d * (float)sc0) * al - (dmin * (float)m0) * sl + (d * (float)sc1) * ah -
           (dmin * (float)m1) * sh;
}

// q4k_chunk_dot with the activation sums over the two 16-element runs
// precomputed (they are the same for every row a lane visits).
__device__ __forceinline__ float q4k_chunk_dot_sx(uint4 hd, uint4 q, uint32_t j, const float (&xl)[16],
                                                  const float (&xh)[16], float sl, float sh)
{
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * j, hd.y, hd.z, hd.w, sc0, m0);
    scale_min_k4(2 * j + 1, hd.y, hd.z, hd.w, sc1, m1);
    const float d = h2f(hd.x);
    const float dmin = h2f(hd.x >> 16);
    float al = 0.f, ah = 0.f;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t lo = qw[t] & 0x0F0F0F0Fu;
        const uint32_t hi = (qw[t] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            al = fmaf((float)byte_of(lo, k), xl[4 * t + k], al);
            ah = fmaf((float)byte_of(hi, k), xh[4 * t + k], ah);
        }
    }
    return (d * (float)sc0) * al - (dmin * (float)m0) * sl + (d * (float)sc1) * ah -
           (dmin * (float)m1) * sh;
}

typedef _Float16 qd_half2 __attribute__((ext_vector_type(2)));

// Activations in 16-bit block fixed point for the small-batch gate/up
// kernel (H = 2048): per 32-column block s = max|x| / 32511 and x ~= s (256
// hi + lo) with hi, lo signed bytes, plus fp32 sums of 16-column runs (the
// min term).  One token's record, XQ_TOKEN_BYTES bytes: hi bytes [H / 4]
// words (4 columns a word), lo bytes [H / 4], block scales [H / 32], run sums
// [H / 16].
constexpr int XQ_H = 2048;
constexpr int XQ_HI = 0, XQ_LO = XQ_H, XQ_SC = 2 * XQ_H, XQ_SUM = 2 * XQ_H + XQ_H / 8;
constexpr int XQ_TOKEN_BYTES = 2 * XQ_H + XQ_H / 8 + XQ_H / 4;

// Thread i of 256 consecutive threads holds columns 8 i .. 8 i + 7 of one
// token in v and writes their part of the token's record (blocks of 32
// columns are four consecutive lanes).  Exactly the conversion the gate/up
// kernel did itself: the same block maxima, scale, rounding and sum order.
__device__ __forceinline__ void xq16_store(const float (&v)[8], int i, uint8_t *rec)
{
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(v[k]));
    m = fmaxf(m, dpp_f<0xB1>(m));  // quad_perm [1,0,3,2]
    m = fmaxf(m, dpp_f<0x4E>(m));  // quad_perm [2,3,0,1]
    const float inv = m > 0.f ? 32511.0f / m : 0.f;
    uint32_t hw[2], lw[2];
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        hw[hf] = 0;
        lw[hf] = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int q = __float2int_rn(v[4 * hf + k] * inv);
            const int hi = (q + 128) >> 8;
            const int lo = q - 256 * hi;
            hw[hf] |= ((uint32_t)hi & 0xFFu) << (8 * k);
            lw[hf] |= ((uint32_t)lo & 0xFFu) << (8 * k);
        }
    }
    *reinterpret_cast<uint2 *>(rec + XQ_HI + 8 * i) = make_uint2(hw[0], hw[1]);
    *reinterpret_cast<uint2 *>(rec + XQ_LO + 8 * i) = make_uint2(lw[0], lw[1]);
    if ((i & 3) == 0) reinterpret_cast<float *>(rec + XQ_SC)[i >> 2] = m / 32511.0f;
    const float r0 = (v[0] + v[1]) + (v[2] + v[3]), r1 = (v[4] + v[5]) + (v[6] + v[7]);
    float r = r0 + r1;
    r += dpp_f<0xB1>(r);
    if ((i & 1) == 0) reinterpret_cast<float *>(rec + XQ_SUM)[i >> 1] = r;
}
