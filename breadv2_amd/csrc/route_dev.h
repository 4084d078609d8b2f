// route_dev.h — device routing pieces shared by the multi-kernel path and the
// single-launch decode kernel: router row dot and the softmax / top-k wave.
#pragma once

#include "bread_device.h"
#include "bread_expf.h"

// Selection key of a softmax output p: probabilities are in [0, 1] or NaN
// (exp(l - max) / sum), so their bit patterns order like the values; numbers
// map to bits + 2, NaN to 1 (below every number), and 0 marks an entry that
// is taken or out of range.
__device__ __forceinline__ uint32_t prob_key(float p)
{
    return p != p ? 1u : __builtin_bit_cast(uint32_t, p) + 2u;
}

__device__ __forceinline__ float prob_from_key(uint32_t k)
{
    return k == 1u ? __builtin_bit_cast(float, 0x7FC00000u) : __builtin_bit_cast(float, k - 2u);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b)
{
    return a > b ? a : b;
}

// Unsigned max over the wave (lanes outside a DPP row read 0, the identity).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = umax32(v, dpp_u32<0xB1>(v));
    v = umax32(v, dpp_u32<0x4E>(v));
    v = umax32(v, dpp_u32<0x141>(v));
    v = umax32(v, dpp_u32<0x140>(v));
    lane_pair p = swap16(v);
    v = umax32(p.a, p.b);
    p = swap32(v);
    return __builtin_amdgcn_readfirstlane(umax32(p.a, p.b));
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, true);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double readlane_f64(double v, int l)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Inclusive prefix sum over the wave's lanes in lane order (fp64): shifts
// of 1, 2, 4, 8 inside each 16-lane row (lanes without a source read 0),
// then the totals of the rows below added.
__device__ __forceinline__ double wave_scan_incl_f64(double v)
{
    v += dpp_f64<0x111>(v);  // row_shr:1
    v += dpp_f64<0x112>(v);  // row_shr:2
    v += dpp_f64<0x114>(v);  // row_shr:4
    v += dpp_f64<0x118>(v);  // row_shr:8
    const double r0 = readlane_f64(v, 15), r1 = readlane_f64(v, 31), r2 = readlane_f64(v, 47);
    const int row = lane_id() >> 4;
    double off = 0.0;
    if (row >= 1) off += r0;
    if (row >= 2) off += r1;
    if (row >= 3) off += r2;
    return v + off;
}

// Inclusive prefix sum over the wave's lanes in lane order (fp32; as the
// fp64 form).
__device__ __forceinline__ float wave_scan_incl_f32(float v)
{
    v += dpp_f<0x111>(v);  // row_shr:1
    v += dpp_f<0x112>(v);  // row_shr:2
    v += dpp_f<0x114>(v);  // row_shr:4
    v += dpp_f<0x118>(v);  // row_shr:8
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 47));
    const int row = lane_id() >> 4;
    float off = 0.f;
    if (row >= 1) off += r0;
    if (row >= 2) off += r1;
    if (row >= 3) off += r2;
    return v + off;
}

// Certified routing for a router dot computed out of the reference's order.
//
// The reference sums each logit sequentially in fp32 (one_layer.cu:969-971):
// s_0 = 0, s_k = fl(s_{k-1} + fl(w_k x_k)).  Running-error analysis of that
// recursion gives, with u = 2^-24, A = sum |w_k x_k| and S = sum_k |s*_k|
// over the exact prefix sums s*_k:
//   |s_n - s*_n| <= u (S + c_H A) + 2 n 2^-150,
//   c_H = 1 + u n + u n^2 (1 + u) / (1 - u n),
// (each add errs by at most u |s_k|, each product by u |w_k x_k| plus
// underflow; sum |s_k| <= S + n (u A + n u M) with M = max |s_k|).  A caller
// computing the dot exactly enough (fp64 products and sums) and tracking S
// from its prefix sums obtains a radius R with |its fp32 logit - s_n| <= R
// (its own rounding error included).
// Selection by the reference (expf faithful, then division by the same sum)
// orders p_a > p_b strictly whenever s_a - s_b > tau, tau = 12 u (1 + max|l| +
// R); so when every consecutive pair of the top K+1 (in the order selected
// here) is more than 2 R_max + tau apart in the fast logits, the reference
// selects the same experts in the same order.
// The tau argument bounds relative errors, so it needs the probabilities it
// compares to be normal floats: the selected ranks' logits lie within
// CERT_SPREAD of the largest (then p >= e^-80 / 256 > 2^-126); an expert
// further below has a smaller probability in any case (subnormal or zero
// when below 2^-126, otherwise ordered by tau).  Wider spreads are left to
// the reference-order recomputation.
constexpr float CERT_U = 5.9604645e-8f;  // 2^-24
constexpr float CERT_SPREAD = 80.f;

// Selection key of a fast logit: its bits mapped so that unsigned order is
// numeric order, dropped to 30 bits (2 or more; NaN 1).  The passes order
// the fast logits themselves, not their probabilities: a softmax is
// monotone, and the certificate only vouches for ranks whose logits are far
// more than the 4 ulps this drops apart, so the probabilities the reference
// computes order them the same way.
__device__ __forceinline__ uint32_t logit_key(float l)
{
    if (l != l) return 1u;
    const uint32_t u = __builtin_bit_cast(uint32_t, l);
    return ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) >> 2;
}

__device__ __forceinline__ float cert_c_h(int n)
{
    const double u = 5.9604644775390625e-8, dn = (double)n;
    return (float)((1.0 + u * dn + u * dn * dn * (1.0 + u) / (1.0 - u * dn)) * (1.0 + 1e-6));
}

// The reference's sequential fp32 dot ((0 + w_0 x_0) + w_1 x_1) + ... over n
// values in LDS (n % 16 == 0), every product rounded before its add.  All
// lanes run the same chain (broadcast reads).  The adds of a block of 8
// alternate with the products of the next block, whose operands were read
// a block earlier, so the dependent adds are not delayed by LDS latency
// (48 registers of operands and products: it runs inside kernels held to 128).
__device__ __forceinline__ void lds_block8(const float *w, const float *x, int o, float (&wv)[8], float (&xv)[8])
{
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const float4 a = *reinterpret_cast<const float4 *>(w + o + 4 * q);
        const float4 b = *reinterpret_cast<const float4 *>(x + o + 4 * q);
        wv[4 * q] = a.x; wv[4 * q + 1] = a.y; wv[4 * q + 2] = a.z; wv[4 * q + 3] = a.w;
        xv[4 * q] = b.x; xv[4 * q + 1] = b.y; xv[4 * q + 2] = b.z; xv[4 * q + 3] = b.w;
    }
}

__device__ __forceinline__ float seq_dot_lds(const float *w, const float *x, int n)
{
#pragma clang fp contract(off)
    const int nb = n / 8;
    float pa[8], pb[8], wa[8], xa[8], wb[8], xb[8];
    float acc = 0.f;
    lds_block8(w, x, 0, wa, xa);
#pragma unroll
    for (int j = 0; j < 8; j++) pa[j] = wa[j] * xa[j];
    lds_block8(w, x, 8, wa, xa);
    // two blocks an iteration with the register roles swapped, no copies:
    // pa holds block b's products, (wa, xa) block b+1's operands
    for (int b = 0; b < nb; b += 2) {
        lds_block8(w, x, 8 * min(b + 2, nb - 1), wb, xb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            acc = acc + pa[j];
            pb[j] = wa[j] * xa[j];
            __builtin_amdgcn_sched_barrier(0);
        }
        lds_block8(w, x, 8 * min(b + 3, nb - 1), wa, xa);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            acc = acc + pb[j];
            pa[j] = wb[j] * xb[j];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    return acc;
}

// The reference's sequential fp32 sum ((acc + p_0) + p_1) + ... of n values
// in LDS (acc 0 unless a previous part's sum continues; n % 16 == 0; each
// lane may read its own array).  Reads run two blocks of 8 ahead of the
// dependent adds.
__device__ __forceinline__ void lds_read8(const float *p, int o, float (&v)[8])
{
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const float4 a = *reinterpret_cast<const float4 *>(p + o + 4 * q);
        v[4 * q] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
    }
}

__device__ __forceinline__ float seq_sum_lds(const float *p, int n, float acc = 0.f)
{
#pragma clang fp contract(off)
    const int nb = n / 8;
    float va[8], vb[8];
    lds_read8(p, 0, va);
    for (int b = 0; b < nb; b += 2) {
        lds_read8(p, 8 * min(b + 1, nb - 1), vb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            acc = acc + va[j];
            __builtin_amdgcn_sched_barrier(0);
        }
        lds_read8(p, 8 * min(b + 2, nb - 1), va);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            acc = acc + vb[j];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    return acc;
}

// Softmax over E logits held as p[v] = logit lane + 64 v, to selection keys.
// Restates cpu_softmax (layer_ops.cu:222-229):
//   - max is taken over numbers; a NaN in entry 0 makes it NaN, as the
//     reference's `x[i] > mx` scan starting from x[0] does;
//   - every exponential and the division use the device expf and IEEE
//     division; the sum is a wave reduction (not sequential), so p can differ
//     from the host's in the last bits.
template <int MAXV>
// Returns the max and the sum used (the key of any logit x is
// prob_key(expf(x - max) / sum)).
__device__ __forceinline__ float2 softmax_keys(float (&p)[MAXV], int E, uint32_t (&key)[MAXV])
{
    const int lane = lane_id();
    float mx = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        if (i < E && p[v] == p[v]) mx = fmaxf(mx, p[v]);
    }
    mx = wave_max(mx);
    const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p[0]), 0));
    if (l0 != l0) mx = l0;
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        p[v] = i < E ? expf(p[v] - mx) : 0.f;
        s += p[v];
    }
    s = wave_sum(s);
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        key[v] = i < E ? prob_key(p[v] / s) : 0u;
    }
    return make_float2(mx, s);
}

// cpu_softmax (layer_ops.cu:222-229) exactly as the host computes it, to
// selection keys: the max as its first-element scan gives it (softmax_keys),
// e_i = expf(x_i - max) with the C library's expf (libm_expf), the sum
// s = e_0 + e_1 + ... in index order, p_i = e_i / s by IEEE division.  With
// logits equal to the host's, every probability and therefore every key is
// bit-identical.  s_e: LDS scratch of at least E floats, private to the
// wave (every lane then sums the same values in the same order).
template <int MAXV>
__device__ __forceinline__ void softmax_keys_exact(float (&p)[MAXV], int E, uint32_t (&key)[MAXV], float *s_e)
{
#pragma clang fp contract(off)
    const int lane = lane_id();
    float mx = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        if (i < E && p[v] == p[v]) mx = fmaxf(mx, p[v]);
    }
    mx = wave_max(mx);
    const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p[0]), 0));
    if (l0 != l0) mx = l0;
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        if (i < E) {
            p[v] = libm_expf(p[v] - mx);
            s_e[i] = p[v];
        }
    }
    // the wave's own LDS stores are performed in order before its loads
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int e16 = E & ~15;
    float s = e16 ? seq_sum_lds(s_e, e16) : 0.f;
    for (int i = e16; i < E; i++) s += s_e[i];
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int j = lane + WAVE * v;
        key[v] = j < E ? prob_key(p[v] / s) : 0u;
    }
    __builtin_amdgcn_wave_barrier();
}

// One pass of cpu_topk (layer_ops.cu:231-243): the largest key, equal keys
// to the lower index (NaN ranks below every number; a pass that finds only
// NaN takes the lowest unused index, where the reference is undefined).
// Marks the winner used; returns its index (wave-uniform) and key in M.
template <int MAXV>
__device__ __forceinline__ int select_round(uint32_t (&key)[MAXV], uint32_t &M)
{
    const int lane = lane_id();
    uint32_t lm = key[0];
#pragma unroll
    for (int v = 1; v < MAXV; v++) lm = umax32(lm, key[v]);
    M = wave_max_u32(lm);
    int win = 0;
#pragma unroll
    for (int v = MAXV - 1; v >= 0; v--) {
        const uint64_t b = __builtin_amdgcn_ballot_w64(key[v] == M);
        if (b) win = WAVE * v + (int)__builtin_ctzll(b);
    }
#pragma unroll
    for (int v = 0; v < MAXV; v++)
        if (win == lane + WAVE * v) key[v] = 0u;
    return win;
}

// Rank-order sum of the K selected probabilities (lane k < K holds rank k's
// key), then renormalisation when the sum is positive (layer_ops.cu:244-249).
__device__ __forceinline__ float renorm_weight(uint32_t my_key, int K)
{
    float my_w = prob_from_key(my_key);
    float w_sum = 0.f;
    for (int k = 0; k < K; k++)
        w_sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), k));
    if (w_sum > 0.f) my_w = my_w / w_sum;
    return my_w;
}

// One wave: softmax over E logits, K selection passes, renormalisation.
// Entry i = lane + 64 v lives in p[v] of that lane; E <= 64 * MAXV and
// E >= K.  Lane k < K returns idx_k / w_k (rank order).
template <int MAXV>
__device__ __forceinline__ void topk_wave_vals(float (&p)[MAXV], int E, int K, int &idx_k, float &w_k)
{
    const int lane = lane_id();
    uint32_t key[MAXV];
    softmax_keys<MAXV>(p, E, key);
    int my_idx = 0;
    uint32_t my_key = 0;
    for (int k = 0; k < K; k++) {
        uint32_t M;
        const int win = select_round<MAXV>(key, M);
        if (lane == k) {
            my_idx = win;
            my_key = M;
        }
    }
    idx_k = my_idx;
    w_k = renorm_weight(my_key, K);
}

// topk_wave_vals with the host's softmax arithmetic (softmax_keys_exact):
// given the host's logits, indices and weights are bit-identical to
// cpu_softmax + cpu_topk (layer_ops.cu:222-250).
template <int MAXV>
__device__ __forceinline__ void topk_wave_vals_exact(float (&p)[MAXV], int E, int K, float *s_e, int &idx_k,
                                                     float &w_k)
{
    const int lane = lane_id();
    uint32_t key[MAXV];
    softmax_keys_exact<MAXV>(p, E, key, s_e);
    int my_idx = 0;
    uint32_t my_key = 0;
    for (int k = 0; k < K; k++) {
        uint32_t M;
        const int win = select_round<MAXV>(key, M);
        if (lane == k) {
            my_idx = win;
            my_key = M;
        }
    }
    idx_k = my_idx;
    w_k = renorm_weight(my_key, K);
}

template <int MAXV>
__device__ __forceinline__ void topk_wave_exact(const float *logits, int E, int K, float *s_e, int &idx_k, float &w_k)
{
    const int lane = lane_id();
    float p[MAXV];
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        p[v] = i < E ? logits[i] : -__builtin_inff();
    }
    topk_wave_vals_exact<MAXV>(p, E, K, s_e, idx_k, w_k);
}

template <int MAXV>
__device__ __forceinline__ void topk_wave(const float *logits, int E, int K, int &idx_k, float &w_k)
{
    const int lane = lane_id();
    float p[MAXV];
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        p[v] = i < E ? logits[i] : -__builtin_inff();
    }
    topk_wave_vals<MAXV>(p, E, K, idx_k, w_k);
}

// Dot of one fp32 router row (H = 256 * NB4) with x: lane holds columns
// 4*lane + 256*m.  Returns the wave-reduced sum in every lane.
__device__ __forceinline__ float router_row_dot(const float *row, const float *x, int H)
{
    const int lane = lane_id();
    float acc = 0.f;
    for (int m = 0; m < H / 256; m++) {
        const float4 wv = *reinterpret_cast<const float4 *>(row + 4 * lane + 256 * m);
        const float4 xv = *reinterpret_cast<const float4 *>(x + 4 * lane + 256 * m);
        acc = fmaf(wv.x, xv.x, acc);
        acc = fmaf(wv.y, xv.y, acc);
        acc = fmaf(wv.z, xv.z, acc);
        acc = fmaf(wv.w, xv.w, acc);
    }
    return wave_sum(acc);
}

// Dot of the fp16 shared-gate vector with x (one_layer.cu:974-980).
__device__ __forceinline__ float shgate_dot(const uint16_t *g, const float *x, int H)
{
    const int lane = lane_id();
    float acc = 0.f;
    for (int m = 0; m < H / 256; m++) {
        const uint2 gv = *reinterpret_cast<const uint2 *>(g + 4 * lane + 256 * m);
        const float4 xv = *reinterpret_cast<const float4 *>(x + 4 * lane + 256 * m);
        acc = fmaf(h2f(gv.x), xv.x, acc);
        acc = fmaf(h2f(gv.x >> 16), xv.y, acc);
        acc = fmaf(h2f(gv.y), xv.z, acc);
        acc = fmaf(h2f(gv.y >> 16), xv.w, acc);
    }
    return wave_sum(acc);
}

__device__ __forceinline__ float silu_mul(float g, float u)
{
    return (g / (1.0f + expf(-g))) * u;  // layer_ops.cu:214-220
}

__device__ __forceinline__ float sigmoidf_ref(float x)
{
    return 1.0f / (1.0f + expf(-x));  // layer_ops.cu:252-255
}
