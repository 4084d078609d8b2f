// route_dev.h — device routing pieces shared by the multi-kernel path and the
// single-launch decode kernel: router row dot and the softmax / top-k wave.
#pragma once

#include "bread_device.h"

// Totally ordered 32-bit key of a probability: larger key = ranked earlier.
// NaN maps below every number; otherwise the usual sign-magnitude flip.
__device__ __forceinline__ uint32_t prob_key(float p)
{
    if (p != p) return 0u;
    const uint32_t b = __builtin_bit_cast(uint32_t, p);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float prob_from_key(uint32_t k)
{
    if (k == 0u) return __builtin_bit_cast(float, 0x7FC00000u);
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// One wave: softmax over E logits, then K passes of argmax with ties to the
// lower index, then renormalisation by the rank-order sum when positive.
// Restates cpu_softmax / cpu_topk (layer_ops.cu:222-250):
//   - max is taken over numbers; a NaN in entry 0 makes it NaN, as the
//     reference's `x[i] > mx` scan starting from x[0] does;
//   - every exponential and the division use the device expf and IEEE
//     division; the sum is a wave reduction (not sequential), so p can differ
//     from the host's in the last bits;
//   - NaN probabilities rank below every number; the reference's pass that
//     finds nothing above -1e30 is undefined (layer_ops.cu:238-246), here it
//     takes the lowest unused index.
// E <= 64 * MAXV.  Lane k < K returns idx_k / w_k (rank order).
template <int MAXV>
__device__ __forceinline__ void topk_wave_vals(float (&p)[MAXV], int E, int K, int &idx_k, float &w_k)
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
    uint32_t used = 0;
#pragma unroll
    for (int v = 0; v < MAXV; v++) p[v] = p[v] / s;

    int my_idx = 0;
    float my_w = 0.f;
    for (int k = 0; k < K; k++) {
        // candidate = (probability key, ~index): the unsigned max is the
        // largest probability, equal ones going to the lower index; 0 = none
        uint64_t best = 0;
#pragma unroll
        for (int v = 0; v < MAXV; v++) {
            const int i = lane + WAVE * v;
            if (i < E && !((used >> v) & 1u))
                best = u64_max(best, ((uint64_t)prob_key(p[v]) << 32) | (uint32_t)~(uint32_t)i);
        }
        const uint64_t win = wave_max_u64(best);
        const int widx = (int)~(uint32_t)win;
        if ((widx & (WAVE - 1)) == lane) used |= 1u << (widx / WAVE);
        if (lane == k) {
            my_idx = widx;
            my_w = prob_from_key((uint32_t)(win >> 32));
        }
    }
    // rank-order sum, then renormalise (layer_ops.cu:244-249)
    float w_sum = 0.f;
    for (int k = 0; k < K; k++)
        w_sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), k));
    if (w_sum > 0.f) my_w = my_w / w_sum;
    idx_k = my_idx;
    w_k = my_w;
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
