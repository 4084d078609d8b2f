// route_dev.h — device routing pieces shared by the multi-kernel path and the
// single-launch decode kernel: router row dot and the softmax / top-k wave.
#pragma once

#include "bread_device.h"

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

// Softmax over E logits held as p[v] = logit lane + 64 v, to selection keys.
// Restates cpu_softmax (layer_ops.cu:222-229):
//   - max is taken over numbers; a NaN in entry 0 makes it NaN, as the
//     reference's `x[i] > mx` scan starting from x[0] does;
//   - every exponential and the division use the device expf and IEEE
//     division; the sum is a wave reduction (not sequential), so p can differ
//     from the host's in the last bits.
template <int MAXV>
__device__ __forceinline__ void softmax_keys(float (&p)[MAXV], int E, uint32_t (&key)[MAXV])
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
