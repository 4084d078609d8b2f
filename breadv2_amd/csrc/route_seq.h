// route_seq.h — router logits in the reference's exact order, for the
// multi-token paths (see route.hip).  route_seq_block is the body of
// k_route_seq; the grouped path runs it in a launch shared with its
// activation preparation.
//
// The reference sums each logit sequentially (one_layer.cu:969-971):
//   logits[e] = ((0 + W[e][0] x[0]) + W[e][1] x[1]) + ... + W[e][H-1] x[H-1],
// every product rounded to fp32 and then added, never fused.  A workgroup
// of 4 waves takes 4 * NE router rows (NE a wave) and 64 tokens (one a lane);
// each lane runs its tokens' NE sums in that order.  Activations and the
// rows' values travel HBM/L2 -> LDS by gfx950 direct-to-LDS loads in chunks
// of 128 columns, double-buffered, so no register holds staged data.  A
// token's chunk row is 32 16-byte units stored XOR-swizzled (unit u at
// u ^ (token % 16)), so a wave's loads write contiguous LDS and the 16-byte
// reads of 16 consecutive lanes (tokens) fall in distinct banks; each weight
// is read as one broadcast value.  The loop's LDS reads run a block of 16
// columns ahead of their use.
#pragma once

#include "bread_device.h"

namespace route_seq {

constexpr int RS_WAVES = 4;              // waves per workgroup
constexpr int RS_TT = WAVE;              // tokens per tile, one a lane
constexpr int RS_CJ = 128;               // columns per staged chunk
constexpr int RS_NB = 4;                 // chunk buffers: loads run RS_NB - 1 chunks ahead
constexpr int RS_BLK = 16;               // columns per block of the pipelined inner loop
constexpr int RS_XI = RS_TT / 2 / RS_WAVES;  // activation loads a wave issues per chunk (8)
constexpr int RS_LOADS = RS_XI + 1;      // + one load of two router rows

static_assert(RS_CJ == 128 && RS_TT % (2 * RS_WAVES) == 0, "a wave instruction stages two 512-byte rows");

struct RsSmem {
    float x[RS_NB][RS_TT][RS_CJ];            // the tile's activations by chunk, units swizzled
    float w[RS_NB][2 * RS_WAVES][RS_CJ];     // the workgroup's router rows by chunk (2 a wave)
    uint16_t g[RS_NB][WAVE * 8];             // the fp16 shared gate's chunk (first 256 bytes)
};

// Direct-to-LDS load (gfx950 global_load_lds_dwordx4): lane i of the wave
// writes its 16 bytes at lds_wave_base + 16 i; the base must be
// wave-uniform.  The data is in LDS once the issuing wave's vmcnt drains.
__device__ __forceinline__ void lds_load16(const void *src, void *lds_wave_base)
{
    __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, 0);
}

// s_waitcnt on the vector memory counter only (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until at most n of this wave's vector memory operations are
// outstanding (n a multiple of the loads per chunk: RS_LOADS, + 1 for the
// wave that also stages the shared gate).
__device__ __forceinline__ void wait_chunks(int ahead, bool gate)
{
    if (gate) {
        if (ahead == 2) wait_vm<2 * (RS_LOADS + 1)>();
        else if (ahead == 1) wait_vm<RS_LOADS + 1>();
        else wait_vm<0>();
    } else {
        if (ahead == 2) wait_vm<2 * RS_LOADS>();
        else if (ahead == 1) wait_vm<RS_LOADS>();
        else wait_vm<0>();
    }
}

// A workgroup barrier without a memory fence: the direct-to-LDS data a
// barrier publishes is waited for explicitly by its issuing wave, so the
// loads running further ahead stay in flight.  The signal fences keep the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void bar()
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Chunk c into buffer b, every wave the same RS_LOADS loads (so the counted
// waits hold): 8 of activation rows, two an instruction (lanes 0-31 row 2i,
// 32-63 row 2i+1; lane l writes unit l % 32 from unit (l % 32) ^ (row % 16)
// of the token's chunk), and one of router rows 2 wv, 2 wv + 1.  Tokens
// beyond T read token T-1 and rows beyond E row E-1 (neither is stored).
// The gate wave (wave 0 of the workgroup holding the shared gate) also
// loads the gate's 256-byte fp16 chunk (lanes 16-63 repeat lanes 0-15).
__device__ __forceinline__ void stage(RsSmem &S, int b, const float *__restrict__ x,
                                      const float *__restrict__ router, const uint16_t *__restrict__ shg, int t0,
                                      int T, int e0, int E, int H, int c, bool gate)
{
    const int lane = lane_id(), wv = wave_id();
    const int half = lane >> 5, u = lane & 31;
#pragma unroll
    for (int i = 0; i < RS_XI; i++) {
        const int row = 2 * (wv + RS_WAVES * i) + half;   // token row of the tile
        const int t = min(t0 + row, T - 1);
        lds_load16(x + (size_t)t * H + c * RS_CJ + 4 * (u ^ (row & 15)), &S.x[b][row - half][0]);
    }
    const int e = min(e0 + 2 * wv + half, E - 1);
    lds_load16(router + (size_t)e * H + c * RS_CJ + 4 * u, &S.w[b][2 * wv][0]);
    if (gate) lds_load16(shg + c * RS_CJ + 8 * (lane & 15), &S.g[b][0]);
}

// Operands of one block of 16 columns from LDS: the lane's activations
// (swizzled units) and the wave's NE rows (broadcast reads; F16: the fp16
// shared gate, widened exactly).
template <int NE, bool F16>
__device__ __forceinline__ void load_block(const float *xrow, int sw, const float (*wrows)[RS_CJ], const uint16_t *g,
                                           int blk, float (&xv)[RS_BLK], float (&wv)[NE][RS_BLK])
{
#pragma unroll
    for (int q = 0; q < RS_BLK / 4; q++) {
        const int unit = blk * (RS_BLK / 4) + q;
        const float4 x4 = *reinterpret_cast<const float4 *>(xrow + 4 * (unit ^ sw));
        xv[4 * q] = x4.x;
        xv[4 * q + 1] = x4.y;
        xv[4 * q + 2] = x4.z;
        xv[4 * q + 3] = x4.w;
#pragma unroll
        for (int n = 0; n < NE; n++) {
            float4 w4;
            if (F16) {
                const uint2 h = *reinterpret_cast<const uint2 *>(g + 4 * unit);
                w4 = make_float4(h2f(h.x), h2f(h.x >> 16), h2f(h.y), h2f(h.y >> 16));
            } else {
                w4 = *reinterpret_cast<const float4 *>(&wrows[n][4 * unit]);
            }
            wv[n][4 * q] = w4.x;
            wv[n][4 * q + 1] = w4.y;
            wv[n][4 * q + 2] = w4.z;
            wv[n][4 * q + 3] = w4.w;
        }
    }
}

// acc[n] += w_n[j] * x[j] for the chunk's 128 columns in order, each product
// rounded before its add.  The adds of a lane are one dependent chain (on
// gfx950 a dependent v_add_f32 waits ~9 cycles for its predecessor, twice
// the issue interval), so the schedule is pinned: the adds of block b
// alternate with the independent products of block b+1, and the LDS reads
// of block b+2 are issued before them.
template <int NE, bool F16>
__device__ __forceinline__ void chunk_dot(const float *xrow, int sw, const float (*wrows)[RS_CJ], const uint16_t *g,
                                          float (&acc)[NE])
{
#pragma clang fp contract(off)
    constexpr int NBK = RS_CJ / RS_BLK;
    float x1[RS_BLK], w1[NE][RS_BLK], x2[RS_BLK], w2[NE][RS_BLK];
    float p[NE][RS_BLK], pn[NE][RS_BLK];
    load_block<NE, F16>(xrow, sw, wrows, g, 0, x1, w1);
#pragma unroll
    for (int j = 0; j < RS_BLK; j++)
#pragma unroll
        for (int n = 0; n < NE; n++) p[n][j] = w1[n][j] * x1[j];
    load_block<NE, F16>(xrow, sw, wrows, g, 1, x1, w1);
#pragma unroll
    for (int blk = 0; blk < NBK; blk++) {
        if (blk + 2 < NBK) load_block<NE, F16>(xrow, sw, wrows, g, blk + 2, x2, w2);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < RS_BLK; j++) {
#pragma unroll
            for (int n = 0; n < NE; n++) acc[n] = acc[n] + p[n][j];
            if (blk + 1 < NBK) {
#pragma unroll
                for (int n = 0; n < NE; n++) pn[n][j] = w1[n][j] * x1[j];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < RS_BLK; j++) {
            x1[j] = x2[j];
#pragma unroll
            for (int n = 0; n < NE; n++) {
                p[n][j] = pn[n][j];
                w1[n][j] = w2[n][j];
            }
        }
    }
}

// Workgroup (bx, by) of a grid (nbx + shg_row, ceil(T / 64)) of 256
// threads, nbx = ceil(E / (4 NE)): router rows 4 NE bx .. + 4 NE - 1 (NE a
// wave) for tokens 64 by .. (one a lane); with shg_row, workgroup bx = nbx
// takes the fp16 shared gate (on wave 0; written to gsh, 0 when shg is NULL).
// H % 128 == 0.
template <int NE>
__device__ __forceinline__ void route_seq_block(RsSmem &S, int bx, int by, const float *__restrict__ router,
                                                const uint16_t *__restrict__ shg, const float *__restrict__ x,
                                                float *__restrict__ logits, float *__restrict__ gsh, int H, int E,
                                                int T, bool shg_row)
{
    static_assert(NE == 1 || NE == 2, "two router rows a wave are staged");
    const int lane = lane_id(), wv = wave_id();
    const int nbx = (E + RS_WAVES * NE - 1) / (RS_WAVES * NE);
    const bool gate_wg = shg_row && bx == nbx;
    const int e0 = gate_wg ? 0 : bx * RS_WAVES * NE;
    const int t0 = by * RS_TT;
    const int nc = H / RS_CJ;
    const bool active = t0 + lane < T;
    const bool gate_wave = gate_wg && wv == 0 && shg;  // stages and sums the gate
    for (int c = 0; c < RS_NB - 1 && c < nc; c++)
        stage(S, c, x, router, shg, t0, T, e0, E, H, c, gate_wave);
    wait_chunks(nc > 2 ? 2 : nc - 1, gate_wave);
    bar();
    float acc[NE];
#pragma unroll
    for (int n = 0; n < NE; n++) acc[n] = 0.f;
    for (int c = 0; c < nc; c++) {
        const int b = c % RS_NB;
        // buffer (c + 3) % 4 was last read in chunk c - 1, before the barrier
        // that ended it
        if (c + RS_NB - 1 < nc)
            stage(S, (c + RS_NB - 1) % RS_NB, x, router, shg, t0, T, e0, E, H, c + RS_NB - 1, gate_wave);
        // lanes past T skip the chunk (their LDS reads would only cost
        // bandwidth), and so do the gate workgroup's other waves
        if (active && (!gate_wg || gate_wave)) {
            if (gate_wave) chunk_dot<NE, true>(S.x[b][lane], lane & 15, nullptr, S.g[b], acc);
            else chunk_dot<NE, false>(S.x[b][lane], lane & 15, &S.w[b][wv * NE], nullptr, acc);
        }
        if (c + 1 < nc) {
            // chunk c + 1 has landed once only the chunks after it are outstanding
            wait_chunks(min(nc - 2 - c, RS_NB - 2), gate_wave);
            bar();
        }
    }
    if (!active) return;
    const int t = t0 + lane;
    if (gate_wg) {
        if (wv == 0) gsh[t] = shg ? acc[0] : 0.f;
        return;
    }
#pragma unroll
    for (int n = 0; n < NE; n++) {
        const int e = e0 + wv * NE + n;
        if (e < E) logits[(size_t)t * E + e] = acc[n];
    }
}

} // namespace route_seq
