// route_seq.h — router logits in the reference's exact order, for the
// multi-token paths (see route.hip).  route_seq_block is the body of
// k_route_seq.
//
// The reference sums each logit sequentially (one_layer.cu:969-971):
//   logits[e] = ((0 + W[e][0] x[0]) + W[e][1] x[1]) + ... + W[e][H-1] x[H-1],
// every product rounded to fp32 and then added, never fused.  A workgroup
// of 4 waves takes 4 * NE router rows (NE a wave) and 64 tokens (one a lane);
// each lane runs its token's NE sums in that order.  A sum is one dependent
// chain, so the kernel's time is a lane's H columns of (product, add) at the
// issue rate of one wave; everything else is kept off that path.
//   - Activations travel HBM/L2 -> LDS by gfx950 direct-to-LDS loads in
//     chunks of 128 columns, RS_NB - 1 chunks in flight.  A token's chunk
//     row is 32 16-byte units stored XOR-swizzled (unit u at u ^ (token %
//     16)), so a wave's loads write contiguous LDS and the 16-byte reads of
//     16 consecutive lanes fall in distinct banks.  Rows past the last token
//     repeat the wave's router chunk (no lane reads them): activation rows
//     that do not exist would otherwise all read one line.
//   - Router rows are the same for every lane: a row's chunk sits in two
//     registers in each 16-lane row of the wave (lane j: columns 4j .. 4j+3
//     of each 64-column half) and each product takes its weight by DPP
//     row_newbcast inside the v_mul, with no LDS traffic and no extra
//     instruction.  The fp16 shared gate travels raw (every wave loads it)
//     and the gate wave widens it when its chunk is used.
//   - With direct-to-LDS loads in the kernel the compiler waits for every
//     LDS read before the first use of any; the block reads are issued
//     right after that wait, a block ahead, so it covers only reads that
//     had a block's time to land.
#pragma once

#include "bread_device.h"

namespace route_seq {

constexpr int RS_WAVES = 4;              // waves per workgroup
constexpr int RS_TT = WAVE;              // tokens per tile, one a lane
constexpr int RS_CJ = 128;               // columns per staged chunk
constexpr int RS_NB = 2;                 // chunk buffers (2 or 4): loads run RS_NB - 1 chunks ahead
constexpr int RS_BLK = 16;               // columns per block of the pipelined inner loop
constexpr int RS_XI = RS_TT / 2 / RS_WAVES;  // activation loads a wave issues per chunk (8)

static_assert(RS_CJ == 128 && RS_TT % (2 * RS_WAVES) == 0, "a wave instruction stages two 512-byte rows");

struct RsSmem {
    float x[RS_NB][RS_TT][RS_CJ];  // the tile's activations by chunk, units swizzled
};

// Native 4-float vectors (HIP's float4 struct is copied through memory).
typedef float rs_f4 __attribute__((ext_vector_type(4)));

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

// Keeps the vector memory operations issued before it ahead of those issued
// after it.  The partial vmcnt waits of rs_run count on that order (gfx9
// completes a wave's vector memory operations in issue order), and nothing
// else pins it: the weight and gate loads read __restrict__ read-only
// arguments, so the optimiser could hoist them above the direct-to-LDS
// batch, and a wait meant for the batch would then leave part of it in
// flight across the barrier.  The empty asm with a memory clobber stops the
// optimiser, the scheduling barrier the machine scheduler.
__device__ __forceinline__ void issue_order()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
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

// Chunk c into buffer b: RS_XI direct-to-LDS loads a wave, two activation
// rows an instruction (lanes 0-31 row 2i, 32-63 row 2i+1; lane l writes unit
// l % 32 from unit (l % 32) ^ (row % 16) of the token's chunk).  Rows past
// T load the same units of fb instead.
__device__ __forceinline__ void rs_stage(RsSmem &S, int b, const float *__restrict__ x, const float *fb, int t0,
                                         int T, int H, int c, int wv, int lane)
{
    const int half = lane >> 5, u = lane & 31;
#pragma unroll
    for (int i = 0; i < RS_XI; i++) {
        const int row = 2 * (wv + RS_WAVES * i) + half;
        const float *base = t0 + row < T ? x + (size_t)(t0 + row) * H : fb;
        lds_load16(base + c * RS_CJ + 4 * (u ^ (row & 15)), &S.x[b][row - half][0]);
    }
}

// The weights of chunk c for the wave's NE rows (w0 and the rows after it)
// and the raw fp16 gate's (four halves a lane; g is a valid stand-in when
// the wave has no gate).  Both are loaded by every wave: a choice between
// loads would make the compiler wait for them where it merges the two.
template <int NE>
__device__ __forceinline__ void rs_load_w(rs_f4 (&w)[NE][2], uint2 (&gw)[2], const float *w0,
                                          const uint16_t *__restrict__ g, int H, int c, int lane)
{
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int col = c * RS_CJ + 64 * h + 4 * (lane & 15);
        gw[h] = *reinterpret_cast<const uint2 *>(g + col);
#pragma unroll
        for (int n = 0; n < NE; n++) w[n][h] = *reinterpret_cast<const rs_f4 *>(w0 + (size_t)n * H + col);
    }
}

// The weights chunk_dot reads: the rows', or for the gate wave the gate's
// widened in place of row 0.
template <int NE>
__device__ __forceinline__ void rs_take(rs_f4 (&wc)[NE][2], const rs_f4 (&w)[NE][2], const uint2 (&gw)[2], bool gate)
{
#pragma unroll
    for (int n = 0; n < NE; n++) {
        wc[n][0] = w[n][0];
        wc[n][1] = w[n][1];
    }
    if (gate) {
#pragma unroll
        for (int h = 0; h < 2; h++)
            wc[0][h] = rs_f4{h2f(gw[h].x), h2f(gw[h].x >> 16), h2f(gw[h].y), h2f(gw[h].y >> 16)};
    }
}

// Lane n of each 16-lane row of v, to the whole row (DPP row_newbcast; the
// compiler folds it into the consuming v_mul).
template <int N>
__device__ __forceinline__ float row_bcast(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + N, 0xF,
                                                                 0xF, false));
}

__device__ __forceinline__ float row_bcast(float v, int n)
{
    switch (n) {
    case 0: return row_bcast<0>(v);
    case 1: return row_bcast<1>(v);
    case 2: return row_bcast<2>(v);
    case 3: return row_bcast<3>(v);
    case 4: return row_bcast<4>(v);
    case 5: return row_bcast<5>(v);
    case 6: return row_bcast<6>(v);
    case 7: return row_bcast<7>(v);
    case 8: return row_bcast<8>(v);
    case 9: return row_bcast<9>(v);
    case 10: return row_bcast<10>(v);
    case 11: return row_bcast<11>(v);
    case 12: return row_bcast<12>(v);
    case 13: return row_bcast<13>(v);
    case 14: return row_bcast<14>(v);
    default: return row_bcast<15>(v);
    }
}

// Router weight of chunk column col (0..127).
__device__ __forceinline__ float rs_weight(const rs_f4 (&w)[2], int col)
{
    return row_bcast(w[col >> 6][col & 3], (col & 63) >> 2);
}

// The lane's activations of one 16-column block from its swizzled LDS row.
__device__ __forceinline__ void rs_load_x(const float *xrow, int sw, int blk, float (&xv)[RS_BLK])
{
#pragma unroll
    for (int q = 0; q < RS_BLK / 4; q++) {
        const rs_f4 x4 = *reinterpret_cast<const rs_f4 *>(xrow + 4 * ((blk * (RS_BLK / 4) + q) ^ sw));
        xv[4 * q] = x4[0];
        xv[4 * q + 1] = x4[1];
        xv[4 * q + 2] = x4[2];
        xv[4 * q + 3] = x4[3];
    }
}

// acc[n] += w_n[j] * x[j] for the chunk's 128 columns in order, each product
// rounded before its add.  The adds of a lane are one dependent chain, so
// the schedule is pinned: the adds of block b alternate with the
// independent products of block b+1, and the LDS reads of block b+2 go out
// right after the first of those products (the compiler's wait for all LDS
// reads sits before it).  Every lane of the wave runs it: the weights come
// from other lanes by DPP.
template <int NE>
__device__ __forceinline__ void chunk_dot(const float *xrow, int sw, const rs_f4 (&w)[NE][2], float (&acc)[NE])
{
#pragma clang fp contract(off)
    constexpr int NBK = RS_CJ / RS_BLK;
    float x1[RS_BLK], x2[RS_BLK];
    float p[NE][RS_BLK], pn[NE][RS_BLK];
    rs_load_x(xrow, sw, 0, x1);
#pragma unroll
    for (int j = 0; j < RS_BLK; j++)
#pragma unroll
        for (int n = 0; n < NE; n++) p[n][j] = rs_weight(w[n], j) * x1[j];
    rs_load_x(xrow, sw, 1, x1);
#pragma unroll
    for (int blk = 0; blk < NBK; blk++) {
#pragma unroll
        for (int j = 0; j < RS_BLK; j++) {
#pragma unroll
            for (int n = 0; n < NE; n++) acc[n] = acc[n] + p[n][j];
            if (blk + 1 < NBK) {
#pragma unroll
                for (int n = 0; n < NE; n++) pn[n][j] = rs_weight(w[n], (blk + 1) * RS_BLK + j) * x1[j];
            }
            if (j == 0 && blk + 2 < NBK) {
                __builtin_amdgcn_sched_barrier(0);
                rs_load_x(xrow, sw, blk + 2, x2);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < RS_BLK; j++) {
            x1[j] = x2[j];
#pragma unroll
            for (int n = 0; n < NE; n++) p[n][j] = pn[n][j];
        }
    }
}

// The chunk loop of one wave (work: the wave sums at all; gate: it sums the
// gate; every wave stages and passes the same barriers).  Per chunk c: take
// the weights loaded during chunk c - 1, issue the direct-to-LDS batch of
// chunk c + RS_NB - 1 and the weights of chunk c + 1, sum chunk c, then wait
// for batch c + 1 and pass a barrier.  Waiting for batch c + 1 leaves in
// flight what was issued after it: with four buffers the weights of chunks
// c - 1 .. c + 1 (2 NE + 2 loads each) and batches c + 2 and c + 3 (RS_XI
// each); with two, the weights of chunk c + 1.
template <int NE>
__device__ __forceinline__ void rs_run(RsSmem &S, const float *__restrict__ x, const float *w0,
                                       const uint16_t *__restrict__ g, int t0, int T, int H, bool work, bool gate,
                                       float (&acc)[NE])
{
    const int lane = lane_id(), wv = wave_id();
    const int nc = H / RS_CJ;
    constexpr int AFTER = 2 * RS_XI + 3 * (2 * NE + 2);
    static_assert(RS_NB != 4 || AFTER < 64, "vmcnt range");
    rs_f4 wn[NE][2], wc[NE][2];
    uint2 gn[2];
    for (int c = 0; c < RS_NB - 1 && c < nc; c++) rs_stage(S, c, x, w0, t0, T, H, c, wv, lane);
    issue_order();
    rs_load_w<NE>(wn, gn, w0, g, H, 0, lane);
    wait_vm<0>();
    bar();
    for (int c = 0; c < nc; c++) {
        rs_take<NE>(wc, wn, gn, gate);
        // buffer (c + RS_NB - 1) % RS_NB was last read in chunk c - 1,
        // before the barrier that ended it
        if (c + RS_NB - 1 < nc)
            rs_stage(S, (c + RS_NB - 1) % RS_NB, x, w0, t0, T, H, c + RS_NB - 1, wv, lane);
        issue_order();
        if (c + 1 < nc) rs_load_w<NE>(wn, gn, w0, g, H, c + 1, lane);
        issue_order();
        if (work) chunk_dot<NE>(S.x[c % RS_NB][lane], lane & 15, wc, acc);
        if (c + 1 < nc) {
            if constexpr (RS_NB == 4) {
                if (c + 3 < nc) wait_vm<AFTER>();
                else wait_vm<0>();
            } else {
                static_assert(RS_NB == 2, "chunk buffers");
                wait_vm<2 * NE + 2>();  // chunk c + 1's weights were issued after its batch
            }
            bar();
        }
    }
}

// Workgroup (bx, by) of a grid (nbx + shg_row, ceil(T / 64)) of 256
// threads, nbx = ceil(E / (4 NE)): router rows 4 NE bx .. + 4 NE - 1 (NE a
// wave) for tokens 64 by .. (one a lane); with shg_row, workgroup bx = nbx
// takes the fp16 shared gate (on wave 0; written to gsh, 0 when shg is NULL).
// H % 128 == 0 and E >= NE.
template <int NE>
__device__ __forceinline__ void route_seq_block(RsSmem &S, int bx, int by, const float *__restrict__ router,
                                                const uint16_t *__restrict__ shg, const float *__restrict__ x,
                                                float *__restrict__ logits, float *__restrict__ gsh, int H, int E,
                                                int T, bool shg_row)
{
    static_assert(NE == 1 || NE == 2, "weight registers");
    const int lane = lane_id(), wv = wave_id();
    const int nbx = (E + RS_WAVES * NE - 1) / (RS_WAVES * NE);
    const bool gate_wg = shg_row && bx == nbx;
    const bool gate_wave = gate_wg && wv == 0 && shg;  // sums the gate
    const int t0 = by * RS_TT;
    // the wave stands for rows eb .. eb + NE - 1 and sums the NE consecutive
    // rows from e0 (moved back from eb so that every row read exists; rows
    // past E are not stored); the gate workgroup's waves read row 0
    const int eb = bx * RS_WAVES * NE + wv * NE;
    const int e0 = gate_wg ? 0 : min(eb, E - NE);
    const float *w0 = router + (size_t)e0 * H;
    float acc[NE];
#pragma unroll
    for (int n = 0; n < NE; n++) acc[n] = 0.f;
    const uint16_t *g = shg ? shg : reinterpret_cast<const uint16_t *>(w0);
    rs_run<NE>(S, x, w0, g, t0, T, H, !gate_wg || gate_wave, gate_wave, acc);
    const int t = t0 + lane;
    if (t >= T) return;
    if (gate_wg) {
        if (wv == 0) gsh[t] = shg ? acc[0] : 0.f;
        return;
    }
#pragma unroll
    for (int n = 0; n < NE; n++) {
        const int e = e0 + n;
        if (e >= eb && e < E) logits[(size_t)t * E + e] = acc[n];
    }
}

} // namespace route_seq
