// moe_small.hip — the small-batch MoE path (2 <= n_tokens <= 32; the
// automatic choice uses it up to 8: batched decode, speculative-verify
// rounds).
//
// Per token the result is the MoE block of one_layer_forward
// (one_layer.cu:1800-1986; CPU form 1413-1471), computed in fp32 like the
// per-token path.  At these batch sizes an expert is chosen by a handful of
// tokens, so matrix-core tiles would run mostly empty and the time goes to
// latency: this path streams each selected expert's rows once over the whole
// GPU and dots every row with the few tokens that chose the expert, on the
// vector ALUs.
//
// Kernels per layer, stream-ordered:
//   k_sb_router   one router row a wave held in registers, dotted with every
//                 token (the next token's activations requested while the
//                 current one is summed); the extra row E is the fp16
//                 shared-gate vector.
//   k_sb_select   one workgroup: softmax / top-k per token, then slots: an
//                 expert's tokens in chunks of at most SB_CH (the shared
//                 expert's chunks first, with every token, then the chosen
//                 experts in expert order), each with its (token, rank) pairs
//                 in token order.  Chunks spread a hot expert over more
//                 workgroups.
//   k_sb_gateup   grid (slot, 32-row chunk): 8 lanes per gate/up row pair,
//                 one Q4_K superblock a lane, dotted with the slot's tokens
//                 (staged in LDS), then SwiGLU.
//   k_sb_down     grid (slot, 128-row chunk): the rows staged in LDS by
//                 16-byte loads, 16 lanes per row (8 per Q6_K superblock),
//                 dotted with the slot's SwiGLU rows (staged in LDS).
//   k_sb_combine  per token, the reference order: shared expert first, then
//                 the routed experts by rank.
// Pair p = t * (K + 1) + k' (k' = 0 shared, 1 + rank) indexes the SwiGLU rows
// and the expert outputs, so the combine does not depend on the slot order.
// In each workgroup the pair ids are loaded first, then the activations,
// then the weights: a wait for a load also waits for every load issued
// before it.  Every sum has a fixed order: repeated calls are bit-identical.
#include "bread_internal.h"
#include "quant_dot.h"
#include "route_dev.h"

namespace {

constexpr int SB_MAX_T = 32;      // tokens per call (token bitmasks are 32 bits)
constexpr int SB_AUTO_T = 8;      // the automatic choice takes this path up to here (measured crossover)
constexpr int RT_WAVES = 16;      // selection waves
constexpr int RT_THREADS = RT_WAVES * WAVE;
constexpr int SB_CH = 4;          // pairs per slot: an expert's tokens in chunks of this many
constexpr int GU_RG = 32;         // gate/up rows per workgroup (8 a wave)
constexpr int DN_IT = 8;          // down: row groups per wave (4 rows each with 16 lanes a row)
constexpr int DN_RG = 128;        // down rows per workgroup
constexpr int DN_W16 = (DN_RG * 2 * 210 / 16 + 255) / 256;  // 16-byte pieces a thread stages
constexpr int MAX_H = 2048;
constexpr int MAX_I = 512;
constexpr int MAX_E = 1024;
constexpr int MAX_K = 16;

struct SbLayer {
    const uint8_t *gate_exps, *up_exps, *down_exps;
    const uint8_t *gate_sh, *up_sh, *down_sh;
    uint64_t gate_eb, up_eb, down_eb;
};

// Marks a register as changed here, so code that depends on it stays at its
// use: keeps the compiler from hoisting the code conversions out of the token
// loops, which would hold every converted weight in registers at once.
__device__ __forceinline__ void pin(uint32_t &v)
{
    asm volatile("" : "+v"(v));
}

struct SbSlots {
    const int32_t *expert;  // [S]: expert id, -1 for the shared expert's slots
    const int32_t *cnt;     // [S]: pairs in the slot (<= SB_CH)
    const int32_t *pair;    // [S][SB_CH]: pair ids in token order
    const int32_t *n;       // slots in use
};

// ---- routing ---------------------------------------------------------------------

__device__ __forceinline__ void load_row4(const float *p, int lane, int nm, float4 (&v)[MAX_H / 256])
{
#pragma unroll
    for (int m = 0; m < MAX_H / 256; m++)
        v[m] = m < nm ? *reinterpret_cast<const float4 *>(p + 4 * lane + 256 * m) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// Softmax / top-k per token (the routing waves of the other paths), then the
// experts chosen by any token numbered into slots in expert order (slot 0 is
// the shared expert with every token), each slot with its (token, rank)
// pairs in token order, from per-expert token bitmasks.  One workgroup of
// 1024 threads.
template <int MAXV>
__device__ void sb_select(const float *__restrict__ logits, int E, int K, int T, int32_t *__restrict__ idx,
                          float *__restrict__ w, int32_t *__restrict__ slot_expert, int32_t *__restrict__ slot_cnt,
                          int32_t *__restrict__ slot_pair, int32_t *__restrict__ n_slots)
{
    __shared__ int sidx[SB_MAX_T * MAX_K];
    __shared__ uint32_t mask[MAX_E];  // tokens that chose expert e
    __shared__ int slot_of[MAX_E];
    __shared__ int wave_tot[RT_WAVES];
    const int tid = (int)threadIdx.x, wv = tid / WAVE, lane = lane_id();
    for (int e = tid; e < E; e += RT_THREADS) mask[e] = 0u;
    for (int t = wv; t < T; t += RT_WAVES) {
        int ik;
        float wk;
        topk_wave<MAXV>(logits + (size_t)t * E, E, K, ik, wk);
        if (lane < K) {
            idx[(size_t)t * K + lane] = ik;
            w[(size_t)t * K + lane] = wk;
            sidx[t * K + lane] = ik;
        }
    }
    __syncthreads();
    const int P = T * K;
    for (int i = tid; i < P; i += RT_THREADS) {
        const int e = sidx[i];
        if (e >= 0 && e < E) atomicOr(&mask[e], 1u << (i / K));
    }
    __syncthreads();
    // slots: the shared expert's tokens in chunks of SB_CH (slots 0 .. nsh-1),
    // then every chosen expert's tokens in chunks of SB_CH, in expert order
    // (E <= blockDim); chunks spread a hot expert's tokens over more workgroups
    const int nsh = (T + SB_CH - 1) / SB_CH;
    const int ncnt = tid < E ? __popc(mask[tid]) : 0;
    const int nch = (ncnt + SB_CH - 1) / SB_CH;
    int incl = nch;  // inclusive scan of the chunk counts over the experts
    for (int off = 1; off < WAVE; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
    }
    if (lane == WAVE - 1) wave_tot[wv] = incl;
    __syncthreads();
    int before = 0;
    for (int v = 0; v < wv; v++) before += wave_tot[v];
    const int first = nsh + before + incl - nch;
    if (tid < E) slot_of[tid] = first;
    for (int k = 0; k < nch; k++) {
        slot_expert[first + k] = tid;
        slot_cnt[first + k] = ncnt - k * SB_CH < SB_CH ? ncnt - k * SB_CH : SB_CH;
    }
    for (int k = tid; k < nsh; k += RT_THREADS) {
        slot_expert[k] = -1;
        slot_cnt[k] = T - k * SB_CH < SB_CH ? T - k * SB_CH : SB_CH;
    }
    if (tid == 0) {
        int tot = 0;
        for (int v = 0; v < RT_WAVES; v++) tot += wave_tot[v];
        *n_slots = nsh + tot;
    }
    __syncthreads();
    // pair (t, k) sits at the rank of token t among the expert's tokens
    for (int i = tid; i < P; i += RT_THREADS) {
        const int e = sidx[i];
        if (e < 0 || e >= E) continue;
        const int t = i / K, k = i - t * K;
        const int pos = __popc(mask[e] & ((1u << t) - 1u));
        slot_pair[(size_t)(slot_of[e] + pos / SB_CH) * SB_CH + pos % SB_CH] = t * (K + 1) + 1 + k;
    }
    for (int t = tid; t < T; t += RT_THREADS) slot_pair[t] = t * (K + 1);  // slot t / SB_CH, place t % SB_CH
}

// Router rows: one a wave held in registers, dotted with every token (the
// next token's activations requested while the current one is summed); the
// extra row E is the fp16 shared-gate vector.
__global__ __launch_bounds__(256) void k_sb_router(const float *__restrict__ router, const uint16_t *__restrict__ shg,
                                                   const float *__restrict__ x, float *__restrict__ logits,
                                                   float *__restrict__ gsh, int H, int E, int T)
{
    const int wv = (int)threadIdx.x / WAVE, lane = lane_id();
    const int e = (int)blockIdx.x * 4 + wv;
    if (e > E) return;
    const int nm = H / 256;
    // this wave's row: lane holds columns 4 lane + 256 m (router_row_dot's order)
    float4 r[MAX_H / 256];
    if (e < E) {
        load_row4(router + (size_t)e * H, lane, nm, r);
    } else {
#pragma unroll
        for (int m = 0; m < MAX_H / 256; m++) {
            r[m] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < nm && shg) {
                const uint2 g = *reinterpret_cast<const uint2 *>(shg + 4 * lane + 256 * m);
                r[m] = make_float4(h2f(g.x), h2f(g.x >> 16), h2f(g.y), h2f(g.y >> 16));
            }
        }
    }
    float4 xc[MAX_H / 256], xn[MAX_H / 256];
    load_row4(x, lane, nm, xc);
    for (int t = 0; t < T; t++) {
        if (t + 1 < T) load_row4(x + (size_t)(t + 1) * H, lane, nm, xn);
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < MAX_H / 256; m++) {
            acc = fmaf(r[m].x, xc[m].x, acc);
            acc = fmaf(r[m].y, xc[m].y, acc);
            acc = fmaf(r[m].z, xc[m].z, acc);
            acc = fmaf(r[m].w, xc[m].w, acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            if (e < E) logits[(size_t)t * E + e] = acc;
            else gsh[t] = shg ? acc : 0.f;
        }
#pragma unroll
        for (int m = 0; m < MAX_H / 256; m++) xc[m] = xn[m];
    }
}

template <int MAXV>
__global__ __launch_bounds__(RT_THREADS) void k_sb_select(const float *__restrict__ logits, int E, int K, int T,
                                                          int32_t *__restrict__ idx, float *__restrict__ w,
                                                          int32_t *__restrict__ slot_expert,
                                                          int32_t *__restrict__ slot_cnt,
                                                          int32_t *__restrict__ slot_pair,
                                                          int32_t *__restrict__ n_slots)
{
    sb_select<MAXV>(logits, E, K, T, idx, w, slot_expert, slot_cnt, slot_pair, n_slots);
}

// ---- gate / up + SwiGLU ---------------------------------------------------------

// Lane layout: 8 lanes per row, 8 rows a wave; lane b of a row reads the
// whole superblock b (nb = H / 256 <= 8; lanes b >= nb hold zeros): header
// (d, dmin, 12 scale bytes) and the 128-byte qs.  Chunk c = 2 j + hh of qs
// holds elements 64 j + 16 hh + [0, 16) (low nibbles, sub-block 2j) and + 32
// (high nibbles, sub-block 2j + 1) (dequant_q4k_cpu.c:111-121).  Codes are
// converted as they are used; each sub-block's sum(q x) is then scaled once,
// d sc sum(q x) - dmin m sum(x) (q4k_chunk_dot_sx's factored form), with the
// 32-element activation sums computed once per token while staging.
struct Q4Sb {
    float dsc[8], dm[8];  // d sc_s and dmin m_s of the 8 sub-blocks
};

__device__ __forceinline__ void q4_sb_scales(uint4 hd, Q4Sb &o)
{
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
#pragma unroll
    for (int sb = 0; sb < 8; sb++) {
        uint32_t sc, mn;
        scale_min_k4((uint32_t)sb, hd.y, hd.z, hd.w, sc, mn);
        o.dsc[sb] = d * (float)sc;
        o.dm[sb] = dmin * (float)mn;
    }
}

// Activation rows staged in LDS with 4 floats of padding after every 256: the
// 8 superblock lanes of a row read 16-byte runs 256 floats apart, which the
// padding spreads over all 32 banks (the 8 rows of a wave read the same ones).
constexpr int XPAD_ROW = MAX_H + 4 * (MAX_H / 256);

__device__ __forceinline__ int xpad(int i)
{
    return i + 4 * (i >> 8);
}

__global__ __launch_bounds__(256) void k_sb_gateup(SbLayer L, const float *__restrict__ x, SbSlots S,
                                                   float *__restrict__ h, int H, int I, int Ish, int E, int K, int T,
                                                   int Imax)
{
    __shared__ float xs[SB_CH][XPAD_ROW];
    __shared__ float xsum[SB_CH][MAX_H / 32];  // sums of the 32-element sub-blocks
    __shared__ int tok[SB_CH];
    const int s = (int)blockIdx.x;
    const int wv = (int)threadIdx.x / WAVE, lane = lane_id();
    // slot metadata requested together
    const int ns = *S.n, e = S.expert[s], cnt_s = S.cnt[s];
    // the selection writes consistent slots; the checks keep every access in
    // bounds whatever the metadata holds
    if (s >= ns || e < -1 || e >= E) return;
    const int cnt = cnt_s < SB_CH ? (cnt_s > 0 ? cnt_s : 0) : SB_CH;
    const int Is = e < 0 ? Ish : I;
    const int r0 = (int)blockIdx.y * GU_RG;
    if (r0 >= Is) return;
    const int P = T * (K + 1);
    // pair ids first: the in-order wait for them must not include the weights
    if (threadIdx.x < (unsigned)cnt) {
        const int pr = S.pair[(size_t)s * SB_CH + threadIdx.x];
        tok[threadIdx.x] = pr >= 0 && pr < P ? pr : -1;
    }
    __syncthreads();
    // then the activations: thread i takes 32-element sub-block i % 64 of token
    // i / 64 (columns beyond H read as zeros) ...
    const int st_t = (int)threadIdx.x / (MAX_H / 32), st_sb = (int)threadIdx.x % (MAX_H / 32);
    const int st_pr = st_t < cnt ? tok[st_t] : -1;
    float4 xv[8];
#pragma unroll
    for (int m = 0; m < 8; m++)
        xv[m] = (st_pr >= 0 && 32 * st_sb < H)
                    ? reinterpret_cast<const float4 *>(x + (size_t)(st_pr / (K + 1)) * H + 32 * st_sb)[m]
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    // ... and last the weights: the lane's superblock of its gate and up rows
    const int b = lane & 7;
    const int r = r0 + wv * 8 + (lane >> 3);  // this lane's row
    const int nb = H / QK;
    const uint64_t rb = (uint64_t)nb * Q4K_BYTES;
    const uint8_t *gb = e < 0 ? L.gate_sh : L.gate_exps + (uint64_t)e * L.gate_eb;
    const uint8_t *ub = e < 0 ? L.up_sh : L.up_exps + (uint64_t)e * L.up_eb;
    const bool act = b < nb && r < Is;
    uint4 gh = make_uint4(0u, 0u, 0u, 0u), uh = gh;
    uint4 gq[8], uq[8];
#pragma unroll
    for (int m = 0; m < 8; m++) gq[m] = uq[m] = make_uint4(0u, 0u, 0u, 0u);
    if (act) {
        const uint8_t *g = gb + (uint64_t)r * rb + (uint64_t)b * Q4K_BYTES;
        const uint8_t *u = ub + (uint64_t)r * rb + (uint64_t)b * Q4K_BYTES;
        gh = ld_b128(g);
        uh = ld_b128(u);
#pragma unroll
        for (int m = 0; m < 8; m++) {
            gq[m] = ld_b128(g + 16 + 16 * m);
            uq[m] = ld_b128(u + 16 + 16 * m);
        }
    }
    if (st_t < cnt) {
        float sm = 0.f;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            *reinterpret_cast<float4 *>(&xs[st_t][xpad(32 * st_sb + 4 * m)]) = xv[m];
            sm += xv[m].x;
            sm += xv[m].y;
            sm += xv[m].z;
            sm += xv[m].w;
        }
        xsum[st_t][st_sb] = sm;
    }
    Q4Sb gs, us;  // scales once per row (the headers die here)
    q4_sb_scales(gh, gs);
    q4_sb_scales(uh, us);
    __syncthreads();
    for (int t = 0; t < cnt; t++) {
        float ag[8], au[8];  // sum(q x) per sub-block
#pragma unroll
        for (int sb = 0; sb < 8; sb++) ag[sb] = au[sb] = 0.f;
#pragma unroll
        for (int cc = 0; cc < 8; cc++) {
            const int jj = cc >> 1, hh = cc & 1;
            const int c0 = QK * b + 64 * jj + 16 * hh;
            uint32_t gw[4] = {gq[cc].x, gq[cc].y, gq[cc].z, gq[cc].w};
            uint32_t uw[4] = {uq[cc].x, uq[cc].y, uq[cc].z, uq[cc].w};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                pin(gw[m]);  // converted here for each token, not hoisted out of the loop
                pin(uw[m]);
            }
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const float4 xl = *reinterpret_cast<const float4 *>(&xs[t][xpad(c0 + 4 * m)]);
                const float4 xh = *reinterpret_cast<const float4 *>(&xs[t][xpad(c0 + 32 + 4 * m)]);
                const uint32_t glo = gw[m] & 0x0F0F0F0Fu, ghi = (gw[m] >> 4) & 0x0F0F0F0Fu;
                const uint32_t ulo = uw[m] & 0x0F0F0F0Fu, uhi = (uw[m] >> 4) & 0x0F0F0F0Fu;
                ag[2 * jj] = fmaf((float)byte_of(glo, 0), xl.x, ag[2 * jj]);
                ag[2 * jj] = fmaf((float)byte_of(glo, 1), xl.y, ag[2 * jj]);
                ag[2 * jj] = fmaf((float)byte_of(glo, 2), xl.z, ag[2 * jj]);
                ag[2 * jj] = fmaf((float)byte_of(glo, 3), xl.w, ag[2 * jj]);
                ag[2 * jj + 1] = fmaf((float)byte_of(ghi, 0), xh.x, ag[2 * jj + 1]);
                ag[2 * jj + 1] = fmaf((float)byte_of(ghi, 1), xh.y, ag[2 * jj + 1]);
                ag[2 * jj + 1] = fmaf((float)byte_of(ghi, 2), xh.z, ag[2 * jj + 1]);
                ag[2 * jj + 1] = fmaf((float)byte_of(ghi, 3), xh.w, ag[2 * jj + 1]);
                au[2 * jj] = fmaf((float)byte_of(ulo, 0), xl.x, au[2 * jj]);
                au[2 * jj] = fmaf((float)byte_of(ulo, 1), xl.y, au[2 * jj]);
                au[2 * jj] = fmaf((float)byte_of(ulo, 2), xl.z, au[2 * jj]);
                au[2 * jj] = fmaf((float)byte_of(ulo, 3), xl.w, au[2 * jj]);
                au[2 * jj + 1] = fmaf((float)byte_of(uhi, 0), xh.x, au[2 * jj + 1]);
                au[2 * jj + 1] = fmaf((float)byte_of(uhi, 1), xh.y, au[2 * jj + 1]);
                au[2 * jj + 1] = fmaf((float)byte_of(uhi, 2), xh.z, au[2 * jj + 1]);
                au[2 * jj + 1] = fmaf((float)byte_of(uhi, 3), xh.w, au[2 * jj + 1]);
            }
            // one chunk's activations at a time: keeps the scheduler from
            // hoisting every chunk's LDS reads (and their registers) ahead
            __builtin_amdgcn_sched_barrier(0);
        }
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int sb = 0; sb < 8; sb++) {
            const float xsb = xsum[t][8 * b + sb];
            pg = fmaf(gs.dsc[sb], ag[sb], pg);
            pg = fmaf(-gs.dm[sb], xsb, pg);
            pu = fmaf(us.dsc[sb], au[sb], pu);
            pu = fmaf(-us.dm[sb], xsb, pu);
        }
        pg = sum8(pg);
        pu = sum8(pu);
        const int pr = tok[t];
        if (b == 0 && r < Is && pr >= 0) h[(size_t)pr * Imax + r] = silu_mul(pg, pu);
    }
}

// ---- down ----------------------------------------------------------------------

// Lane layout of a Q6_K row of I = 256 nbi (nbi <= 2) columns: a row takes
// LR = 8 nbi adjacent lanes, lane q = 8 b + u of them reads superblock b's
// unit u (quant_dot.h: half n = u / 4, l in [8 tt, 8 tt + 8), tt = u % 4,
// elements 128 n + 32 s + l, s < 4); a wave holds 64 / LR rows at a time and
// DN_IT such groups.  A group's codes are converted to floats once; each
// pair's dot is q6k_unit_dot_sx's factored form, d sum_s sc_s (sum(q x) -
// 32 sum(x)), with the 8-element sums computed once per pair while staging.
__device__ __forceinline__ void q6_codes(uint2 ql0, uint2 ql1, uint2 qh, float (&qf)[4][8])
{
#pragma unroll
    for (int w = 0; w < 2; w++) {
        uint32_t q[4];
        q6k_unpack(w ? ql0.y : ql0.x, w ? ql1.y : ql1.x, w ? qh.y : qh.x, q);
#pragma unroll
        for (int ss = 0; ss < 4; ss++)
#pragma unroll
            for (int k = 0; k < 4; k++) qf[ss][4 * w + k] = (float)byte_of(q[ss], k);
    }
}

// SwiGLU rows staged in LDS with 4 floats of padding after every 128: the 8
// lanes of a superblock read 16-byte runs at 128 n + 8 tt (+ 4), which the
// padding spreads over all 32 banks.
constexpr int HPAD_ROW = MAX_I + 4 * (MAX_I / 128);

__device__ __forceinline__ int hpad(int i)
{
    return i + 4 * (i >> 7);
}

__global__ __launch_bounds__(256) void k_sb_down(SbLayer L, const float *__restrict__ h, SbSlots S,
                                                 float *__restrict__ eo, int H, int I, int Ish, int E, int K, int T,
                                                 int Imax)
{
    __shared__ float hs[SB_CH][HPAD_ROW];
    __shared__ float4 hsum[SB_CH][16];  // per unit (b, n, tt): the sums of its 4 runs of 8
    __shared__ int prs[SB_CH];
    __shared__ uint32_t wsm[DN_RG * 2 * Q6K_BYTES / 4];  // the workgroup's down rows
    const int s = (int)blockIdx.x;
    const int wv = (int)threadIdx.x / WAVE, lane = lane_id();
    const int ns = *S.n, e = S.expert[s], cnt_s = S.cnt[s];
    if (s >= ns || e < -1 || e >= E) return;
    const int cnt = cnt_s < SB_CH ? (cnt_s > 0 ? cnt_s : 0) : SB_CH;
    const int Is = e < 0 ? Ish : I;
    const int nbi = Is / QK;
    const int LR = 8 * nbi, RW = WAVE / LR;
    const int j0 = (int)blockIdx.y * DN_RG + wv * (DN_RG / 4);  // this wave's first row
    const int P = T * (K + 1);
    // pair ids first, then the SwiGLU rows, then the weights (in-order waits)
    if (threadIdx.x < (unsigned)cnt) {
        const int pr = S.pair[(size_t)s * SB_CH + threadIdx.x];
        prs[threadIdx.x] = pr >= 0 && pr < P ? pr : -1;
    }
    __syncthreads();
    // thread i takes 8-element run i % 64 of pair i / 64 (Is / 8 <= 64 runs)
    const int st_p = (int)threadIdx.x / (MAX_I / 8), st_r = (int)threadIdx.x % (MAX_I / 8);
    const int st_pr = st_p < cnt && st_r < Is / 8 ? prs[st_p] : -1;
    float4 hv0 = make_float4(0.f, 0.f, 0.f, 0.f), hv1 = hv0;
    if (st_pr >= 0) {
        hv0 = reinterpret_cast<const float4 *>(h + (size_t)st_pr * Imax + 8 * st_r)[0];
        hv1 = reinterpret_cast<const float4 *>(h + (size_t)st_pr * Imax + 8 * st_r)[1];
    }
    const uint64_t rbd = (uint64_t)nbi * Q6K_BYTES;
    const uint8_t *db = e < 0 ? L.down_sh : L.down_exps + (uint64_t)e * L.down_eb;
    // the workgroup's rows, staged whole with 16-byte loads (Q6_K rows are
    // only 4-byte aligned, so lanes read their pieces from LDS); the region
    // starts 16-byte aligned: the tensor and expert stride are, and DN_RG rows
    // of 210 nbi bytes are a multiple of 16
    const int rows = H - (int)blockIdx.y * DN_RG < DN_RG ? H - (int)blockIdx.y * DN_RG : DN_RG;
    const int n16 = (int)((uint64_t)rows * rbd / 16);
    const uint4 *src = reinterpret_cast<const uint4 *>(db + (uint64_t)blockIdx.y * DN_RG * rbd);
    uint4 wv4[DN_W16];
#pragma unroll
    for (int m = 0; m < DN_W16; m++) {
        const int i = (int)threadIdx.x + 256 * m;
        wv4[m] = i < n16 ? src[i] : make_uint4(0u, 0u, 0u, 0u);
    }
    const int q = lane % LR, rw = lane / LR;
    const int b = q >> 3, u = q & 7, n = u >> 2, tt = u & 3;
    const uint32_t i2 = (uint32_t)tt >> 1;
    const int n_it = (DN_RG / 4) / RW;  // row groups of this wave: 8 (nbi 2) or 4 (nbi 1)
#pragma unroll
    for (int m = 0; m < DN_W16; m++) {
        const int i = (int)threadIdx.x + 256 * m;
        if (i < n16) reinterpret_cast<uint4 *>(wsm)[i] = wv4[m];
    }
    if (st_p < cnt && st_r < Is / 8) {
        *reinterpret_cast<float4 *>(&hs[st_p][hpad(8 * st_r)]) = hv0;
        *reinterpret_cast<float4 *>(&hs[st_p][hpad(8 * st_r + 4)]) = hv1;
        float sm = hv0.x;
        sm += hv0.y;
        sm += hv0.z;
        sm += hv0.w;
        sm += hv1.x;
        sm += hv1.y;
        sm += hv1.z;
        sm += hv1.w;
        // run r8 of a row: superblock r8 / 32, half (r8 / 16) % 2, s = (r8 / 4) % 4, tt = r8 % 4
        const int rb8 = st_r >> 5, rn = (st_r >> 4) & 1, rs = (st_r >> 2) & 3, rt = st_r & 3;
        reinterpret_cast<float *>(&hsum[st_p][(2 * rb8 + rn) * 4 + rt])[rs] = sm;
    }
    __syncthreads();
    const int base = b * QK + 128 * n + 8 * tt;
    const int ui = (2 * b + n) * 4 + tt;  // this lane's unit
#pragma unroll
    for (int it = 0; it < DN_IT; it++) {
        if (it >= n_it) break;  // uniform over the wave
        const int jr = j0 + it * RW + rw;
        const uint32_t blk = (uint32_t)((jr - (int)blockIdx.y * DN_RG) * (int)rbd + b * Q6K_BYTES);
        const uint2 a0 = lds8_a2(wsm, blk + 64 * n + 8 * tt);
        const uint2 a1 = lds8_a2(wsm, blk + 64 * n + 32 + 8 * tt);
        const uint2 ah = lds8_a2(wsm, blk + 128 + 32 * n + 8 * tt);
        const uint2 sw = lds8_a2(wsm, blk + 192 + 8 * n);
        const float dd = h2f(lds16_a2(wsm, blk + 208));
        float qf[4][8], sc[4];
        q6_codes(a0, a1, ah, qf);
#pragma unroll
        for (int ss = 0; ss < 4; ss++) sc[ss] = q6k_scale(sw, i2 + 2 * ss);
        for (int p = 0; p < cnt; p++) {
            float A[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ss = 0; ss < 4; ss++) {
                const float4 va = *reinterpret_cast<const float4 *>(&hs[p][hpad(base + 32 * ss)]);
                const float4 vb = *reinterpret_cast<const float4 *>(&hs[p][hpad(base + 32 * ss + 4)]);
                A[ss] = fmaf(qf[ss][0], va.x, A[ss]);
                A[ss] = fmaf(qf[ss][1], va.y, A[ss]);
                A[ss] = fmaf(qf[ss][2], va.z, A[ss]);
                A[ss] = fmaf(qf[ss][3], va.w, A[ss]);
                A[ss] = fmaf(qf[ss][4], vb.x, A[ss]);
                A[ss] = fmaf(qf[ss][5], vb.y, A[ss]);
                A[ss] = fmaf(qf[ss][6], vb.z, A[ss]);
                A[ss] = fmaf(qf[ss][7], vb.w, A[ss]);
            }
            const float4 X = hsum[p][ui];
            float rr = 0.f;
            rr = fmaf(sc[0], fmaf(-32.f, X.x, A[0]), rr);
            rr = fmaf(sc[1], fmaf(-32.f, X.y, A[1]), rr);
            rr = fmaf(sc[2], fmaf(-32.f, X.z, A[2]), rr);
            rr = fmaf(sc[3], fmaf(-32.f, X.w, A[3]), rr);
            float v = dd * rr;
            v = LR == 16 ? sum16(v) : sum8(v);
            const int pr = prs[p];
            if (q == 0 && jr < H && pr >= 0) eo[(size_t)pr * H + jr] = v;
        }
    }
}

// ---- combine -------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_sb_combine(float *__restrict__ hidden, const float *__restrict__ eo,
                                                    const float *__restrict__ w, const float *__restrict__ gsh, int H,
                                                    int K)
{
#pragma clang fp contract(off)
    const int t = (int)blockIdx.x;
    const int c = ((int)blockIdx.y * 256 + (int)threadIdx.x) * 4;
    if (c >= H) return;
    const float sw = 1.0f / (1.0f + expf(-gsh[t]));  // one_layer.cu:1443-1447
    const float *et = eo + (size_t)t * (K + 1) * H + c;
    float4 v = *reinterpret_cast<const float4 *>(hidden + (size_t)t * H + c);
    float4 a = *reinterpret_cast<const float4 *>(et);
    v.x += sw * a.x;
    v.y += sw * a.y;
    v.z += sw * a.z;
    v.w += sw * a.w;
    for (int k = 0; k < K; k++) {
        const float wk = w[(size_t)t * K + k];
        a = *reinterpret_cast<const float4 *>(et + (size_t)(k + 1) * H);
        v.x += wk * a.x;
        v.y += wk * a.y;
        v.z += wk * a.z;
        v.w += wk * a.w;
    }
    *reinterpret_cast<float4 *>(hidden + (size_t)t * H + c) = v;
}

}  // namespace

bool bread_small_supported(const bread_moe_shape_t &s, const bread_moe_layer_t *L)
{
    const bool io = (s.expert_inter == 256 || s.expert_inter == 512) &&
                    (s.shared_inter == 256 || s.shared_inter == 512);
    return s.hidden % QK == 0 && s.hidden <= MAX_H && io && s.n_experts <= MAX_E && s.top_k <= MAX_K &&
           L->gate_type == BREAD_QTYPE_Q4_K && L->up_type == BREAD_QTYPE_Q4_K && L->down_type == BREAD_QTYPE_Q6_K &&
           L->gate_shexp_type == BREAD_QTYPE_Q4_K && L->up_shexp_type == BREAD_QTYPE_Q4_K &&
           L->down_shexp_type == BREAD_QTYPE_Q6_K && (((uintptr_t)L->down_exps | (uintptr_t)L->down_shexp |
                                                       L->down_expert_bytes) & 15) == 0;
}

int bread_small_max_tokens()
{
    return SB_MAX_T;
}

extern "C" int bread_small_auto_tokens(void)
{
    return SB_AUTO_T;
}

// Slots of a call with T tokens: the shared expert's chunks plus, per chosen
// expert, ceil(n_e / SB_CH) <= 1 + (n_e - 1) / SB_CH chunks.
static int sb_slots(int T, int K, int E)
{
    const int pairs = T * K;
    return (T + SB_CH - 1) / SB_CH + (pairs < E ? pairs : E) + pairs / SB_CH + 1;
}

int bread_small_alloc(bread_moe_ctx_t *c)
{
    const bread_moe_shape_t &s = c->shape;
    const size_t T = (size_t)(c->max_tokens < SB_MAX_T ? c->max_tokens : SB_MAX_T);
    const size_t K = (size_t)s.top_k, H = (size_t)s.hidden;
    const size_t S = (size_t)sb_slots((int)T, (int)K, s.n_experts);
    bread_small_ws &g = c->sws;
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = hipMalloc((void **)&g.slot_expert, S * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&g.slot_cnt, S * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&g.slot_pair, S * SB_CH * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&g.n_slots, sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&g.eo, T * (K + 1) * H * sizeof(float));
    if (e == hipSuccess) e = hipMemset(g.n_slots, 0, sizeof(int32_t));
    if (e == hipSuccess) e = hipMemset(g.slot_expert, 0, S * sizeof(int32_t));
    if (e == hipSuccess) e = hipMemset(g.slot_cnt, 0, S * sizeof(int32_t));
    if (e == hipSuccess) e = hipMemset(g.slot_pair, 0, S * SB_CH * sizeof(int32_t));
    return e == hipSuccess ? BREAD_OK : (e == hipErrorOutOfMemory ? BREAD_ERR_NOMEM : BREAD_ERR_HIP);
}

void bread_small_free(bread_moe_ctx_t *c)
{
    bread_small_ws &g = c->sws;
    (void)hipFree(g.slot_expert);
    (void)hipFree(g.slot_cnt);
    (void)hipFree(g.slot_pair);
    (void)hipFree(g.n_slots);
    (void)hipFree(g.eo);
    g = bread_small_ws{};
}

int bread_launch_moe_small(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, float *hidden, int T,
                           hipStream_t st)
{
    const bread_moe_shape_t &s = c->shape;
    if (T < 1 || T > SB_MAX_T || T > c->max_tokens || !bread_small_supported(s, L)) return BREAD_ERR_SHAPE;
    const int H = s.hidden, I = s.expert_inter, Ish = s.shared_inter, E = s.n_experts, K = s.top_k;
    const int Imax = I > Ish ? I : Ish;
    const int S = sb_slots(T, K, E);
    const bread_small_ws &g = c->sws;
    const SbLayer sl{(const uint8_t *)L->gate_exps, (const uint8_t *)L->up_exps, (const uint8_t *)L->down_exps,
                     (const uint8_t *)L->gate_shexp, (const uint8_t *)L->up_shexp, (const uint8_t *)L->down_shexp,
                     L->gate_expert_bytes, L->up_expert_bytes, L->down_expert_bytes};
    const SbSlots ss{g.slot_expert, g.slot_cnt, g.slot_pair, g.n_slots};
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_sb_router, dim3((E + 1 + 3) / 4), dim3(256), 0, st, L->router, L->shexp_gate, x, c->logits,
                       c->gsh, H, E, T);
    if (E <= 4 * WAVE)
        hipLaunchKernelGGL(k_sb_select<4>, dim3(1), dim3(RT_THREADS), 0, st, c->logits, E, K, T, c->idx, c->w,
                           g.slot_expert, g.slot_cnt, g.slot_pair, g.n_slots);
    else
        hipLaunchKernelGGL(k_sb_select<16>, dim3(1), dim3(RT_THREADS), 0, st, c->logits, E, K, T, c->idx, c->w,
                           g.slot_expert, g.slot_cnt, g.slot_pair, g.n_slots);
    hipLaunchKernelGGL(k_sb_gateup, dim3(S, (Imax + GU_RG - 1) / GU_RG), dim3(256), 0, st, sl, x, ss, c->h, H, I,
                       Ish, E, K, T, Imax);
    hipLaunchKernelGGL(k_sb_down, dim3(S, (H + DN_RG - 1) / DN_RG), dim3(256), 0, st, sl, c->h, ss, g.eo, H, I, Ish,
                       E, K, T, Imax);
    hipLaunchKernelGGL(k_sb_combine, dim3(T, (H + 1023) / 1024), dim3(256), 0, st, hidden, g.eo, c->w, c->gsh, H,
                       K);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}
