// moe_small.hip — the small-batch MoE path (2 <= n_tokens <= 32; the
// automatic choice uses it up to 16: batched decode, speculative-verify
// rounds).  At the decode shape (H 2048, I = I_sh = 512, K <= 8) and up to
// 16 tokens, k_sw_gateup and k_sw_down (end of the file) replace the
// per-slot gate/up, down and combine kernels.
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
//   k_route_fast  router logits and shared-gate scores summed in parallel,
//                 each logit with a rigorous radius around the reference's
//                 sequential sum (route.hip).
//   k_sb_route    one workgroup: per token, the certificate and selection
//                 from the fast logits, or the reference-order sums of the
//                 candidate rows (route_cert.h; indices bit-identical to the
//                 reference's), then slots: an expert's tokens in chunks of
//                 at most SB_CH (the shared expert's chunks first, with every
//                 token, then the chosen experts in expert order), each with
//                 its (token, rank) pairs in token order.  Chunks spread a
//                 hot expert over more workgroups.  Shapes beyond the fast
//                 sums' limits take k_route_seq (the reference's order) and
//                 k_sb_select (the host's selection) instead.
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
#include "route_cert.h"
#include "route_dev.h"

namespace {

constexpr int SB_MAX_T = 32;      // tokens per call (token bitmasks are 32 bits)
constexpr int SB_AUTO_T = 16;     // the automatic choice takes this path up to here (measured crossover)
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

// The experts chosen by any token numbered into slots in expert order (the
// shared expert's slots first, with every token), each slot with its
// (token, rank) pairs in token order, from per-expert token bitmasks.
// sidx[t K + k] (LDS): rank k's expert of token t, complete before the call.
// One workgroup of RT_THREADS.
__device__ void sb_number_slots(const int *sidx, int E, int K, int T, int32_t *__restrict__ slot_expert,
                         int32_t *__restrict__ slot_cnt, int32_t *__restrict__ slot_pair,
                         int32_t *__restrict__ n_slots)
{
    __shared__ uint32_t mask[MAX_E];  // tokens that chose expert e
    __shared__ int slot_of[MAX_E];
    __shared__ int wave_tot[RT_WAVES];
    const int tid = (int)threadIdx.x, wv = tid / WAVE, lane = lane_id();
    for (int e = tid; e < E; e += RT_THREADS) mask[e] = 0u;
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
    const int incl = wave_scan_incl(nch);  // inclusive scan of the chunk counts over the experts
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

// Softmax / top-k per token with the host's arithmetic (topk_wave_exact) on
// the reference-order logits, then the slots.  One workgroup.
template <int MAXV>
__global__ __launch_bounds__(RT_THREADS) void k_sb_select(const float *__restrict__ logits, int E, int K, int T,
                                                          int32_t *__restrict__ idx, float *__restrict__ w,
                                                          int32_t *__restrict__ slot_expert,
                                                          int32_t *__restrict__ slot_cnt,
                                                          int32_t *__restrict__ slot_pair,
                                                          int32_t *__restrict__ n_slots)
{
    __shared__ int sidx[SB_MAX_T * MAX_K];
    __shared__ __attribute__((aligned(16))) float s_e[RT_WAVES][WAVE * MAXV];  // softmax scratch of each wave
    const int wv = (int)threadIdx.x / WAVE, lane = lane_id();
    for (int t = wv; t < T; t += RT_WAVES) {
        int ik;
        float wk;
        topk_wave_exact<MAXV>(logits + (size_t)t * E, E, K, s_e[wv], ik, wk);
        if (lane < K) {
            idx[(size_t)t * K + lane] = ik;
            w[(size_t)t * K + lane] = wk;
            sidx[t * K + lane] = ik;
        }
    }
    __syncthreads();
    sb_number_slots(sidx, E, K, T, slot_expert, slot_cnt, slot_pair, n_slots);
}

// Certified routing from the fast logits and radii (k_route_fast), then the
// slots.  Wave v takes tokens v, v + 16, ...: a token the certificate
// vouches for (cert_select_wave) gets its experts and weights at once; the
// others are then routed one after another by the whole workgroup from the
// reference-order sums of their candidate rows (route_token_exact).  Counts
// the three outcomes in stats.  One workgroup.
template <int MAXV>
__global__ __launch_bounds__(RT_THREADS) void k_sb_route(const float *__restrict__ router,
                                                         const float *__restrict__ x, const float *__restrict__ logits,
                                                         const float *__restrict__ radii, int H, int E, int K, int T,
                                                         int32_t *__restrict__ idx, float *__restrict__ w,
                                                         int32_t *__restrict__ slot_expert,
                                                         int32_t *__restrict__ slot_cnt,
                                                         int32_t *__restrict__ slot_pair,
                                                         int32_t *__restrict__ n_slots, uint32_t *__restrict__ stats)
{
    __shared__ RxSmem S;
    __shared__ int sidx[SB_MAX_T * MAX_K];
    __shared__ int s_cand[SB_MAX_T][RX_CAND];
    __shared__ int s_ncand[SB_MAX_T];
    __shared__ int s_list[SB_MAX_T];
    __shared__ int s_n;
    __shared__ uint64_t s_tab[32];
    static_assert(RT_WAVES * 2 * RX_MAX_E <= RX_CH * RX_ROW, "certificate scratch in S.prod");
    const int tid = (int)threadIdx.x, wv = tid / WAVE, lane = lane_id();
    if (tid == 0) s_n = 0;
    __syncthreads();
    // expf's table for the exact selection, requested now and stored after
    // the certificates (its wait then costs nothing)
    const uint64_t tabv = libm_expf_tab(tid);
    for (int t = wv; t < T; t += RT_WAVES) {
        int ik = 0, nc = 0;
        float wk = 0.f;
        // scratch: S.prod, free until the reference-order sums below
        const int r = cert_select_wave<MAXV>(logits + (size_t)t * E, radii + (size_t)t * E, E, K, ik, wk,
                                             s_cand[t], nc, &S.prod[0][0] + wv * 2 * RX_MAX_E);
        if (r == 1) {
            if (lane < K) {
                idx[(size_t)t * K + lane] = ik;
                w[(size_t)t * K + lane] = wk;
                sidx[t * K + lane] = ik;
            }
        } else if (lane == 0) {
            s_ncand[t] = r == 0 ? nc : -1;
            s_list[atomicAdd(&s_n, 1)] = t;
        }
    }
    if (tid < 32) s_tab[tid] = tabv;
    __syncthreads();
    const int n = s_n;
    int nfull = 0;
    for (int i = 0; i < n; i++) {
        const int t = s_list[i];
        int ik = 0;
        float wk = 0.f;
        const int how = route_token_exact<MAXV, RT_THREADS>(S, router, x + (size_t)t * H, s_cand[t], s_ncand[t], H,
                                                            E, K, s_tab, ik, wk);
        if (tid < K) {
            idx[(size_t)t * K + tid] = ik;
            w[(size_t)t * K + tid] = wk;
            sidx[t * K + tid] = ik;
        }
        nfull += how == 2 ? 1 : 0;
    }
    __syncthreads();
    if (tid == 0) {
        if (n < T) atomicAdd(&stats[BREAD_RSTAT_MT_CERT], (uint32_t)(T - n));
        if (n > nfull) atomicAdd(&stats[BREAD_RSTAT_MT_CAND], (uint32_t)(n - nfull));
        if (nfull) atomicAdd(&stats[BREAD_RSTAT_MT_EXACT], (uint32_t)nfull);
    }
    sb_number_slots(sidx, E, K, T, slot_expert, slot_cnt, slot_pair, n_slots);
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

// ---- wide kernels at the decode shape (H 2048, I = I_sh = 512, K <= 8) ---------------
//
// k_sw_gateup and k_sw_down replace k_sb_gateup, k_sb_down and k_sb_combine at
// the decode kernel's shape.  Every workgroup owns a slice of every slot, as
// the decode kernel's workgroups do: gate/up rows 2g and 2g+1, output rows
// 8g..8g+7.  Each CU then has loads of all its slots in flight at once,
// where the per-slot workgroups of the general kernels form chains of small
// dependent steps.  The gate/up dots use the decode kernel's integer form
// (x in 16-bit block fixed point, q4k_chunk_dot_q16; k_route_fast converts
// each token once, xq16_store); the down dots are fp32
// on pre-decoded weights; the combine runs in the down kernel.

constexpr int SW_G = 256;                                         // workgroups
constexpr int SW_NT = 1024;                                       // threads per workgroup
constexpr int SW_NW = SW_NT / WAVE;                               // 16 waves
constexpr int SW_H = 2048;
constexpr int SW_I = 512;
constexpr int SW_K = 8;                                           // top-k at most
constexpr int SW_MAX_T = 16;
constexpr int SW_GU_BYTES = 4 * (SW_H / QK) * Q4K_BYTES;          // gate rows 2g, 2g+1, then up: 4608
constexpr int SW_GU_CH = SW_GU_BYTES / 16;                        // 288 16-byte chunks
constexpr int SW_GU_LOADS = (SW_GU_CH + WAVE - 1) / WAVE;         // 5
constexpr int SW_ROW16 = (SW_H / QK) * Q4K_BYTES / 16;            // one gate/up row: 72 chunks
constexpr int SW_DN_BYTES = 4 * (SW_I / QK) * Q6K_BYTES;          // four down rows: 1680
constexpr int SW_DN_CH = SW_DN_BYTES / 16;                        // 105
constexpr int SW_DN_LOADS = (SW_DN_CH + WAVE - 1) / WAVE;         // 2
constexpr int SW_DN_ROW = (SW_I / QK) * Q6K_BYTES;                // 420
constexpr int SW_MAX_P = SW_MAX_T * (SW_K + 1);                   // pairs
// s_waitcnt lgkmcnt(0) with vmcnt and expcnt left at their maxima (gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int WAITCNT_LGKM0 = 0xF | (0x7 << 4) | (0x3 << 14);
static_assert(SW_I / SW_G == 2 && SW_H / SW_G == 8, "row ownership assumes 256 workgroups");
static_assert(SW_GU_BYTES % 16 == 0 && SW_DN_BYTES % 16 == 0, "16-byte loads");

struct SwGuSmem {
    uint4 w[SW_NW][SW_GU_LOADS][WAVE];       // each wave's slot: gate rows 2g, 2g+1, up rows 2g, 2g+1
    uint32_t xqh[SW_MAX_T][SW_H / 4];        // x in 16-bit block fixed point: high bytes
    uint32_t xql[SW_MAX_T][SW_H / 4];        // low bytes
    float xqs[SW_MAX_T][SW_H / 32];          // block scales
    float xsum[SW_MAX_T][SW_H / 16];         // fp32 sums of 16-column runs
    float red[SW_NW][16];                    // each wave's reduced dots
};
static_assert(sizeof(SwGuSmem) <= 160 * 1024, "LDS");

// The slot's gate/up rows of this workgroup into the wave's LDS staging.
__device__ __forceinline__ void sw_gu_issue(SwGuSmem &M, const SbLayer &L, int e, int g, int wid, int lane)
{
    const uint8_t *gs = (e < 0 ? L.gate_sh : L.gate_exps + (uint64_t)e * L.gate_eb) + (size_t)(2 * g) * SW_ROW16 * 16;
    const uint8_t *us = (e < 0 ? L.up_sh : L.up_exps + (uint64_t)e * L.up_eb) + (size_t)(2 * g) * SW_ROW16 * 16;
#pragma unroll
    for (int k = 0; k < SW_GU_LOADS; k++) {
        const int c = WAVE * k + lane;
        if (c < SW_GU_CH) {
            const uint8_t *src = c < 2 * SW_ROW16 ? gs + 16 * c : us + 16 * (c - 2 * SW_ROW16);
            __builtin_amdgcn_global_load_lds(src, &M.w[wid][k][0], 16, 0, 0);
        }
    }
}

// Transposed wave reduction steps: two values a, b a lane become one, each
// summed over a pair of lane groups, a kept by the lower group and b by the
// upper.  tr32 pairs lane L with L^32 (permlane32 swap), tr16 L with L^16
// inside each half (permlane16 swap), tr8 and tr4 L with the mirrored lane
// of the 16- or 8-lane group (DPP).  The swaps' two results pass through an
// empty asm: hipcc (ROCm 7.2) otherwise adds result 0 to itself when both
// results of a swap with two different operands meet in one sum.
__device__ __forceinline__ float tr32(float a, float b)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                    false, false);
    uint32_t r0 = r[0], r1 = r[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float tr16(float a, float b)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                    false, false);
    uint32_t r0 = r[0], r1 = r[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float tr8(float a, float b, int lane)
{
    const bool hi = (lane & 8) != 0;
    return (hi ? b : a) + dpp_f<0x140>(hi ? a : b);  // row_mirror: lane i reads 15 - i
}

__device__ __forceinline__ float tr4(float a, float b, int lane)
{
    const bool hi = (lane & 4) != 0;
    return (hi ? b : a) + dpp_f<0x141>(hi ? a : b);  // row_half_mirror: lane i reads 7 - i of its 8
}

// v[i] summed over the wave lands in lanes 4i .. 4i+3.
__device__ __forceinline__ float reduce16(const float (&v)[16], int lane)
{
    float u[8], w4[4], x2[2];
#pragma unroll
    for (int i = 0; i < 8; i++) u[i] = tr32(v[i], v[i + 8]);
#pragma unroll
    for (int i = 0; i < 4; i++) w4[i] = tr16(u[i], u[i + 4]);
#pragma unroll
    for (int i = 0; i < 2; i++) x2[i] = tr8(w4[i], w4[i + 2], lane);
    float y = tr4(x2[0], x2[1], lane);
    y += dpp_f<0xB1>(y);  // quad_perm [1,0,3,2]
    y += dpp_f<0x4E>(y);  // quad_perm [2,3,0,1]
    return y;
}

__global__ __launch_bounds__(SW_NT, 1) void k_sw_gateup(SbLayer L, const uint8_t *__restrict__ xq, SbSlots S,
                                                        float *__restrict__ h, int E, int K, int T, int max_slots)
{
    __shared__ SwGuSmem M;
    static_assert(XQ_H == SW_H, "fixed-point record layout");
    const int g = (int)blockIdx.x, tid = (int)threadIdx.x, wid = tid / WAVE, lane = lane_id();
    const int P = T * (K + 1);
    int ns = *S.n;
    ns = ns < max_slots ? (ns > 0 ? ns : 0) : max_slots;
    // the activations' fixed-point records requested first (a wait for them
    // must not include the weights), then the first slot's weights, then the
    // records into LDS
    constexpr int XU = XQ_TOKEN_BYTES / 16;                   // 16-byte units a token (304)
    constexpr int XI = (SW_MAX_T * XU + SW_NT - 1) / SW_NT;   // units a thread (5)
    uint4 xr[XI];
#pragma unroll
    for (int i = 0; i < XI; i++) {
        const int it = SW_NT * i + tid;
        xr[i] = it < T * XU ? reinterpret_cast<const uint4 *>(xq)[it] : make_uint4(0u, 0u, 0u, 0u);
    }
    int e0 = -2;
    if (wid < ns) {
        e0 = __builtin_amdgcn_readfirstlane(S.expert[wid]);
        if (e0 >= -1 && e0 < E) sw_gu_issue(M, L, e0, g, wid, lane);
    }
#pragma unroll
    for (int i = 0; i < XI; i++) {
        const int it = SW_NT * i + tid, t = it / XU, u = it % XU;
        if (it < T * XU) {
            uint4 *dst = u < XQ_LO / 16   ? reinterpret_cast<uint4 *>(&M.xqh[t][0]) + u
                         : u < XQ_SC / 16 ? reinterpret_cast<uint4 *>(&M.xql[t][0]) + (u - XQ_LO / 16)
                         : u < XQ_SUM / 16 ? reinterpret_cast<uint4 *>(&M.xqs[t][0]) + (u - XQ_SC / 16)
                                           : reinterpret_cast<uint4 *>(&M.xsum[t][0]) + (u - XQ_SUM / 16);
            *dst = xr[i];
        }
    }
    __syncthreads();
    const int base = (lane >> 3) * QK + 64 * ((lane & 7) >> 1) + 16 * (lane & 1);  // the lane's columns (gu_base)
    const uint32_t j = (uint32_t)(lane & 7) >> 1;
    const int sbl = lane >> 3, cq = lane & 7;
    const uint4 *wf = &M.w[wid][0][0];
    // the staging holds slot s; the next slot's loads go out as soon as slot
    // s is unpacked into registers, so they overlap its dot products
    int e = e0;
    for (int s = wid; s < ns; s += SW_NW) {
        const int sn = s + SW_NW;
        const int en = sn < ns ? __builtin_amdgcn_readfirstlane(S.expert[sn]) : -2;
        const int cnt_s = __builtin_amdgcn_readfirstlane(S.cnt[s]);
        const bool ok = e >= -1 && e < E;
        const int cnt = ok ? (cnt_s < SB_CH ? (cnt_s > 0 ? cnt_s : 0) : SB_CH) : 0;
        int pr[SB_CH], tk[SB_CH];
#pragma unroll
        for (int k = 0; k < SB_CH; k++) {
            const int p = k < cnt ? __builtin_amdgcn_readfirstlane(S.pair[(size_t)s * SB_CH + k]) : -1;
            pr[k] = p >= 0 && p < P ? p : -1;
            // the pair's token, divided on the scalar unit (the pair index
            // is wave-uniform; a vector division costs ~15 instructions a token)
            tk[k] = __builtin_amdgcn_readfirstlane(pr[k] >= 0 ? pr[k] : 0) / (K + 1);
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's staging has landed
        // the four row chunks of the lane (m = 2 mat + row: gate rows 0, 1,
        // up rows 0, 1), unpacked once for every token of the slot
        uint32_t qlo[4][4], qhi[4][4];
        float dsc0[4], dsc1[4], dm0[4], dm1[4];
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int hx = SW_ROW16 * (m & 1) + 2 * SW_ROW16 * (m >> 1) + 9 * sbl;
            const uint4 hd = wf[hx], q = wf[hx + 1 + cq];
            const uint32_t scm = q4k_scale_pair(hd, j);
            const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
            dsc0[m] = d * (float)byte_of(scm, 0);
            dsc1[m] = d * (float)byte_of(scm, 1);
            dm0[m] = dmin * (float)byte_of(scm, 2);
            dm1[m] = dmin * (float)byte_of(scm, 3);
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                qlo[m][t] = qw[t] & 0x0F0F0F0Fu;
                qhi[m][t] = (qw[t] >> 4) & 0x0F0F0F0Fu;
            }
        }
        // the staging is read (the LDS reads above completed): next slot's loads
        __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
        if (en >= -1 && en < E) sw_gu_issue(M, L, en, g, wid, lane);
        e = en;
        if (!ok) continue;
        // v[4 m + k]: the lane's part of row chunk m times token k
        float v[16];
#pragma unroll
        for (int k = 0; k < SB_CH; k++) {
            if (k >= cnt) {  // wave-uniform: a slot's missing tokens cost nothing
#pragma unroll
                for (int m = 0; m < 4; m++) v[4 * m + k] = 0.f;
                continue;
            }
            const int t = tk[k];
            const uint4 lh = *reinterpret_cast<const uint4 *>(&M.xqh[t][base >> 2]);
            const uint4 ll = *reinterpret_cast<const uint4 *>(&M.xql[t][base >> 2]);
            const uint4 hh = *reinterpret_cast<const uint4 *>(&M.xqh[t][(base >> 2) + 8]);
            const uint4 hl = *reinterpret_cast<const uint4 *>(&M.xql[t][(base >> 2) + 8]);
            const float2 sc = *reinterpret_cast<const float2 *>(&M.xqs[t][base >> 5]);
            const float sxl = M.xsum[t][base >> 4], sxh = M.xsum[t][(base >> 4) + 2];
            const uint32_t xlh[4] = {lh.x, lh.y, lh.z, lh.w}, xll[4] = {ll.x, ll.y, ll.z, ll.w};
            const uint32_t xhh[4] = {hh.x, hh.y, hh.z, hh.w}, xhl[4] = {hl.x, hl.y, hl.z, hl.w};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                // 256 sum(q hi) + sum(q lo) in one chain per nibble half
                // (exact: below 2^23), one zeroed accumulator each
                int a_l = 0, a_h = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    a_l = __builtin_amdgcn_sdot4((int)qlo[m][q], (int)xlh[q], a_l, false);
                    a_h = __builtin_amdgcn_sdot4((int)qhi[m][q], (int)xhh[q], a_h, false);
                }
                a_l *= 256;
                a_h *= 256;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    a_l = __builtin_amdgcn_sdot4((int)qlo[m][q], (int)xll[q], a_l, false);
                    a_h = __builtin_amdgcn_sdot4((int)qhi[m][q], (int)xhl[q], a_h, false);
                }
                const float al = (float)a_l * sc.x;
                const float ah = (float)a_h * sc.y;
                v[4 * m + k] = dsc0[m] * al - dm0[m] * sxl + dsc1[m] * ah - dm1[m] * sxh;
            }
        }
        const float tot = reduce16(v, lane);
        if ((lane & 3) == 0) M.red[wid][lane >> 2] = tot;
        __builtin_amdgcn_wave_barrier();
        // lane k < cnt: token k's SwiGLU of rows 2g, 2g+1 (gate m = row, up m = 2 + row)
        if (lane < cnt) {
            int p = pr[0];
#pragma unroll
            for (int k = 1; k < SB_CH; k++)
                if (lane == k) p = pr[k];
            if (p >= 0) {
                const float h0 = silu_mul(M.red[wid][lane], M.red[wid][8 + lane]);
                const float h1 = silu_mul(M.red[wid][4 + lane], M.red[wid][12 + lane]);
                *reinterpret_cast<float2 *>(h + (size_t)p * SW_I + 2 * g) = make_float2(h0, h1);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

struct SwDnSmem {
    uint4 band[SW_NW][SW_DN_LOADS][WAVE];  // each wave's four down rows of its slot
    float hst[SW_NW / 2][SB_CH][SW_I];     // the slot's SwiGLU rows, shared by its two waves
    float dot[SW_MAX_P][8];                // per pair: the workgroup's eight output rows
    int hin[SW_NW];                        // per wave: rounds whose loads have landed
    int hout[SW_NW];                       // per wave: rounds whose SwiGLU rows it has used
    int bad;                               // a wait on a partner wave ran out: no output
};
static_assert(sizeof(SwDnSmem) <= 160 * 1024, "LDS");

// Sleeps a partner wait allows after its first look, by default.
constexpr uint32_t SW_SPIN_DEFAULT = 1u << 20;

// Bounded wait on a partner wave's LDS round counter, sleeping at most lim
// times; false when it runs out.
__device__ __forceinline__ bool sw_wait(const int *p, int target, uint32_t lim)
{
    bool ok = false;
    for (uint32_t it = 0;; it++) {
        if (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) {
            ok = true;
            break;
        }
        if (it >= lim) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return ok;
}

__device__ __forceinline__ void sw_put(int *p, int v)
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waves 2m and 2m+1 take slots m, m + 8, ...: each its four of the
// workgroup's eight down rows, and half of the slot's SwiGLU rows staged in
// LDS for both.  Lane l = lane % 16 of row rr = lane / 16 owns columns
// 64 jj + 4 l + k (jj < 8, k < 4), so a 16-byte read of one SwiGLU row covers
// 256 consecutive bytes: superblock b = jj / 4, half n = (jj / 2) % 2, group
// s = 2 (jj % 2) + l / 8, element 4 (l % 8) + k: the low / high nibbles of ql
// bytes 64n + 32 (l / 8) + 4 (l % 8) + k and bit pairs s of the qh bytes
// 32n + 4 (l % 8) + k, with scales 8n + (l % 8) / 4 + 2s
// (dequant_q4k_cpu.c:155-170).
// A partner wait that runs out (after spin sleeps) leaves that round's dots
// unstored; the workgroup then writes none of its rows of hidden and sets
// BREAD_DEV_ERR_PAIR in *err.
__global__ __launch_bounds__(SW_NT, 1) void k_sw_down(SbLayer L, const float *__restrict__ h, SbSlots S,
                                                      float *__restrict__ hidden, const float *__restrict__ w,
                                                      const float *__restrict__ gsh, int E, int K, int T,
                                                      int max_slots, uint32_t *err, uint32_t spin)
{
    __shared__ SwDnSmem M;
    const int g = (int)blockIdx.x, tid = (int)threadIdx.x, wid = tid / WAVE, lane = lane_id();
    const int P = T * (K + 1);
    for (int i = tid; i < SW_MAX_P * 8; i += SW_NT) (&M.dot[0][0])[i] = 0.f;
    if (tid < SW_NW) {
        M.hin[tid] = 0;
        M.hout[tid] = 0;
    }
    if (tid == 0) M.bad = 0;
    int ns = *S.n;
    ns = ns < max_slots ? (ns > 0 ? ns : 0) : max_slots;
    const int m2 = wid >> 1, u = wid & 1, pw = wid ^ 1;
    const int l = lane & 15, rr = lane >> 4, sl = l >> 3, l7 = l & 7;
    const uint32_t *band = reinterpret_cast<const uint32_t *>(&M.band[wid][0][0]);
    __syncthreads();
    // slot metadata of a round; an invalid slot has no pairs (both waves of
    // a pair see the same slots and keep the round counters in step)
    auto meta = [&](int s, int &e, int &cnt, int (&pr)[SB_CH]) {
        e = s < ns ? __builtin_amdgcn_readfirstlane(S.expert[s]) : -2;
        const bool ok = e >= -1 && e < E;
        const int cnt_s = ok ? __builtin_amdgcn_readfirstlane(S.cnt[s]) : 0;
        cnt = ok ? (cnt_s < SB_CH ? (cnt_s > 0 ? cnt_s : 0) : SB_CH) : 0;
#pragma unroll
        for (int k = 0; k < SB_CH; k++) {
            const int p = k < cnt ? __builtin_amdgcn_readfirstlane(S.pair[(size_t)s * SB_CH + k]) : -1;
            pr[k] = p >= 0 && p < P ? p : -1;
        }
    };
    auto issue_band = [&](int e) {
        const uint8_t *src = (e < 0 ? L.down_sh : L.down_exps + (uint64_t)e * L.down_eb) +
                             (size_t)(8 * g + 4 * u) * SW_DN_ROW;
#pragma unroll
        for (int k = 0; k < SW_DN_LOADS; k++) {
            const int c = WAVE * k + lane;
            if (c < SW_DN_CH) __builtin_amdgcn_global_load_lds(src + 16 * c, &M.band[wid][k][0], 16, 0, 0);
        }
    };
    // this wave's pairs (k % 2 == u) of the slot's SwiGLU rows: 2 KB, two loads each
    auto issue_h = [&](const int (&pr)[SB_CH]) {
#pragma unroll
        for (int k = 0; k < SB_CH; k++) {
            if ((k & 1) != u || pr[k] < 0) continue;
            const float *hs = h + (size_t)pr[k] * SW_I;
#pragma unroll
            for (int q = 0; q < SW_I / (4 * WAVE); q++)
                __builtin_amdgcn_global_load_lds(hs + 4 * (WAVE * q + lane), &M.hst[m2][k][4 * WAVE * q], 16, 0, 0);
        }
    };
    int e, cnt, pr[SB_CH];
    meta(m2, e, cnt, pr);
    if (cnt > 0) {
        issue_band(e);
        issue_h(pr);
    }
    int rnd = 0;
    for (int s = m2; s < ns; s += SW_NW / 2, rnd++) {
        int en, cntn, prn[SB_CH];
        meta(s + SW_NW / 2, en, cntn, prn);
        __builtin_amdgcn_s_waitcnt(0);  // this round's band and this wave's SwiGLU rows
        if (lane == 0) sw_put(&M.hin[wid], rnd + 1);
        const bool in = sw_wait(&M.hin[pw], rnd + 1, spin);
        if (!in && lane == 0) sw_put(&M.bad, 1);
        if (cnt > 0) {
            // pre-decode the lane's 32 weights of row rr: w[4 jj + k] = (d sc)
            // (q - 32) as fma(q, ds, -32 ds), one rounding
            float wq[32];
#pragma unroll
            for (int bn = 0; bn < 4; bn++) {
                const int b = bn >> 1, n = bn & 1;
                const uint32_t ob = (uint32_t)(rr * SW_DN_ROW + b * Q6K_BYTES);
                const uint32_t o1 = ob + 64 * n + 32 * sl + 4 * l7, o2 = ob + 128 + 32 * n + 4 * l7;
                const uint32_t ql = __builtin_amdgcn_alignbyte(band[(o1 + 3) >> 2], band[o1 >> 2], o1 & 3u);
                const uint32_t qh = __builtin_amdgcn_alignbyte(band[(o2 + 3) >> 2], band[o2 >> 2], o2 & 3u);
                const uint2 scw = lds8_a2(band, ob + 192 + 8 * n);
                const float d = h2f(lds16_a2(band, ob + 208));
                const uint32_t q[2] = {(ql & 0x0F0F0F0Fu) | (((qh >> (2 * sl)) & 0x03030303u) << 4),
                                       ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * sl + 4)) & 0x03030303u) << 4)};
#pragma unroll
                for (int ee = 0; ee < 2; ee++) {
                    const float ds = d * q6k_scale(scw, (uint32_t)((l7 >> 2) + 2 * (2 * ee + sl)));
                    const float nds = -32.0f * ds;
                    const int jj = 4 * b + 2 * n + ee;
#pragma unroll
                    for (int k = 0; k < 4; k++) wq[4 * jj + k] = fmaf((float)byte_of(q[ee], k), ds, nds);
                }
            }
            // the band is read: the next round's band goes out during the dots
            __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
            if (cntn > 0) issue_band(en);
#pragma unroll
            for (int k = 0; k < SB_CH; k++) {
                if (pr[k] < 0) continue;
                const float *hr = &M.hst[m2][k][4 * l];
                float acc = 0.f;
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const float4 hv = *reinterpret_cast<const float4 *>(hr + 64 * jj);
                    acc = fmaf(wq[4 * jj + 0], hv.x, acc);
                    acc = fmaf(wq[4 * jj + 1], hv.y, acc);
                    acc = fmaf(wq[4 * jj + 2], hv.z, acc);
                    acc = fmaf(wq[4 * jj + 3], hv.w, acc);
                }
                acc = sum16(acc);
                if (l == 0 && in) M.dot[pr[k]][4 * u + rr] = acc;
            }
        } else if (cntn > 0) {
            issue_band(en);
        }
        // both waves are done with this round's SwiGLU rows: the next round's
        __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
        if (lane == 0) sw_put(&M.hout[wid], rnd + 1);
        if (!sw_wait(&M.hout[pw], rnd + 1, spin) && lane == 0) sw_put(&M.bad, 1);
        if (cntn > 0) issue_h(prn);
        e = en;
        cnt = cntn;
#pragma unroll
        for (int k = 0; k < SB_CH; k++) pr[k] = prn[k];
    }
    __syncthreads();
    if (M.bad) {
        if (tid == 0) __hip_atomic_fetch_or(err, BREAD_DEV_ERR_PAIR, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // combine in the reference order (one_layer.cu:1443-1471): shared expert
    // first, then the routed experts by rank
    if (tid < T * 8) {
#pragma clang fp contract(off)
        const int t = tid >> 3, r = tid & 7;
        const int pb = t * (K + 1);
        float v = hidden[(size_t)t * SW_H + 8 * g + r];
        const float sw = 1.0f / (1.0f + expf(-gsh[t]));
        v += sw * M.dot[pb][r];
        for (int k = 0; k < K; k++) v += w[(size_t)t * K + k] * M.dot[pb + 1 + k][r];
        hidden[(size_t)t * SW_H + 8 * g + r] = v;
    }
}

}  // namespace

bool bread_small_supported(const bread_moe_shape_t &s, const bread_moe_layer_t *L)
{
    const bool io = (s.expert_inter == 256 || s.expert_inter == 512) &&
                    (s.shared_inter == 256 || s.shared_inter == 512);
    return s.hidden % QK == 0 && s.hidden <= MAX_H && io && s.n_experts <= MAX_E && s.top_k <= MAX_K &&
           bread_standard_qtypes(L) &&
           (((uintptr_t)L->down_exps | (uintptr_t)L->down_shexp | L->down_expert_bytes) & 15) == 0;
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
    if (e == hipSuccess) e = hipMalloc((void **)&g.xq, (size_t)SW_MAX_T * XQ_TOKEN_BYTES);
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
    (void)hipFree(g.xq);
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
    // routing: fast logits with radii (route.hip), then the certificate, the
    // reference-order sums it asks for and the slots in one workgroup
    // (k_sb_route); beyond the certified path's limits, the reference's
    // order for every logit and the host's selection (k_sb_select)
    const bool mv4 = E <= 4 * WAVE;
    // the decode shape: every workgroup owns a slice of every slot
    // (k_sw_gateup / k_sw_down), on the activations in fixed point that
    // k_route_fast writes
    const bool cert = bread_route_certified_ok(c, T);
    const bool sw = cert && H == SW_H && I == SW_I && Ish == SW_I && K <= SW_K && T <= SW_MAX_T;
    if (cert) {
        float *radii = c->h;
        const int rc = bread_launch_route_fast(c, L, x, T, c->gsh, radii, sw ? g.xq : nullptr, st);
        if (rc) return rc;
        if (mv4)
            hipLaunchKernelGGL(k_sb_route<4>, dim3(1), dim3(RT_THREADS), 0, st, L->router, x, c->logits, radii, H, E,
                               K, T, c->idx, c->w, g.slot_expert, g.slot_cnt, g.slot_pair, g.n_slots,
                               c->dsync->rstat.v);
        else
            hipLaunchKernelGGL(k_sb_route<16>, dim3(1), dim3(RT_THREADS), 0, st, L->router, x, c->logits, radii, H,
                               E, K, T, c->idx, c->w, g.slot_expert, g.slot_cnt, g.slot_pair, g.n_slots,
                               c->dsync->rstat.v);
    } else {
        const int rc =
            bread_launch_route_logits(L->router, L->shexp_gate, x, c->logits, c->gsh, H, E, T, true, st);
        if (rc) return rc;
        if (mv4)
            hipLaunchKernelGGL(k_sb_select<4>, dim3(1), dim3(RT_THREADS), 0, st, c->logits, E, K, T, c->idx, c->w,
                               g.slot_expert, g.slot_cnt, g.slot_pair, g.n_slots);
        else
            hipLaunchKernelGGL(k_sb_select<16>, dim3(1), dim3(RT_THREADS), 0, st, c->logits, E, K, T, c->idx,
                               c->w, g.slot_expert, g.slot_cnt, g.slot_pair, g.n_slots);
    }
    BREAD_HIP(hipGetLastError());
    if (sw) {
        hipLaunchKernelGGL(k_sw_gateup, dim3(SW_G), dim3(SW_NT), 0, st, sl, g.xq, ss, c->h, E, K, T, S);
        const uint32_t spin = c->spin_limit >= 0 ? (uint32_t)c->spin_limit : SW_SPIN_DEFAULT;
        hipLaunchKernelGGL(k_sw_down, dim3(SW_G), dim3(SW_NT), 0, st, sl, c->h, ss, hidden, c->w, c->gsh, E, K, T,
                           S, &c->dsync->error.v, spin);
        BREAD_HIP(hipGetLastError());
        return BREAD_OK;
    }
    hipLaunchKernelGGL(k_sb_gateup, dim3(S, (Imax + GU_RG - 1) / GU_RG), dim3(256), 0, st, sl, x, ss, c->h, H, I,
                       Ish, E, K, T, Imax);
    hipLaunchKernelGGL(k_sb_down, dim3(S, (H + DN_RG - 1) / DN_RG), dim3(256), 0, st, sl, c->h, ss, g.eo, H, I, Ish,
                       E, K, T, Imax);
    hipLaunchKernelGGL(k_sb_combine, dim3(T, (H + 1023) / 1024), dim3(256), 0, st, hidden, g.eo, c->w, c->gsh, H,
                       K);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}
