// moe_grouped.hip — the multi-token MoE path (batched decode, speculative
// verify, prefill chunks): tokens bucketed by expert, the expert products as
// grouped GEMMs on the gfx950 matrix cores with the K-quant weights
// dequantised in registers, and a combine in the reference order.
//
// The reference has no multi-token MoE: prefill runs token by token
// (main.cu:615-639) and speculative verify is sequential
// (main_speculative.cu:477-497).  Per token the result is the MoE block of
// one_layer_forward (one_layer.cu:1800-1986; CPU form 1413-1471).
//
// Numerics.  MFMA operands are fp16 with fp32 accumulation.  A bf16 operand
// (8-bit significand) leaves about 4e-3 relative L2 error on one expert's
// output, above the 1e-3 bound of this path; fp16 weights (one rounding of
// the exact K-quant value) times activations carried as two fp16 terms
// (hi + lo, 22 significant bits) leave about 4e-4.  Before the split each
// activation row is scaled by a power of two so that its largest magnitude
// lies in [2^13, 2^14) (exact, undone on the fp32 result): SwiGLU outputs
// reach 1e5 at the synthetic weight scale, beyond fp16's range.
//
// Weight dequantisation, one instruction per weight: a byte holding a 4- or
// 6-bit code q becomes the fp16 value 1024 + q by byte permutation (0x64 in
// the high byte), and v_fma_mix{lo,hi}_f16 computes (1024 + q) * d + c in
// fp32 with c = -(1024 * d + m) and rounds once to fp16, giving d * q - m
// (Q4_K, dequant_q4k_cpu.c:117-118) or d * sc * (q - 32) (Q6_K, c = -1056 *
// d * sc, dequant_q4k_cpu.c:160-165).
//
// Expert GEMMs use v_mfma_f32_32x32x16_f16 with the weights as the M side
// (32 rows) and the M-tile's 32 (token, expert) pairs as the N side: each
// dequantised weight fragment meets 32 tokens in one instruction, and each
// activation fragment read from LDS serves 32 weight rows.
//
// Kernels per layer, stream-ordered:
//   k_route_seq   router logits in the reference's sequential order
//                 (route.hip: one lane a token, one or two router rows a wave)
//   k_mt_topk_xprep  one workgroup per token: softmax / top-k /
//                 renormalisation with the host's arithmetic (routing
//                 bit-identical to the reference's), and the activation
//                 preparation: row scale, hi/lo fp16 activations in the
//                 gate/up operand order, shared-gate logit
//   k_mt_bucket   one workgroup: expert histogram, token lists by expert,
//                 M-tiles of 32 pairs
//   k_mt_gateup   per (M-tile, 128 rows): gate and up GEMMs, SwiGLU
//   k_mt_down     per (M-tile, 512 rows): the tile's SwiGLU rows split into
//                 hi/lo fp16 with a row scale, then the down GEMM
//   k_mt_combine  per token: shared expert, then routed experts in rank order
// The shared expert is expert index E with every token, so both GEMMs treat
// it like a routed expert with its own weights.
#include <float.h>
#include <stdlib.h>

#include "bread_internal.h"
#include "bread_device.h"
#include "quant_dot.h"
#include "route_dev.h"

namespace {

constexpr int MT = 32;                           // (token, expert) pairs per M-tile
constexpr int GU_WAVES = 8;                      // one 32-row gate or up block per wave
constexpr int GU_ROWS = GU_WAVES / 2 * 32;       // SwiGLU rows per gate/up workgroup
constexpr int DN_WAVES = 8, DN_BLOCKS = 2;       // 32-row down blocks per wave
constexpr int DN_ROWS = DN_WAVES * DN_BLOCKS * 32;  // output rows per down workgroup
constexpr int MAX_INTER = 512;                   // largest intermediate size the LDS plan holds
constexpr int NXCD = 8;                          // L2 domains; workgroup L runs on XCD L % 8
constexpr int SEG = 4;                           // tiles of one expert kept on one XCD
constexpr uint32_t MAGIC = 0x64646464u;          // fp16 0x64xx = 1024 + xx

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct MtTile {
    int e;   // expert (E = the shared expert)
    int p0;  // first pair in the sorted pair list
    int nr;  // pairs in the tile (1..MT)
    int pad;
};

struct MtArgs {
    bread_moe_layer_t L;
    uint32_t *err;           // device error word of the context
    int H, I, Ish, Imax, E, K, T;
    const uint4 *xhi, *xlo;  // [T][H/8] units of 8 fp16, gate/up operand order
    const int *xexp;         // [T] row scale exponents
    const int *pair_tok;     // [T*K + T] token of each sorted pair
    const MtTile *tiles;
    const int *n_tiles;
    const int *work_gu, *work_dn;  // per-XCD work items (tile << 8 | chunk) of the two GEMMs
    const int *n_work;             // [2][NXCD] items per XCD (gate/up, down)
    int slots_gu, slots_dn;        // list capacity per XCD
    float *h;                // [T*K + T][Imax] SwiGLU outputs by pair
    float *eo;               // [T*K + T][H] expert outputs by pair
};

__device__ __forceinline__ void lds_load16(const void *src, void *lds_wave_base)
{
    __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, 0);
}

__device__ __forceinline__ uint32_t comp(const uint4 &q, int i)
{
    return i == 0 ? q.x : (i == 1 ? q.y : (i == 2 ? q.z : q.w));
}

// s_waitcnt with vmcnt <= n (n < 16) and the other counters unconstrained
// (gfx9 encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 16, "vmcnt");
    __builtin_amdgcn_s_waitcnt(N | (7 << 4) | (15 << 8));
}

// Exponent e with max_abs * 2^-e in [2^13, 2^14); 0 for an all-zero or
// non-finite row.
__device__ __forceinline__ int row_exp(float max_abs)
{
    int e = 0;
    if (max_abs > 0.f && max_abs <= FLT_MAX) {
        (void)frexpf(max_abs, &e);
        e -= 14;
    }
    return e;
}

// v (already scaled) as hi + lo fp16: hi = fp16(v), lo = fp16(v - hi).
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo)
{
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    const _Float16 la = (_Float16)(a - (float)ha), lb = (_Float16)(b - (float)hb);
    hi = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
    lo = (uint32_t)__builtin_bit_cast(uint16_t, la) | ((uint32_t)__builtin_bit_cast(uint16_t, lb) << 16);
}

__device__ __forceinline__ void split8(const float (&v)[8], int e, uint4 &hi, uint4 &lo)
{
    split2(ldexpf(v[0], -e), ldexpf(v[1], -e), hi.x, lo.x);
    split2(ldexpf(v[2], -e), ldexpf(v[3], -e), hi.y, lo.y);
    split2(ldexpf(v[4], -e), ldexpf(v[5], -e), hi.z, lo.z);
    split2(ldexpf(v[6], -e), ldexpf(v[7], -e), hi.w, lo.w);
}

// Two fp16 values (1024 + q0, 1024 + q1) -> fp16(fp32 (1024 + q) * d + c).
__device__ __forceinline__ uint32_t mix2(uint32_t q2, float d, float c)
{
    const half2v h = __builtin_bit_cast(half2v, q2);
    half2v r;
    r[0] = (_Float16)__builtin_fmaf((float)h[0], d, c);
    r[1] = (_Float16)__builtin_fmaf((float)h[1], d, c);
    return __builtin_bit_cast(uint32_t, r);
}

// Bytes b0..b3 of v (codes < 256) -> four fp16 weights in byte order,
// (b0, b1) in r0 and (b2, b3) in r1.
__device__ __forceinline__ void bytes_to_w(uint32_t v, float d, float c, uint32_t &r0, uint32_t &r1)
{
    r0 = mix2(__builtin_amdgcn_perm(MAGIC, v, 0x07010700u), d, c);
    r1 = mix2(__builtin_amdgcn_perm(MAGIC, v, 0x07030702u), d, c);
}

// D[32 weight rows][32 pairs] += W[32][16] * X[16][32].  Lane l holds W row
// l%32 and X column l%32, K elements 8*(l/32) .. +7 of the step; D register
// i holds row 8*(i/4) + 4*(l/32) + i%4 of column l%32.
__device__ __forceinline__ f32x16 mfma32(const uint4 &w, const uint4 &x, f32x16 acc)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, w), __builtin_bit_cast(half8, x), acc,
                                                  0, 0, 0);
}

// ---------------------------------------------------------------------------
// Gate/up operand order (Q4_K).  Lane (row r = lane%32, group g = lane/32) of
// a 32-row block reads qs bytes [64g, 64g+64) of each superblock row, i.e.
// sub-block pairs p = 2g and 2g+1.  K-step s (0..15) of a superblock uses qs
// dword s%8 of pair p = 2g + s/8: B element j of the lane is superblock
// element 64p + 4(s%8) + j (j < 4, low nibbles, sub-block 2p) or
// 64p + 32 + 4(s%8) + (j - 4) (j >= 4, high nibbles, sub-block 2p + 1).
// The activations are stored in the same order: unit u = 32*sb + 2*s + g of
// a token row holds those 8 elements.
// ---------------------------------------------------------------------------

// Packed-fp16 form of the same weights, two per instruction:
//   t = fma(1024 + q, sc, -1024 sc) = sc * q   (exact: |sc q| <= 945)
//   w = fma(t, d, fp16(-dmin * m))             (one rounding, as above, plus
//                                               the fp16 rounding of dmin * m)
// Valid while d * 945 and dmin * 63 stay inside fp16's range (|d| < 64,
// |dmin| < 1024), which fp16 weights need anyway; superblocks outside it
// raise BREAD_DEV_ERR_RANGE.
struct Q4Pk {
    half2v sc[4], nsc[4], m[4], d;
};

__device__ __forceinline__ Q4Pk q4k_lane_pk(const uint4 &hd, uint32_t g)
{
    Q4Pk s;
    const float dmin = h2f(hd.x >> 16);
    const _Float16 d16 = __builtin_bit_cast(_Float16, (uint16_t)(hd.x & 0xFFFFu));
    s.d = half2v{d16, d16};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        uint32_t sc, m;
        scale_min_k4(4 * g + q, hd.y, hd.z, hd.w, sc, m);
        const _Float16 scf = (_Float16)(float)sc, nscf = (_Float16)(-1024.f * (float)sc);
        const _Float16 mf = (_Float16)(-(dmin * (float)m));
        s.sc[q] = half2v{scf, scf};
        s.nsc[q] = half2v{nscf, nscf};
        s.m[q] = half2v{mf, mf};
    }
    return s;
}

__device__ __forceinline__ uint32_t pk_w(uint32_t qb, const Q4Pk &s, int q)
{
    const half2v t = __builtin_elementwise_fma(__builtin_bit_cast(half2v, qb), s.sc[q], s.nsc[q]);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(t, s.d, s.m[q]));
}

__device__ __forceinline__ bool q4k_pk_ok(const uint4 &hd)
{
    const float d = fabsf(h2f(hd.x)), dmin = fabsf(h2f(hd.x >> 16));
    return d < 64.f && dmin < 1024.f;  // false for NaN
}

// ---------------------------------------------------------------------------
// Down operand order (Q6_K).  Lane (row r, group g) of a 32-row block takes
// half g (elements 128g .. 128g+127) of each superblock row; K-step t (0..15)
// of the half covers its elements 8t .. 8t+7 (natural order): low nibbles
// of ql bytes 8t.. (t < 8) or high nibbles of ql bytes 8(t-8).. (t >= 8),
// with qh bits 2*(t/4) of qh bytes 8(t%4).. and scale sc[8g + t/2]
// (dequant_q4k_cpu.c:155-170).  Activation unit ((16b + t)*2 + g) of a row
// holds elements 256b + 128g + 8t .. +7.
//
// The lane's bytes are 2-byte aligned (superblocks are 210 bytes), so each
// range is loaded as whole dwords from the aligned-down address and shifted
// with v_alignbyte.  Every dword loaded holds a byte of the superblock or of
// the next one in the same expert block (an expert block ends 16-byte
// aligned, so a superblock starting at a multiple of 4 is never its last).
// ---------------------------------------------------------------------------

struct Q6Raw {
    uint4 ql[4];
    uint32_t ql4;
    uint4 qh[2];
    uint32_t qh2;
    uint4 sc;
    uint32_t sc1;
};

__device__ __forceinline__ void q6k_load(const uint8_t *sb, int g, Q6Raw &R)
{
    // aligned down by pointer arithmetic: a pointer rebuilt from an integer
    // is generic to the compiler, which would emit flat loads (counted on
    // lgkmcnt too, so every LDS wait would also wait for these)
    const uint8_t *p = sb - (reinterpret_cast<uintptr_t>(sb) & 3u);
    const uint8_t *ql = p + 64 * g, *qh = p + 128 + 32 * g, *sc = p + 192;
#pragma unroll
    for (int i = 0; i < 4; i++) R.ql[i] = *reinterpret_cast<const uint4 *>(ql + 16 * i);
    R.ql4 = *reinterpret_cast<const uint32_t *>(ql + 64);
    R.qh[0] = *reinterpret_cast<const uint4 *>(qh);
    R.qh[1] = *reinterpret_cast<const uint4 *>(qh + 16);
    R.qh2 = *reinterpret_cast<const uint32_t *>(qh + 32);
    R.sc = *reinterpret_cast<const uint4 *>(sc);
    R.sc1 = *reinterpret_cast<const uint32_t *>(sc + 16);
}

// ---------------------------------------------------------------------------
// Activation preparation and router
// ---------------------------------------------------------------------------

__device__ __forceinline__ void mt_xprep(int t, const float *__restrict__ x, const uint16_t *__restrict__ shg, int H,
                                         uint4 *__restrict__ xhi, uint4 *__restrict__ xlo, int *__restrict__ xexp,
                                         float *__restrict__ gsh)
{
    __shared__ float smax[4], sdot[4];
    const float *xt = x + (size_t)t * H;
    float mx = 0.f, dot = 0.f;
    for (int i = 4 * (int)threadIdx.x; i < H; i += 1024) {
        const float4 v = *reinterpret_cast<const float4 *>(xt + i);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        if (shg) {
            const uint2 g = *reinterpret_cast<const uint2 *>(shg + i);
            dot = fmaf(h2f(g.x), v.x, dot);
            dot = fmaf(h2f(g.x >> 16), v.y, dot);
            dot = fmaf(h2f(g.y), v.z, dot);
            dot = fmaf(h2f(g.y >> 16), v.w, dot);
        }
    }
    mx = wave_max(mx);
    dot = wave_sum(dot);
    if (lane_id() == 0) {
        smax[threadIdx.x / WAVE] = mx;
        sdot[threadIdx.x / WAVE] = dot;
    }
    __syncthreads();
    const int e = row_exp(fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3])));
    if (threadIdx.x == 0) {
        xexp[t] = e;
        if (gsh) gsh[t] = shg ? (sdot[0] + sdot[1]) + (sdot[2] + sdot[3]) : 0.f;
    }
    const int nu = H / 8;
    for (int u = threadIdx.x; u < nu; u += 256) {
        const int sb = u >> 5, s = (u >> 1) & 15, g = u & 1;
        const int b = QK * sb + 64 * (2 * g + (s >> 3)) + 4 * (s & 7);
        const float4 lo4 = *reinterpret_cast<const float4 *>(xt + b);
        const float4 hi4 = *reinterpret_cast<const float4 *>(xt + b + 32);
        const float v[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
        uint4 h, l;
        split8(v, e, h, l);
        xhi[(size_t)t * nu + u] = h;
        xlo[(size_t)t * nu + u] = l;
    }
}

// Per token, one workgroup: the activation preparation (row scale, hi/lo
// fp16 activations in the gate/up operand order, shared-gate logit) and, on
// wave 0, softmax / top-k / renormalisation with the host's arithmetic on
// the router logits (route_dev.h topk_wave_exact).
template <int MAXV>
__global__ __launch_bounds__(256) void k_mt_topk_xprep(const float *__restrict__ logits, int E, int K,
                                                       int32_t *__restrict__ idx, float *__restrict__ w,
                                                       const float *__restrict__ x, const uint16_t *__restrict__ shg,
                                                       int H, uint4 *__restrict__ xhi, uint4 *__restrict__ xlo,
                                                       int *__restrict__ xexp, float *__restrict__ gsh)
{
    __shared__ __attribute__((aligned(16))) float s_e[WAVE * MAXV];
    const int t = (int)blockIdx.x;
    if (wave_id() == 0) {
        int ik;
        float wk;
        topk_wave_exact<MAXV>(logits + (size_t)t * E, E, K, s_e, ik, wk);
        if (lane_id() < K) {
            idx[(size_t)t * K + lane_id()] = ik;
            w[(size_t)t * K + lane_id()] = wk;
        }
    }
    mt_xprep(t, x, shg, H, xhi, xlo, xexp, gsh);
}

// ---------------------------------------------------------------------------
// Bucketing
// ---------------------------------------------------------------------------

// Exclusive prefix sums of two per-thread values over the workgroup.
__device__ __forceinline__ void block_scan2(int a, int b, int *wsa, int *wsb, int &xa, int &xb, int &ta, int &tb)
{
    const int lane = lane_id(), w = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
    const int ia = wave_scan_incl(a), ib = wave_scan_incl(b);
    if (lane == WAVE - 1) {
        wsa[w] = ia;
        wsb[w] = ib;
    }
    __syncthreads();
    int pa = 0, pb = 0;
    ta = 0;
    tb = 0;
    for (int i = 0; i < nw; i++) {
        if (i < w) {
            pa += wsa[i];
            pb += wsb[i];
        }
        ta += wsa[i];
        tb += wsb[i];
    }
    xa = pa + ia - a;
    xb = pb + ib - b;
}

// Pairs (token t, rank k) sorted by expert; the shared expert's pairs
// (every token in order) follow at T*K.  pos_of[t*K + k] = sorted position
// (-1 for an index outside [0, E), which the combine skips).
__global__ __launch_bounds__(1024) void k_mt_bucket(const int32_t *__restrict__ idx, int T, int K, int E,
                                                    int *__restrict__ pair_tok, int *__restrict__ pos_of,
                                                    MtTile *__restrict__ tiles, int *__restrict__ n_tiles,
                                                    int *__restrict__ work_gu, int *__restrict__ work_dn,
                                                    int *__restrict__ n_work, int c_gu, int c_dn, int slots_gu,
                                                    int slots_dn)
{
    __shared__ int cnt[1024], base[1024], cur[1024];
    __shared__ int wsa[16], wsb[16];
    __shared__ int xfirst[NXCD + 1];
    const int tid = threadIdx.x;
    cnt[tid] = 0;
    cur[tid] = 0;
    __syncthreads();
    const int P = T * K;
    for (int p = tid; p < P; p += 1024) {
        const int e = idx[p];
        if ((unsigned)e < (unsigned)E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    const int c = tid < E ? cnt[tid] : 0;
    const int nt = (c + MT - 1) / MT;
    int xc, xt, tc, tt;
    block_scan2(c, nt, wsa, wsb, xc, xt, tc, tt);
    base[tid] = xc;
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = idx[p];
        int pos = -1;
        if ((unsigned)e < (unsigned)E) {
            pos = base[e] + atomicAdd(&cur[e], 1);
            pair_tok[pos] = p / K;
        }
        pos_of[p] = pos;
    }
    for (int i = 0; i < nt; i++) tiles[xt + i] = {tid, xc + i * MT, min(MT, c - i * MT), 0};
    const int nsh = (T + MT - 1) / MT;
    for (int i = tid; i < nsh; i += 1024) tiles[tt + i] = {E, P + i * MT, min(MT, T - i * MT), 0};
    for (int t = tid; t < T; t += 1024) pair_tok[P + t] = t;
    const int N = tt + nsh;
    if (tid == 0) *n_tiles = N;

    // Work lists.  Segments of at most SEG consecutive tiles of one expert
    // (the shared expert's after the routed ones) stay on one XCD, so the
    // expert's weights are fetched into that L2 once per segment instead of
    // once per tile, while a hot expert's segments still spread over the
    // XCDs.  The segment starting at tile s0 goes to XCD floor(8 s0 / N),
    // and XCD x holds tiles [A(x), A(x + 1)) with A(x) the first segment
    // start >= ceil(x N / 8).  Per XCD, items run segment by segment,
    // chunk-major: (tile s0 + i, chunk c) at (s0 - A(x)) C + c n + i.
    // A(x + 1) - A(x) <= ceil(N / 8) + SEG, which the host sizes the lists
    // for; writes beyond a list are dropped regardless.
    cnt[tid] = xt;  // each expert's first tile (the counts are used up)
    if (tid <= NXCD) xfirst[tid] = N;
    __syncthreads();
    auto xcd_of = [&](int start) { return min(NXCD - 1, (int)(((long long)start * NXCD) / N)); };
    // tile q's segment: start and length.  Below tt the expert is the last
    // one whose first tile is <= q (an empty expert shares its first tile
    // with the next, so that one is never empty).
    auto segment = [&](int q, int &start, int &len) {
        int first = tt, ntiles = nsh;
        if (q < tt) {
            int lo = 0, hi = E - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (cnt[mid] <= q) lo = mid;
                else hi = mid - 1;
            }
            first = cnt[lo];
            ntiles = (cur[lo] + MT - 1) / MT;
        }
        start = first + (q - first) / SEG * SEG;
        len = min(SEG, first + ntiles - start);
    };
    for (int q = tid; q < N; q += 1024) {
        int start, len;
        segment(q, start, len);
        if (q == start) atomicMin(&xfirst[xcd_of(q)], q);
    }
    __syncthreads();
    if (tid == 0)
        for (int x = NXCD - 1; x >= 0; x--) xfirst[x] = min(xfirst[x], xfirst[x + 1]);
    __syncthreads();
    for (int q = tid; q < N; q += 1024) {
        int start, len;
        segment(q, start, len);
        const int x = xcd_of(start), b = start - xfirst[x], i = q - start;
        for (int cc = 0; cc < c_gu; cc++) {
            const int j = b * c_gu + cc * len + i;
            if (j < slots_gu) work_gu[x * slots_gu + j] = (q << 8) | cc;
        }
        for (int cc = 0; cc < c_dn; cc++) {
            const int j = b * c_dn + cc * len + i;
            if (j < slots_dn) work_dn[x * slots_dn + j] = (q << 8) | cc;
        }
    }
    if (tid < NXCD) {
        const int nx = xfirst[tid + 1] - xfirst[tid];
        n_work[tid] = min(nx * c_gu, slots_gu);
        n_work[NXCD + tid] = min(nx * c_dn, slots_dn);
    }
}

// ---------------------------------------------------------------------------
// Gate/up: tile (M-tile, 128 rows).  Waves 0..3 own gate rows n0 + 32w +
// [0, 32), waves 4..7 the same rows of up, one 32-row block per wave.  The
// tile's 32 activation rows are staged per superblock (32 KB, hi and lo) in
// two LDS buffers by LDS-direct loads one superblock ahead; each wave loads
// its raw weight bytes one superblock ahead into registers and dequantises
// them there.  One barrier per superblock; two workgroups (16 waves) per CU.
// At the end the up waves pass their results through LDS to the gate waves
// (same lane layout), which apply the SwiGLU (layer_ops.cu:214-220).
// ---------------------------------------------------------------------------

// Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its
// own L2.  Workgroup L takes item L / 8 of XCD L % 8's list (k_mt_bucket);
// false when that list is shorter.
__device__ __forceinline__ bool xcd_item(const int *work, const int *n_work, int slots, int &tile, int &chunk)
{
    const int L = (int)blockIdx.x;
    const int x = L & (NXCD - 1), j = L / NXCD;
    if (j >= n_work[x]) return false;
    const int v = work[x * slots + j];
    tile = v >> 8;
    chunk = v & 255;
    return true;
}

__global__ __launch_bounds__(GU_WAVES * WAVE, 2) void k_mt_gateup(const MtArgs a)
{
    __shared__ uint4 sA[2][2][1024];  // [buffer][hi, lo][unit (s, g, n)]
    __shared__ int stok[MT], sexp[MT];
    int tile, chunk;
    if (!xcd_item(a.work_gu, a.n_work, a.slots_gu, tile, chunk) || tile >= *a.n_tiles) return;
    const MtTile tl = a.tiles[tile];
    const bool sh = tl.e == a.E;
    const int I = sh ? a.Ish : a.I;
    const int n0 = chunk * GU_ROWS;
    if (n0 >= I) return;
    const int tid = threadIdx.x, w = wave_id(), lane = lane_id();
    const bool up = w >= GU_WAVES / 2;
    const int wr = up ? w - GU_WAVES / 2 : w;
    const int g = lane >> 5, r = lane & 31;
    if (tid < MT) {
        const int tok = a.pair_tok[tl.p0 + min(tid, tl.nr - 1)];
        stok[tid] = tok;
        sexp[tid] = a.xexp[tok];
    }
    __syncthreads();

    const int HU = a.H / 8, nsb = a.H / QK;
    const uint64_t rb = (uint64_t)nsb * Q4K_BYTES;
    const uint8_t *base = up ? (sh ? (const uint8_t *)a.L.up_shexp
                                   : (const uint8_t *)a.L.up_exps + (uint64_t)tl.e * a.L.up_expert_bytes)
                             : (sh ? (const uint8_t *)a.L.gate_shexp
                                   : (const uint8_t *)a.L.gate_exps + (uint64_t)tl.e * a.L.gate_expert_bytes);
    const int row0 = n0 + 32 * wr;
    const uint8_t *wrow = base + (uint64_t)(row0 + r) * rb;
    // unit (s, g, n) of a buffer: lane (n = r, g) of wave w stages s = w + 8i
    const uint4 *ahi = a.xhi + (size_t)stok[r] * HU + 2 * w + g;
    const uint4 *alo = a.xlo + (size_t)stok[r] * HU + 2 * w + g;

    auto stage = [&](int sb, int st) {
#pragma unroll
        for (int i = 0; i < 16 / GU_WAVES; i++) {
            lds_load16(ahi + 32 * sb + 2 * GU_WAVES * i, &sA[st][0][64 * (w + GU_WAVES * i)]);
            lds_load16(alo + 32 * sb + 2 * GU_WAVES * i, &sA[st][1][64 * (w + GU_WAVES * i)]);
        }
    };
    auto load_b = [&](int sb, uint4 (&B)[5]) {
        const uint8_t *p = wrow + (uint64_t)sb * Q4K_BYTES;
        B[0] = ld_b128(p);
#pragma unroll
        for (int i = 0; i < 4; i++) B[1 + i] = ld_b128(p + 16 + 64 * g + 16 * i);
    };
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;
    // K-step s: activation fragments one step ahead of their MFMAs; the
    // weight fragment from qs dword s%8 of pair 2g + s/8
    auto ksteps = [&](int st, const uint4 (&B)[5], auto &&frag) {
        uint4 xa[2][2];
        xa[0][0] = sA[st][0][lane];
        xa[0][1] = sA[st][1][lane];
#pragma unroll
        for (int s = 0; s < 16; s++) {
            if (s + 1 < 16) {
                xa[(s + 1) & 1][0] = sA[st][0][64 * (s + 1) + lane];
                xa[(s + 1) & 1][1] = sA[st][1][64 * (s + 1) + lane];
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of this step's work
            const int pp = s >> 3, ds = s & 7;
            const uint4 bw = frag(comp(B[1 + 2 * pp + (ds >> 2)], ds & 3), 2 * pp);
            acc = mfma32(bw, xa[s & 1][0], acc);
            acc = mfma32(bw, xa[s & 1][1], acc);
        }
    };
    auto compute = [&](int st, const uint4 (&B)[5]) {
        if (__builtin_amdgcn_ballot_w64(!q4k_pk_ok(B[0])) != 0 && lane == 0)
            __hip_atomic_fetch_or(a.err, BREAD_DEV_ERR_RANGE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const Q4Pk pk = q4k_lane_pk(B[0], (uint32_t)g);
        ksteps(st, B, [&](uint32_t v, int q) {
            const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
            uint4 r;
            r.x = pk_w(__builtin_amdgcn_perm(MAGIC, lo, 0x07010700u), pk, q);
            r.y = pk_w(__builtin_amdgcn_perm(MAGIC, lo, 0x07030702u), pk, q);
            r.z = pk_w(__builtin_amdgcn_perm(MAGIC, hi, 0x07010700u), pk, q + 1);
            r.w = pk_w(__builtin_amdgcn_perm(MAGIC, hi, 0x07030702u), pk, q + 1);
            return r;
        });
    };

    // Iteration k: wait for weights and activations of k (issued in
    // iteration k-1), barrier (everyone is done with buffer (k+1)%2), issue
    // k+1, compute k.
    uint4 B0[5], B1[5];
    load_b(0, B0);
    stage(0, 0);
    for (int sb = 0; sb < nsb; sb += 2) {
        wait_vmcnt<0>();
        __syncthreads();
        if (sb + 1 < nsb) {
            load_b(sb + 1, B1);
            stage(sb + 1, 1);
        }
        compute(0, B0);
        if (sb + 1 >= nsb) break;
        wait_vmcnt<0>();
        __syncthreads();
        if (sb + 2 < nsb) {
            load_b(sb + 2, B0);
            stage(sb + 2, 0);
        }
        compute(1, B1);
    }

    const int e = sexp[r];
    float *xch = reinterpret_cast<float *>(&sA[0][0][0]);  // [wave 0..3][16][64] up results
    __syncthreads();
    if (up) {
#pragma unroll
        for (int i = 0; i < 16; i++) xch[(wr * 16 + i) * WAVE + lane] = ldexpf(acc[i], e);
    }
    __syncthreads();
    if (!up && r < tl.nr) {
        float *hp = a.h + (size_t)(tl.p0 + r) * a.Imax + row0 + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float4 o;
            o.x = silu_mul(ldexpf(acc[4 * j + 0], e), xch[(wr * 16 + 4 * j + 0) * WAVE + lane]);
            o.y = silu_mul(ldexpf(acc[4 * j + 1], e), xch[(wr * 16 + 4 * j + 1) * WAVE + lane]);
            o.z = silu_mul(ldexpf(acc[4 * j + 2], e), xch[(wr * 16 + 4 * j + 2) * WAVE + lane]);
            o.w = silu_mul(ldexpf(acc[4 * j + 3], e), xch[(wr * 16 + 4 * j + 3) * WAVE + lane]);
            *reinterpret_cast<float4 *>(hp + 8 * j) = o;
        }
    }
}

// ---------------------------------------------------------------------------
// Down: tile (M-tile, 512 output rows).  Wave w owns rows n0 + 64w + [0, 64)
// as two 32-row blocks.  The tile's fp32 SwiGLU rows are read once, scaled
// by a power of two per row and split into hi and lo fp16 parts in LDS (64 KB
// for I = 512); each wave walks its (block, superblock) items loading the next
// item's raw Q6_K bytes into registers while dequantising the current one.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(DN_WAVES * WAVE, 2) void k_mt_down(const MtArgs a)
{
    __shared__ uint4 sA[2][(MAX_INTER / 8) * MT];  // [hi, lo][unit ((16b + t)*2 + g)*32 + n]
    __shared__ int sexp[MT];
    int tile, chunk;
    if (!xcd_item(a.work_dn, a.n_work + NXCD, a.slots_dn, tile, chunk) || tile >= *a.n_tiles) return;
    const MtTile tl = a.tiles[tile];
    const bool sh = tl.e == a.E;
    const int I = sh ? a.Ish : a.I;
    const int n0 = chunk * DN_ROWS;
    const int w = wave_id(), lane = lane_id();
    const int g = lane >> 5, r = lane & 31;
    const int nb = I / QK;
    const uint64_t rbd = (uint64_t)nb * Q6K_BYTES;
    const uint8_t *db = sh ? (const uint8_t *)a.L.down_shexp
                           : (const uint8_t *)a.L.down_exps + (uint64_t)tl.e * a.L.down_expert_bytes;
    const int row0 = n0 + 32 * DN_BLOCKS * w;
    const int nblk = max(0, min(DN_BLOCKS, (a.H - row0) / 32));
    const int items = nblk * nb;
    auto item_ptr = [&](int it) {
        return db + (uint64_t)(row0 + 32 * (it / nb) + r) * rbd + (uint64_t)(it % nb) * Q6K_BYTES;
    };

    Q6Raw R0, R1;
    if (items > 0) q6k_load(item_ptr(0), g, R0);

    {
        // the tile's SwiGLU rows (fp32, by pair) scaled by a power of two per
        // row and split into hi/lo fp16 in LDS: element group v (8 floats)
        // of pair row p0 + n is LDS unit 64 (16 (v / 32) + v % 16) + 32 ((v /
        // 16) % 2) + n.  Wave w takes rows 4w .. 4w+3, 16 lanes a row, groups
        // gl + 16 k of the row.
        const int rw = 4 * w + (lane >> 4), gl = lane & 15;
        const int ng = I / 8;
        const float *hr = a.h + (size_t)(tl.p0 + min(rw, tl.nr - 1)) * a.Imax;
        float4 va[4], vb[4];
        float mx = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int v = gl + 16 * k;
            va[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            vb[k] = va[k];
            if (v < ng) {
                va[k] = *reinterpret_cast<const float4 *>(hr + 8 * v);
                vb[k] = *reinterpret_cast<const float4 *>(hr + 8 * v + 4);
            }
            mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(fabsf(va[k].x), fabsf(va[k].y)), fmaxf(fabsf(va[k].z), fabsf(va[k].w))),
                                 fmaxf(fmaxf(fabsf(vb[k].x), fabsf(vb[k].y)), fmaxf(fabsf(vb[k].z), fabsf(vb[k].w)))));
        }
        mx = fmaxf(mx, dpp_f<0xB1>(mx));   // the 16 lanes of the row
        mx = fmaxf(mx, dpp_f<0x4E>(mx));
        mx = fmaxf(mx, dpp_f<0x141>(mx));
        mx = fmaxf(mx, dpp_f<0x140>(mx));
        const int e = row_exp(mx);
        if (gl == 0) sexp[rw] = e;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int v = gl + 16 * k;
            if (v < ng) {
                const float x8[8] = {va[k].x, va[k].y, va[k].z, va[k].w, vb[k].x, vb[k].y, vb[k].z, vb[k].w};
                uint4 hi, lo;
                split8(x8, e, hi, lo);
                const int u = 64 * (16 * (v >> 5) + (v & 15)) + 32 * ((v >> 4) & 1) + rw;
                sA[0][u] = hi;
                sA[1][u] = lo;
            }
        }
    }
    __syncthreads();

    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;
    auto compute = [&](int it, const Q6Raw &R) {
        const uint32_t sh8 = (uint32_t)(reinterpret_cast<uintptr_t>(item_ptr(it)) & 3u);
        const uint32_t qw[17] = {R.ql[0].x, R.ql[0].y, R.ql[0].z, R.ql[0].w, R.ql[1].x, R.ql[1].y,
                                 R.ql[1].z, R.ql[1].w, R.ql[2].x, R.ql[2].y, R.ql[2].z, R.ql[2].w,
                                 R.ql[3].x, R.ql[3].y, R.ql[3].z, R.ql[3].w, R.ql4};
        const uint32_t hw[9] = {R.qh[0].x, R.qh[0].y, R.qh[0].z, R.qh[0].w, R.qh[1].x,
                                R.qh[1].y, R.qh[1].z, R.qh[1].w, R.qh2};
        // sc[8g .. 8g+3] and sc[8g+4 .. 8g+7]; g is per lane, so the words
        // are picked by selects rather than by an indexed array
        const uint32_t w0 = g ? R.sc.z : R.sc.x, w1 = g ? R.sc.w : R.sc.y, w2 = g ? R.sc1 : R.sc.z;
        const uint32_t s0 = __builtin_amdgcn_alignbyte(w1, w0, sh8);
        const uint32_t s1 = __builtin_amdgcn_alignbyte(w2, w1, sh8);
        const float d = h2f(R.sc1 >> (8 * sh8));
        const int b = it % nb;
        bool bad = false;  // |d sc| * 32 beyond fp16's range
        // K-steps t and t + 8 use the same ql bytes (low and high nibbles)
        // and the same qh bytes (bits 2(t/4) and 2(t/4) + 4)
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t l0 = __builtin_amdgcn_alignbyte(qw[2 * t + 1], qw[2 * t], sh8);
            const uint32_t l1 = __builtin_amdgcn_alignbyte(qw[2 * t + 2], qw[2 * t + 1], sh8);
            const uint32_t h0 = __builtin_amdgcn_alignbyte(hw[2 * (t & 3) + 1], hw[2 * (t & 3)], sh8);
            const uint32_t h1 = __builtin_amdgcn_alignbyte(hw[2 * (t & 3) + 2], hw[2 * (t & 3) + 1], sh8);
#pragma unroll
            for (int hi = 0; hi < 2; hi++) {
                const int tt = t + 8 * hi;
                const int hs = 2 * (tt >> 2);
                const uint32_t scw = hi ? s1 : s0;
                const float ds = d * (float)(int8_t)byte_of(scw, (uint32_t)((t >> 1) & 3));
                const float c = -1056.f * ds;
                bad |= !(fabsf(ds) < 2047.f);
                const uint32_t n0v = (hi ? l0 >> 4 : l0) & 0x0F0F0F0Fu;
                const uint32_t n1v = (hi ? l1 >> 4 : l1) & 0x0F0F0F0Fu;
                const uint32_t q0 = n0v | (((h0 >> hs) & 0x03030303u) << 4);
                const uint32_t q1 = n1v | (((h1 >> hs) & 0x03030303u) << 4);
                uint4 bw;
                bytes_to_w(q0, ds, c, bw.x, bw.y);
                bytes_to_w(q1, ds, c, bw.z, bw.w);
                const int unit = (16 * b + tt) * 64 + lane;
                acc = mfma32(bw, sA[0][unit], acc);
                acc = mfma32(bw, sA[1][unit], acc);
            }
        }
        if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0)
            __hip_atomic_fetch_or(a.err, BREAD_DEV_ERR_RANGE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (b == nb - 1) {
            if (r < tl.nr) {
                const int e = sexp[r];
                float *op = a.eo + (size_t)(tl.p0 + r) * a.H + row0 + 32 * (it / nb) + 4 * g;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float4 o;
                    o.x = ldexpf(acc[4 * j + 0], e);
                    o.y = ldexpf(acc[4 * j + 1], e);
                    o.z = ldexpf(acc[4 * j + 2], e);
                    o.w = ldexpf(acc[4 * j + 3], e);
                    *reinterpret_cast<float4 *>(op + 8 * j) = o;
                }
            }
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i] = 0.f;
        }
    };

    for (int it = 0; it < items; it += 2) {
        if (it + 1 < items) q6k_load(item_ptr(it + 1), g, R1);
        compute(it, R0);
        if (it + 1 >= items) break;
        if (it + 2 < items) q6k_load(item_ptr(it + 2), g, R0);
        compute(it + 1, R1);
    }
}

// hidden[t] += sigmoid(gsh[t]) * shared(t), then += w_k * expert_k(t) for
// k = 0..K-1 (one_layer.cu:1447-1449, 1469), one float4 per thread;
// blockIdx.x = token, blockIdx.y = 1024-column chunk.
__global__ __launch_bounds__(256) void k_mt_combine(const float *__restrict__ eo, const int *__restrict__ pos_of,
                                                    const float *__restrict__ w, const float *__restrict__ gsh,
                                                    float *__restrict__ hidden, int H, int K, int T)
{
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    const int c = 4 * (blockIdx.y * blockDim.x + threadIdx.x);
    if (c >= H) return;
    float4 acc = *reinterpret_cast<const float4 *>(hidden + (size_t)t * H + c);
    const float sg = sigmoidf_ref(gsh[t]);
    const float4 s = *reinterpret_cast<const float4 *>(eo + ((size_t)T * K + t) * H + c);
    acc.x = acc.x + sg * s.x;
    acc.y = acc.y + sg * s.y;
    acc.z = acc.z + sg * s.z;
    acc.w = acc.w + sg * s.w;
#pragma unroll 8
    for (int k = 0; k < K; k++) {
        const int p = pos_of[t * K + k];
        if (p < 0) continue;
        const float wk = w[t * K + k];
        const float4 v = *reinterpret_cast<const float4 *>(eo + (size_t)p * H + c);
        acc.x = acc.x + wk * v.x;
        acc.y = acc.y + wk * v.y;
        acc.z = acc.z + wk * v.z;
        acc.w = acc.w + wk * v.w;
    }
    *reinterpret_cast<float4 *>(hidden + (size_t)t * H + c) = acc;
}

int max_tiles(const bread_moe_shape_t &s, int T)
{
    const int P = T * s.top_k;
    return P / MT + (P < s.n_experts ? P : s.n_experts) + (T + MT - 1) / MT;
}

// Tiles one XCD's list can hold: an eighth of the tiles plus one segment.
int xcd_tiles(const bread_moe_shape_t &s, int T)
{
    return (max_tiles(s, T) + NXCD - 1) / NXCD + SEG;
}

int chunks_gu(const bread_moe_shape_t &s)
{
    const int Imax = s.expert_inter > s.shared_inter ? s.expert_inter : s.shared_inter;
    return (Imax + GU_ROWS - 1) / GU_ROWS;
}

int chunks_dn(const bread_moe_shape_t &s)
{
    return (s.hidden + DN_ROWS - 1) / DN_ROWS;
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

int bread_grouped_alloc(bread_moe_ctx_t *c)
{
    const bread_moe_shape_t &s = c->shape;
    const size_t T = (size_t)c->max_tokens, K = (size_t)s.top_k, H = (size_t)s.hidden;
    const size_t P = T * (K + 1);
    hipError_t e = hipSuccess;
    bread_grouped_ws &g = c->gws;
    if (e == hipSuccess) e = hipMalloc(&g.xhi, T * H * 2);
    if (e == hipSuccess) e = hipMalloc(&g.xlo, T * H * 2);
    if (e == hipSuccess) e = hipMalloc((void **)&g.xexp, T * sizeof(int));
    if (e == hipSuccess) e = hipMalloc((void **)&g.pair_tok, P * sizeof(int));
    if (e == hipSuccess) e = hipMalloc((void **)&g.pos_of, T * K * sizeof(int));
    if (e == hipSuccess) e = hipMalloc(&g.tiles, (size_t)max_tiles(s, c->max_tokens) * sizeof(MtTile));
    if (e == hipSuccess) e = hipMalloc((void **)&g.n_tiles, sizeof(int));
    const size_t xt = (size_t)xcd_tiles(s, c->max_tokens);
    if (e == hipSuccess) e = hipMalloc((void **)&g.work, NXCD * xt * (chunks_gu(s) + chunks_dn(s)) * sizeof(int));
    if (e == hipSuccess) e = hipMalloc((void **)&g.n_work, 2 * NXCD * sizeof(int));
    if (e == hipSuccess) e = hipMalloc((void **)&g.eo, P * H * sizeof(float));
    return e == hipSuccess ? BREAD_OK : (e == hipErrorOutOfMemory ? BREAD_ERR_NOMEM : BREAD_ERR_HIP);
}

void bread_grouped_free(bread_moe_ctx_t *c)
{
    bread_grouped_ws &g = c->gws;
    (void)hipFree(g.xhi);
    (void)hipFree(g.xlo);
    (void)hipFree(g.xexp);
    (void)hipFree(g.pair_tok);
    (void)hipFree(g.pos_of);
    (void)hipFree(g.tiles);
    (void)hipFree(g.n_tiles);
    (void)hipFree(g.work);
    (void)hipFree(g.n_work);
    (void)hipFree(g.eo);
    g = bread_grouped_ws{};
}

bool bread_grouped_supported(const bread_moe_shape_t &s, const bread_moe_layer_t *L)
{
    if (s.expert_inter > MAX_INTER || s.shared_inter > MAX_INTER || !bread_standard_qtypes(L)) return false;
    // Q6_K expert blocks must end 16-byte aligned (see the down operand order)
    const uintptr_t a16 = (uintptr_t)L->down_exps | (uintptr_t)L->down_shexp | L->down_expert_bytes;
    return (a16 & 15) == 0;
}

int bread_launch_moe_grouped(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, float *hidden, int T,
                             hipStream_t st)
{
    const bread_moe_shape_t &s = c->shape;
    if (!bread_grouped_supported(s, L)) return BREAD_ERR_SHAPE;
    BREAD_REQUIRE(((uintptr_t)hidden & 15) == 0, BREAD_ERR_ALIGN, "hidden must be 16-byte aligned");
    const int H = s.hidden, E = s.n_experts, K = s.top_k;
    const int Imax = s.expert_inter > s.shared_inter ? s.expert_inter : s.shared_inter;
    bread_grouped_ws &g = c->gws;
    bread_clear_stale_error();
    // router logits in the reference's order (route.hip), then per token the
    // exact softmax / top-k with the activation preparation
    {
        const int rc = bread_launch_route_logits((const float *)L->router, nullptr, x, c->logits, nullptr, H, E, T,
                                                 false, st);
        if (rc) return rc;
    }
    if ((E + WAVE - 1) / WAVE <= 4)
        hipLaunchKernelGGL(k_mt_topk_xprep<4>, dim3(T), dim3(256), 0, st, c->logits, E, K, c->idx, c->w, x,
                           (const uint16_t *)L->shexp_gate, H, (uint4 *)g.xhi, (uint4 *)g.xlo, g.xexp, c->gsh);
    else
        hipLaunchKernelGGL(k_mt_topk_xprep<16>, dim3(T), dim3(256), 0, st, c->logits, E, K, c->idx, c->w, x,
                           (const uint16_t *)L->shexp_gate, H, (uint4 *)g.xhi, (uint4 *)g.xlo, g.xexp, c->gsh);
    BREAD_HIP(hipGetLastError());
    const int cgu = chunks_gu(s), cdn = chunks_dn(s);
    const int slots_gu = xcd_tiles(s, T) * cgu, slots_dn = xcd_tiles(s, T) * cdn;
    int *work_gu = g.work, *work_dn = g.work + (size_t)NXCD * slots_gu;
    hipLaunchKernelGGL(k_mt_bucket, dim3(1), dim3(1024), 0, st, c->idx, T, K, E, g.pair_tok, g.pos_of,
                       (MtTile *)g.tiles, g.n_tiles, work_gu, work_dn, g.n_work, cgu, cdn, slots_gu, slots_dn);
    BREAD_HIP(hipGetLastError());
    MtArgs a;
    a.L = *L;
    a.err = &c->dsync->error.v;
    a.H = H;
    a.I = s.expert_inter;
    a.Ish = s.shared_inter;
    a.Imax = Imax;
    a.E = E;
    a.K = K;
    a.T = T;
    a.xhi = (const uint4 *)g.xhi;
    a.xlo = (const uint4 *)g.xlo;
    a.xexp = g.xexp;
    a.pair_tok = g.pair_tok;
    a.tiles = (const MtTile *)g.tiles;
    a.n_tiles = g.n_tiles;
    a.work_gu = work_gu;
    a.work_dn = work_dn;
    a.n_work = g.n_work;
    a.slots_gu = slots_gu;
    a.slots_dn = slots_dn;
    a.h = c->h;
    a.eo = g.eo;
    hipLaunchKernelGGL(k_mt_gateup, dim3(NXCD * slots_gu), dim3(GU_WAVES * WAVE), 0, st, a);
    BREAD_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_mt_down, dim3(NXCD * slots_dn), dim3(DN_WAVES * WAVE), 0, st, a);
    BREAD_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_mt_combine, dim3(T, (H / 4 + 255) / 256), dim3(256), 0, st, g.eo, g.pos_of, c->w, c->gsh,
                       hidden, H, K, T);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}
