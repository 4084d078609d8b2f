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
// Kernels per layer, stream-ordered:
//   k_mt_xprep    one workgroup per token: row scale, hi/lo fp16 activations
//                 in the gate/up operand order, shared-gate logit
//   k_mt_router   router logits on fp32 MFMA (16 tokens x 16 experts per
//                 workgroup, K split over 4 waves)
//   k_topk        softmax / top-k / renormalisation (moe.hip, route_dev.h)
//   k_mt_bucket   one workgroup: expert histogram, token lists by expert,
//                 M-tiles of 16 (token, expert) pairs
//   k_mt_gateup   per (M-tile, 128 rows): gate and up GEMMs, SwiGLU
//   k_mt_down     per (M-tile, 256 rows): down GEMM
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

constexpr int MT = 16;                           // (token, expert) pairs per M-tile
constexpr int GU_WAVES = 4, GU_CB = 2;           // 16-row column blocks of gate (and up) per wave
constexpr int GU_ROWS = GU_WAVES * GU_CB * 16;   // gate rows per gate/up workgroup
constexpr int DN_WAVES = 8, DN_CB = 2;
constexpr int DN_ROWS = DN_WAVES * DN_CB * 16;   // output rows per down workgroup
constexpr int MAX_INTER = 512;                   // largest intermediate size the LDS plan holds
constexpr int DN_BAND = 16 * (MAX_INTER / QK) * Q6K_BYTES;  // bytes of 16 down rows
constexpr uint32_t MAGIC = 0x64646464u;          // fp16 0x64xx = 1024 + xx

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MtTile {
    int e;   // expert (E = the shared expert)
    int p0;  // first pair in the sorted pair list
    int nr;  // pairs in the tile (1..MT)
    int pad;
};

struct MtArgs {
    bread_moe_layer_t L;
    int H, I, Ish, Imax, E, K, T;
    const uint4 *xhi, *xlo;  // [T][H/8] units of 8 fp16, gate/up operand order
    const int *xexp;         // [T] row scale exponents
    const int *pair_tok;     // [T*K + T] token of each sorted pair
    const MtTile *tiles;
    const int *n_tiles;
    float *hbuf;             // [T*K + T][Imax] SwiGLU outputs by pair
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

__device__ __forceinline__ f32x4 mfma16(const uint4 &a, const uint4 &b, f32x4 acc)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), acc,
                                                  0, 0, 0);
}

// ---------------------------------------------------------------------------
// Gate/up operand order (Q4_K).  Lane group g = lane/16 of a 16-row column
// block reads qs bytes [32g, 32g+32) of each superblock row, i.e. sub-blocks
// 2g (low nibbles) and 2g+1 (high nibbles).  K-step s (0..7) of a superblock
// uses qs dword s of that range: B element j of the lane is superblock
// element 64g + 4s + j (j < 4) or 64g + 32 + 4s + (j - 4) (j >= 4).  The
// activations are stored in the same order: unit u = 32*sb + 4*s + g of a
// token row holds those 8 elements.
// ---------------------------------------------------------------------------

struct Q4Sc {
    float da, ca, db, cb;
};

__device__ __forceinline__ Q4Sc q4k_lane_scales(const uint4 &hd, uint32_t g)
{
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * g, hd.y, hd.z, hd.w, sc0, m0);
    scale_min_k4(2 * g + 1, hd.y, hd.z, hd.w, sc1, m1);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    Q4Sc s;
    s.da = d * (float)sc0;
    s.ca = fmaf(-1024.f, s.da, -(dmin * (float)m0));
    s.db = d * (float)sc1;
    s.cb = fmaf(-1024.f, s.db, -(dmin * (float)m1));
    return s;
}

__device__ __forceinline__ uint4 q4k_frag(uint32_t v, const Q4Sc &s)
{
    uint4 r;
    bytes_to_w(v & 0x0F0F0F0Fu, s.da, s.ca, r.x, r.y);
    bytes_to_w((v >> 4) & 0x0F0F0F0Fu, s.db, s.cb, r.z, r.w);
    return r;
}

// ---------------------------------------------------------------------------
// Activation preparation and router
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_mt_xprep(const float *__restrict__ x, const uint16_t *__restrict__ shg,
                                                  int H, uint4 *__restrict__ xhi, uint4 *__restrict__ xlo,
                                                  int *__restrict__ xexp, float *__restrict__ gsh)
{
    __shared__ float smax[4], sdot[4];
    const int t = blockIdx.x;
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
        gsh[t] = shg ? (sdot[0] + sdot[1]) + (sdot[2] + sdot[3]) : 0.f;
    }
    const int nu = H / 8;
    for (int u = threadIdx.x; u < nu; u += 256) {
        const int sb = u >> 5, s = (u >> 2) & 7, g = u & 3;
        const int b = QK * sb + 64 * g + 4 * s;
        const float4 lo4 = *reinterpret_cast<const float4 *>(xt + b);
        const float4 hi4 = *reinterpret_cast<const float4 *>(xt + b + 32);
        const float v[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
        uint4 h, l;
        split8(v, e, h, l);
        xhi[(size_t)t * nu + u] = h;
        xlo[(size_t)t * nu + u] = l;
    }
}

// logits[t][e] = router row e . x[t] (one_layer.cu:964-971), fp32 products
// and sums.  Wave w covers K range [w*H/4, (w+1)*H/4); lane (r, g) feeds
// token t0 + r and expert e0 + r, 4 consecutive K each step.
__global__ __launch_bounds__(256) void k_mt_router(const float *__restrict__ router, const float *__restrict__ x,
                                                   float *__restrict__ logits, int H, int E, int T)
{
    __shared__ f32x4 part[3][WAVE];
    const int w = wave_id(), lane = lane_id();
    const int r = lane & 15, g = lane >> 4;
    const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
    const float *xr = x + (size_t)min(t0 + r, T - 1) * H;
    const float *wr = router + (size_t)min(e0 + r, E - 1) * H;
    const int kq = H / 4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k = w * kq + 4 * g; k < (w + 1) * kq; k += 16) {
        const float4 a = *reinterpret_cast<const float4 *>(xr + k);
        const float4 b = *reinterpret_cast<const float4 *>(wr + k);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
    }
    if (w > 0) part[w - 1][lane] = acc;
    __syncthreads();
    if (w != 0) return;
    const f32x4 s = ((acc + part[0][lane]) + part[1][lane]) + part[2][lane];
    const int e = e0 + r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = t0 + 4 * g + i;
        if (t < T && e < E) logits[(size_t)t * E + e] = s[i];
    }
}

// ---------------------------------------------------------------------------
// Bucketing
// ---------------------------------------------------------------------------

// Exclusive prefix sums of two per-thread values over the workgroup.
__device__ __forceinline__ void block_scan2(int a, int b, int *wsa, int *wsb, int &xa, int &xb, int &ta, int &tb)
{
    const int lane = lane_id(), w = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
    int ia = a, ib = b;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const int oa = __shfl_up(ia, d), ob = __shfl_up(ib, d);
        if (lane >= d) {
            ia += oa;
            ib += ob;
        }
    }
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
                                                    MtTile *__restrict__ tiles, int *__restrict__ n_tiles)
{
    __shared__ int cnt[1024], base[1024], cur[1024];
    __shared__ int wsa[16], wsb[16];
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
    if (tid == 0) *n_tiles = tt + nsh;
}

// ---------------------------------------------------------------------------
// Gate/up: tile (M-tile, 128 gate rows).  Wave w owns gate and up rows
// n0 + 32w + [0, 32) as two 16-row column blocks each; the tile's 16
// activation rows are staged per superblock in LDS (LDS-direct loads,
// double-buffered) and shared by the 4 waves; each wave dequantises its own
// weights in registers, prefetching the next superblock.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256, 2) void k_mt_gateup(const MtArgs a)
{
    __shared__ uint4 sA[2][2][512];  // [buffer][hi, lo][unit (s, g, m)]
    __shared__ int stok[MT], sexp[MT];
    const int tile = blockIdx.x;
    if (tile >= *a.n_tiles) return;
    const MtTile tl = a.tiles[tile];
    const bool sh = tl.e == a.E;
    const int I = sh ? a.Ish : a.I;
    const int n0 = blockIdx.y * GU_ROWS;
    if (n0 >= I) return;
    const int tid = threadIdx.x, w = wave_id(), lane = lane_id();
    const int g = lane >> 4, n = lane & 15;
    if (tid < MT) {
        const int tok = a.pair_tok[tl.p0 + min(tid, tl.nr - 1)];
        stok[tid] = tok;
        sexp[tid] = a.xexp[tok];
    }
    __syncthreads();

    const int HU = a.H / 8, nsb = a.H / QK;
    const uint64_t rb = (uint64_t)nsb * Q4K_BYTES;
    const uint8_t *gb = sh ? (const uint8_t *)a.L.gate_shexp
                           : (const uint8_t *)a.L.gate_exps + (uint64_t)tl.e * a.L.gate_expert_bytes;
    const uint8_t *ub = sh ? (const uint8_t *)a.L.up_shexp
                           : (const uint8_t *)a.L.up_exps + (uint64_t)tl.e * a.L.up_expert_bytes;
    const uint8_t *rows[4];  // gate block 0, gate block 1, up block 0, up block 1
#pragma unroll
    for (int c = 0; c < 4; c++)
        rows[c] = (c < 2 ? gb : ub) + (uint64_t)(n0 + 16 * (GU_CB * w + (c & 1)) + n) * rb;
    const uint4 *ahi = a.xhi + (size_t)stok[n] * HU + 4 * w + g;
    const uint4 *alo = a.xlo + (size_t)stok[n] * HU + 4 * w + g;

    // unit (s, g, m) of buffer: lane (m = n, g) of wave w loads s = w and w + 4
    auto stage = [&](int sb, int buf) {
        lds_load16(ahi + 32 * sb, &sA[buf][0][64 * w]);
        lds_load16(ahi + 32 * sb + 16, &sA[buf][0][64 * w + 256]);
        lds_load16(alo + 32 * sb, &sA[buf][1][64 * w]);
        lds_load16(alo + 32 * sb + 16, &sA[buf][1][64 * w + 256]);
    };
    auto load_b = [&](int sb, uint4 (&B)[4][3]) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint8_t *p = rows[c] + (uint64_t)sb * Q4K_BYTES;
            B[c][0] = ld_b128(p);
            B[c][1] = ld_b128(p + 16 + 32 * g);
            B[c][2] = ld_b128(p + 32 + 32 * g);
        }
    };
    f32x4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf, const uint4 (&B)[4][3]) {
        Q4Sc sc[4];
#pragma unroll
        for (int c = 0; c < 4; c++) sc[c] = q4k_lane_scales(B[c][0], (uint32_t)g);
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const uint4 xh = sA[buf][0][(4 * s + g) * 16 + n];
            const uint4 xl = sA[buf][1][(4 * s + g) * 16 + n];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint4 bw = q4k_frag(comp(B[c][1 + (s >> 2)], s & 3), sc[c]);
                acc[c] = mfma16(xh, bw, acc[c]);
                acc[c] = mfma16(xl, bw, acc[c]);
            }
        }
    };

    uint4 B0[4][3], B1[4][3];
    stage(0, 0);
    load_b(0, B0);
    for (int sb = 0; sb < nsb; sb += 2) {
        // superblock sb from buffer 0 / B0
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (sb + 1 < nsb) {
            stage(sb + 1, 1);
            load_b(sb + 1, B1);
        }
        compute(0, B0);
        if (sb + 1 >= nsb) break;
        // superblock sb + 1 from buffer 1 / B1
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (sb + 2 < nsb) {
            stage(sb + 2, 0);
            load_b(sb + 2, B0);
        }
        compute(1, B1);
    }

    float *hrow = a.hbuf + n0 + 16 * GU_CB * w + n;
#pragma unroll
    for (int cb = 0; cb < GU_CB; cb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * g + i;
            if (m < tl.nr) {
                const float gv = ldexpf(acc[cb][i], sexp[m]);
                const float uv = ldexpf(acc[2 + cb][i], sexp[m]);
                hrow[(size_t)(tl.p0 + m) * a.Imax + 16 * cb] = silu_mul(gv, uv);
            }
        }
}

// ---------------------------------------------------------------------------
// Down: tile (M-tile, 256 output rows).  Wave w owns rows n0 + 32w + [0, 32)
// as two 16-row column blocks, each a contiguous band of the expert's Q6_K
// rows staged in LDS (16-byte aligned: 16 rows are 16 * 210 * I/256 bytes);
// the tile's SwiGLU rows are scaled, split and staged once for all waves.
// Operand order: K-step s covers elements [32s, 32s + 32) and lane group g
// elements 32s + 8g + [0, 8) (natural order), from the ql/qh bytes of
// quant_dot.h's Q6_K lane unit.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(512, 1) void k_mt_down(const MtArgs a)
{
    __shared__ uint4 sA[2][(MAX_INTER / 32) * 64];   // [hi, lo][unit (s, g, m)]
    __shared__ uint32_t sB[DN_WAVES][DN_CB][DN_BAND / 4];
    __shared__ int sexp[MT];
    const int tile = blockIdx.x;
    if (tile >= *a.n_tiles) return;
    const MtTile tl = a.tiles[tile];
    const bool sh = tl.e == a.E;
    const int I = sh ? a.Ish : a.I;
    const int n0 = blockIdx.y * DN_ROWS;
    const int tid = threadIdx.x, w = wave_id(), lane = lane_id();
    const int rbd = (I / QK) * Q6K_BYTES;
    const uint8_t *db = sh ? (const uint8_t *)a.L.down_shexp
                           : (const uint8_t *)a.L.down_exps + (uint64_t)tl.e * a.L.down_expert_bytes;

    // weight bands first, so they load while the activations are prepared
#pragma unroll
    for (int cb = 0; cb < DN_CB; cb++) {
        const uint8_t *band = db + (uint64_t)(n0 + 16 * (DN_CB * w + cb)) * rbd;
        for (int k = 0; k < rbd; k += WAVE)
            if (k + lane < rbd) lds_load16(band + 16 * (k + lane), &sB[w][cb][4 * k]);
    }

    {
        const int m = tid >> 5, seg = tid & 31;
        const float *hr = a.hbuf + (size_t)(tl.p0 + min(m, tl.nr - 1)) * a.Imax;
        const int per = I / 32;
        float mx = 0.f;
        for (int j = 0; j < per; j += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(hr + seg * per + j);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const int e = row_exp(mx);
        if (seg == 0) sexp[m] = e;
        for (int j = 0; j < per; j += 8) {
            const int k0 = seg * per + j;
            const float4 p = *reinterpret_cast<const float4 *>(hr + k0);
            const float4 q = *reinterpret_cast<const float4 *>(hr + k0 + 4);
            const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
            uint4 h, l;
            split8(v, e, h, l);
            const int unit = ((k0 >> 5) * 4 + ((k0 >> 3) & 3)) * 16 + m;
            sA[0][unit] = h;
            sA[1][unit] = l;
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    const int g = lane >> 4, n = lane & 15;
    const uint32_t i2 = (uint32_t)g >> 1;
#pragma unroll
    for (int cb = 0; cb < DN_CB; cb++) {
        const uint32_t *band = sB[w][cb];
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int b = 0; b < I / QK; b++) {
            const uint32_t o = (uint32_t)(n * rbd + b * Q6K_BYTES);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint2 ql0 = lds8_a2(band, o + 64 * h + 8 * g);
                const uint2 ql1 = lds8_a2(band, o + 64 * h + 32 + 8 * g);
                const uint2 qh = lds8_a2(band, o + 128 + 32 * h + 8 * g);
                const uint2 scw = lds8_a2(band, o + 192 + 8 * h);
                const float d = h2f(lds16_a2(band, o + 208));
                uint32_t qa[4], qb[4];
                q6k_unpack(ql0.x, ql1.x, qh.x, qa);
                q6k_unpack(ql0.y, ql1.y, qh.y, qb);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float ds = d * q6k_scale(scw, i2 + 2 * t);
                    const float c = -1056.f * ds;
                    uint4 bw;
                    bytes_to_w(qa[t], ds, c, bw.x, bw.y);
                    bytes_to_w(qb[t], ds, c, bw.z, bw.w);
                    const int s = 8 * b + 4 * h + t;
                    acc = mfma16(sA[0][(4 * s + g) * 16 + n], bw, acc);
                    acc = mfma16(sA[1][(4 * s + g) * 16 + n], bw, acc);
                }
            }
        }
        const int r = n0 + 16 * (DN_CB * w + cb) + n;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * g + i;
            if (m < tl.nr) a.eo[(size_t)(tl.p0 + m) * a.H + r] = ldexpf(acc[i], sexp[m]);
        }
    }
}

// hidden[t] += sigmoid(gsh[t]) * shared(t), then += w_k * expert_k(t) for
// k = 0..K-1 (one_layer.cu:1447-1449, 1469), one float4 per thread.
__global__ __launch_bounds__(256) void k_mt_combine(const float *__restrict__ eo, const int *__restrict__ pos_of,
                                                    const float *__restrict__ w, const float *__restrict__ gsh,
                                                    float *__restrict__ hidden, int H, int K, int T)
{
#pragma clang fp contract(off)
    const int h4 = H / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * h4) return;
    const int t = (int)(i / h4), c = (int)(i % h4) * 4;
    float4 acc = *reinterpret_cast<const float4 *>(hidden + (size_t)t * H + c);
    const float sg = sigmoidf_ref(gsh[t]);
    const float4 s = *reinterpret_cast<const float4 *>(eo + ((size_t)T * K + t) * H + c);
    acc.x = acc.x + sg * s.x;
    acc.y = acc.y + sg * s.y;
    acc.z = acc.z + sg * s.z;
    acc.w = acc.w + sg * s.w;
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
    (void)hipFree(g.eo);
    g = bread_grouped_ws{};
}

bool bread_grouped_supported(const bread_moe_shape_t &s, const bread_moe_layer_t *L)
{
    if (s.expert_inter > MAX_INTER || s.shared_inter > MAX_INTER) return false;
    // down bands are loaded 16 bytes a lane
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
    hipLaunchKernelGGL(k_mt_xprep, dim3(T), dim3(256), 0, st, x, (const uint16_t *)L->shexp_gate, H,
                       (uint4 *)g.xhi, (uint4 *)g.xlo, g.xexp, c->gsh);
    BREAD_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_mt_router, dim3((T + 15) / 16, (E + 15) / 16), dim3(256), 0, st, (const float *)L->router, x,
                       c->logits, H, E, T);
    BREAD_HIP(hipGetLastError());
    int rc = bread_launch_topk(c->logits, E, K, T, c->idx, c->w, st);
    if (rc) return rc;
    hipLaunchKernelGGL(k_mt_bucket, dim3(1), dim3(1024), 0, st, c->idx, T, K, E, g.pair_tok, g.pos_of,
                       (MtTile *)g.tiles, g.n_tiles);
    BREAD_HIP(hipGetLastError());
    MtArgs a;
    a.L = *L;
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
    a.hbuf = c->h;
    a.eo = g.eo;
    const int nt = max_tiles(s, T);
    hipLaunchKernelGGL(k_mt_gateup, dim3(nt, (Imax + GU_ROWS - 1) / GU_ROWS), dim3(GU_WAVES * WAVE), 0, st, a);
    BREAD_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_mt_down, dim3(nt, H / DN_ROWS), dim3(DN_WAVES * WAVE), 0, st, a);
    BREAD_HIP(hipGetLastError());
    const int64_t n4 = (int64_t)T * (H / 4);
    hipLaunchKernelGGL(k_mt_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, g.eo, g.pos_of, c->w,
                       c->gsh, hidden, H, K, T);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}
