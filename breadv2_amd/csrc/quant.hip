// quant.hip — standalone quantized matvec (bread_matvec, bread_matvec_f32)
// and the bit-exact dequant export (bread_dequant_rows) for gfx950.
//
// Matvec: one wave64 per row, grid-stride over rows; 8 lanes per superblock
// stream the row with 16-byte (Q4_K) or aligned-dword (Q6_K, Q8_0) loads,
// fp32 accumulate, DPP wave reduction.  Replaces kernels.cu:150-308, whose
// 256-thread blocks read one element per thread with two barriers per
// superblock.
#include <type_traits>

#include "bread_internal.h"
#include "quant_dot.h"

namespace {

template <typename T> __device__ __forceinline__ void store_y(T *y, int r, float v);
template <> __device__ __forceinline__ void store_y<float>(float *y, int r, float v) { y[r] = v; }
template <> __device__ __forceinline__ void store_y<uint16_t>(uint16_t *y, int r, float v)
{
    y[r] = f2h(v);
}

template <int QT, typename XT, typename YT>
__global__ __launch_bounds__(256) void k_matvec(const uint8_t *__restrict__ w, const XT *__restrict__ x,
                                                YT *__restrict__ y, int rows, int cols, uint64_t row_bytes)
{
    const int lane = lane_id();
    const int wv = (int)((blockIdx.x * blockDim.x + threadIdx.x) / WAVE);
    const int nw = (int)(gridDim.x * blockDim.x / WAVE);
    for (int r = wv; r < rows; r += nw) {
        const uint8_t *row = w + (size_t)r * row_bytes;
        float p;
        if (QT == BREAD_QTYPE_Q4_K)
            p = q4k_row_partial(row, cols / QK, x, lane);
        else if (QT == BREAD_QTYPE_Q6_K)
            p = q6k_row_partial(row, cols / QK, x, lane);
        else
            p = q80_row_partial(row, cols / Q80_ELEMS, x, lane);
        p = wave_sum(p);
        if (lane == 0) store_y(y, r, p);
    }
}

// ---- Long matvecs (the lm_head: 248,320 rows): each wave holds its lanes'
// slices of x in registers for all its rows (lane l always reads superblocks
// l/8 + 8j, j < NBL, of a row: cols = 2048 * NBL) and streams two rows per
// iteration, so x is read once per wave instead of once per row.

template <typename XT>
struct XQ4 {
    float xl[16], xh[16], sl, sh;
    __device__ __forceinline__ void load(const XT *x, int b, int c)
    {
        const int base = b * QK + 64 * (c >> 1) + 16 * (c & 1);
        load_x16(x, base, xl);
        load_x16(x, base + 32, xh);
        sl = 0.f;
        sh = 0.f;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            sl += xl[k];
            sh += xh[k];
        }
    }
};

template <typename XT>
struct XQ6 {
    float xs[4][8], X[4];
    __device__ __forceinline__ void load(const XT *x, int b, int c)
    {
        const int n = c >> 2, t = c & 3;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            load_x8(x, b * QK + 128 * n + 32 * s + 8 * t, xs[s]);
            X[s] = 0.f;
#pragma unroll
            for (int k = 0; k < 8; k++) X[s] += xs[s][k];
        }
    }
};

template <int QT, typename XT, typename YT, int NBL>
__global__ __launch_bounds__(256) void k_matvec_xr(const uint8_t *__restrict__ w, const XT *__restrict__ x,
                                                   YT *__restrict__ y, int rows, uint64_t row_bytes)
{
    constexpr int RPI = 4;  // rows per iteration
    const int lane = lane_id();
    const int c = lane & 7, b0 = lane >> 3;
    const int wv = (int)((blockIdx.x * blockDim.x + threadIdx.x) / WAVE);
    const int nw = (int)(gridDim.x * blockDim.x / WAVE);
    typename std::conditional<QT == BREAD_QTYPE_Q4_K, XQ4<XT>, XQ6<XT>>::type xr[NBL];
#pragma unroll
    for (int j = 0; j < NBL; j++) xr[j].load(x, b0 + 8 * j, c);
    for (int r0 = wv * RPI; r0 < rows; r0 += nw * RPI) {
        float p[RPI];
        if constexpr (QT == BREAD_QTYPE_Q4_K) {
            uint4 hd[RPI][NBL], q[RPI][NBL];
#pragma unroll
            for (int u = 0; u < RPI; u++)
#pragma unroll
                for (int j = 0; j < NBL; j++) {
                    const uint8_t *blk = w + (size_t)min(r0 + u, rows - 1) * row_bytes + (size_t)(b0 + 8 * j) * Q4K_BYTES;
                    hd[u][j] = ld_b128(blk);
                    q[u][j] = ld_b128(blk + 16 + 16 * c);
                }
#pragma unroll
            for (int u = 0; u < RPI; u++) {
                p[u] = 0.f;
#pragma unroll
                for (int j = 0; j < NBL; j++)
                    p[u] += q4k_chunk_dot_sx(hd[u][j], q[u][j], (uint32_t)(c >> 1), xr[j].xl, xr[j].xh, xr[j].sl,
                                             xr[j].sh);
            }
        } else {
            const int n = c >> 2, t = c & 3;
            uint2 ql0[RPI][NBL], ql1[RPI][NBL], qh[RPI][NBL], scw[RPI][NBL];
            uint32_t dd[RPI][NBL];
#pragma unroll
            for (int u = 0; u < RPI; u++)
#pragma unroll
                for (int j = 0; j < NBL; j++) {
                    const uint8_t *blk = w + (size_t)min(r0 + u, rows - 1) * row_bytes + (size_t)(b0 + 8 * j) * Q6K_BYTES;
                    ql0[u][j] = ld8_a2(blk + 64 * n + 8 * t);
                    ql1[u][j] = ld8_a2(blk + 64 * n + 32 + 8 * t);
                    qh[u][j] = ld8_a2(blk + 128 + 32 * n + 8 * t);
                    scw[u][j] = ld8_a2(blk + 192 + 8 * n);
                    dd[u][j] = ld16_a2(blk + 208);
                }
#pragma unroll
            for (int u = 0; u < RPI; u++) {
                p[u] = 0.f;
#pragma unroll
                for (int j = 0; j < NBL; j++)
                    p[u] += q6k_unit_dot_sx(ql0[u][j], ql1[u][j], qh[u][j], scw[u][j], (uint32_t)t >> 1,
                                            h2f(dd[u][j]), xr[j].xs, xr[j].X);
            }
        }
#pragma unroll
        for (int u = 0; u < RPI; u++) {
            const float v = wave_sum(p[u]);
            if (lane == 0 && r0 + u < rows) store_y(y, r0 + u, v);
        }
    }
}

// ---- Long Q4_K matvecs with fp16 x (the lm_head at fp16 I/O).  Four lanes
// a superblock, lane j owning its 32 quant bytes 32j .. 32j+31: low nibbles
// are elements 64j + [0, 32), high nibbles 64j + 32 + [0, 32), so each lane
// decodes one scale pair per superblock for 64 weights.  One wave covers
// 2 / NBL rows a slot (cols = 2048 NBL), four slots an iteration.  Every
// nibble q becomes the fp16 1 + q/64 (bytes 0x3C and q << 4, placed by
// v_perm_b32) and v_dot2_f32_f16 sums (1 + q/64) x against the lane's x pairs,
// each product exact in fp32; sum q x = 64 (a - sum x).  Row offsets are
// wave-uniform (scalar), the lane's offset in the slot fixed; raw buffer loads
// return zeros past the matrix, so the last slots need no clamping (their
// rows are not stored).
template <typename YT, int NBL>
__global__ __launch_bounds__(256) void k_matvec_q4h(const uint8_t *__restrict__ w, const uint16_t *__restrict__ x,
                                                    YT *__restrict__ y, int rows, uint32_t row_bytes)
{
    constexpr int RS = 2 / NBL;  // rows a slot
    constexpr int NS = 4;        // slots an iteration
    constexpr int RPI = RS * NS;
    const int lane = lane_id();
    const int j = lane & 3;
    const int b = (lane >> 2) & (8 * NBL - 1);
    const int h = lane / (32 * NBL);
    const int wv = uniform((int)((blockIdx.x * blockDim.x + threadIdx.x) / WAVE));
    const int nw = (int)(gridDim.x * blockDim.x / WAVE);
    uint32_t xl[16], xh[16];
    float sl = 0.f, sh = 0.f;
    {
        const uint4 *xp = reinterpret_cast<const uint4 *>(x + QK * b + 64 * j);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 a = xp[i], c = xp[4 + i];
            xl[4 * i] = a.x; xl[4 * i + 1] = a.y; xl[4 * i + 2] = a.z; xl[4 * i + 3] = a.w;
            xh[4 * i] = c.x; xh[4 * i + 1] = c.y; xh[4 * i + 2] = c.z; xh[4 * i + 3] = c.w;
        }
#pragma unroll
        for (int k = 0; k < 16; k++) {
            sl += h2f(xl[k]) + h2f(xl[k] >> 16);
            sh += h2f(xh[k]) + h2f(xh[k] >> 16);
        }
    }
    const auto wr = rsrc(w, (uint32_t)rows * row_bytes);
    const int voff = (int)((uint32_t)h * row_bytes + (uint32_t)b * Q4K_BYTES);
    // scale bytes of sub-blocks 2j, 2j + 1 (get_scale_min_k4): for j < 2 the
    // low six bits of bytes 2j, 2j+1 (scales) and 2j+4, 2j+5 (mins); for
    // j >= 2 the nibbles of bytes 2j+4, 2j+5 with the top two bits of bytes
    // 2j-4, 2j-3 (scales) and 2j, 2j+1 (mins)
    const bool jlo = j < 2;
    const uint32_t sel_lo = 0x05040100u + 0x02020202u * (uint32_t)j;               // y[2j, 2j+1], z[2j, 2j+1]
    const uint32_t sel_nb = 0x01000100u;
    const uint32_t sel_hi = 0x01000100u + 0x02020202u * (uint32_t)(jlo ? 0 : j - 2) + 0x04040000u;  // y[2j-4, 2j-3], z[2j-4, 2j-3]
    const int wsh = jlo ? 0 : 16 * (j - 2);
    for (int r0 = wv * RPI; r0 < rows; r0 += nw * RPI) {
        uint4 hd[NS], q0[NS], q1[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            // the whole offset in the vector operand: the range check covers it
            const int o = voff + (int)((uint32_t)(r0 + RS * s) * row_bytes);
            hd[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, o, 0, 0));
            q0[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, o + 16 + 32 * j, 0, 0));
            q1[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, o + 32 + 32 * j, 0, 0));
        }
#pragma unroll
        for (int s = 0; s < NS; s++) {
            // [sc0, sc1, m0, m1], one byte each
            uint32_t sm;
            if (jlo) {
                sm = __builtin_amdgcn_perm(hd[s].z, hd[s].y, sel_lo) & 0x3F3F3F3Fu;
            } else {
                const uint32_t n2 = (hd[s].w >> wsh) & 0xFFFFu;                     // bytes 2j+4, 2j+5
                const uint32_t nb = __builtin_amdgcn_perm(0u, n2, sel_nb);          // [b0, b1, b0, b1]
                const uint32_t lo4 = (nb & 0x00000F0Fu) | ((nb >> 4) & 0x0F0F0000u);
                const uint32_t top = __builtin_amdgcn_perm(hd[s].z, hd[s].y, sel_hi);  // [2j-4, 2j-3, 2j, 2j+1]
                sm = lo4 | ((top >> 2) & 0x30303030u);
            }
            const float d = h2f(hd[s].x), dmin = h2f(hd[s].x >> 16);
            const uint32_t qw[8] = {q0[s].x, q0[s].y, q0[s].z, q0[s].w, q1[s].x, q1[s].y, q1[s].z, q1[s].w};
            float al = 0.f, ah = 0.f;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const uint32_t lo = (qw[t] << 4) & 0xF0F0F0F0u;
                const uint32_t hi = qw[t] & 0xF0F0F0F0u;
                al = __builtin_amdgcn_fdot2(__builtin_bit_cast(qd_half2, __builtin_amdgcn_perm(0x3C3C3C3Cu, lo, 0x04010400u)),
                                            __builtin_bit_cast(qd_half2, xl[2 * t]), al, false);
                al = __builtin_amdgcn_fdot2(__builtin_bit_cast(qd_half2, __builtin_amdgcn_perm(0x3C3C3C3Cu, lo, 0x04030402u)),
                                            __builtin_bit_cast(qd_half2, xl[2 * t + 1]), al, false);
                ah = __builtin_amdgcn_fdot2(__builtin_bit_cast(qd_half2, __builtin_amdgcn_perm(0x3C3C3C3Cu, hi, 0x04010400u)),
                                            __builtin_bit_cast(qd_half2, xh[2 * t]), ah, false);
                ah = __builtin_amdgcn_fdot2(__builtin_bit_cast(qd_half2, __builtin_amdgcn_perm(0x3C3C3C3Cu, hi, 0x04030402u)),
                                            __builtin_bit_cast(qd_half2, xh[2 * t + 1]), ah, false);
            }
            float p = (d * (float)(sm & 0xFFu)) * (64.f * (al - sl)) - (dmin * (float)((sm >> 16) & 0xFFu)) * sl +
                      (d * (float)((sm >> 8) & 0xFFu)) * (64.f * (ah - sh)) - (dmin * (float)(sm >> 24)) * sh;
            p = NBL == 1 ? sum32(p) : wave_sum(p);
            const int r = r0 + RS * s + h;
            if ((lane & (32 * NBL - 1)) == 0 && r < rows) store_y(y, r, p);
        }
    }
}

// ---- Long Q6_K matvecs with fp16 x.  Four lanes a superblock: lane j takes
// half n = j / 2 and positions l = 16 (j % 2) + [0, 16) of it, i.e. the four
// 16-element runs 128 n + 32 s + l (s = 0..3) with scales sc[8 n + j % 2 +
// 2 s].  The 6-bit q of each weight becomes the fp16 1024 + q (bytes q, 0x64
// by v_perm_b32), exact; v_dot2_f32_f16 sums (1024 + q) x per run and
// sum (q - 32) x = a - 1056 sum x.  Superblocks are 210 bytes, so a lane's
// ranges sit 2 bytes past a dword boundary for odd superblocks: each range is
// loaded as aligned dwords plus one and realigned by v_alignbyte.  Slots,
// scalar row offsets and range-checked buffer loads as k_matvec_q4h.
template <typename YT, int NBL, int NS>
__global__ __launch_bounds__(256) void k_matvec_q6h(const uint8_t *__restrict__ w, const uint16_t *__restrict__ x,
                                                    YT *__restrict__ y, int rows, uint32_t row_bytes)
{
    constexpr int RS = 2 / NBL;  // rows a slot
    constexpr int RPI = RS * NS;
    const int lane = lane_id();
    const int j = lane & 3, n = j >> 1, hf = j & 1;
    const int b = (lane >> 2) & (8 * NBL - 1);
    const int h = lane / (32 * NBL);
    const int wv = uniform((int)((blockIdx.x * blockDim.x + threadIdx.x) / WAVE));
    const int nw = (int)(gridDim.x * blockDim.x / WAVE);
    uint32_t xs[4][8];
    float X[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint4 *xp = reinterpret_cast<const uint4 *>(x + QK * b + 128 * n + 32 * r + 16 * hf);
        const uint4 a = xp[0], c = xp[1];
        xs[r][0] = a.x; xs[r][1] = a.y; xs[r][2] = a.z; xs[r][3] = a.w;
        xs[r][4] = c.x; xs[r][5] = c.y; xs[r][6] = c.z; xs[r][7] = c.w;
        X[r] = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) X[r] += h2f(xs[r][k]) + h2f(xs[r][k] >> 16);
    }
    const auto wr = rsrc(w, (uint32_t)rows * row_bytes);
    const uint32_t sbo = (uint32_t)h * row_bytes + (uint32_t)b * Q6K_BYTES;
    const uint32_t sh = sbo & 3u;  // realignment, bytes (0 or 2)
    const int voff = (int)(sbo & ~3u);
    auto ld5 = [&](int o, uint32_t (&v)[4]) {
        const uint4 a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, o, 0, 0));
        const uint32_t e = __builtin_amdgcn_raw_buffer_load_b32(wr, o + 16, 0, 0);
        v[0] = __builtin_amdgcn_alignbyte(a.y, a.x, sh);
        v[1] = __builtin_amdgcn_alignbyte(a.z, a.y, sh);
        v[2] = __builtin_amdgcn_alignbyte(a.w, a.z, sh);
        v[3] = __builtin_amdgcn_alignbyte(e, a.w, sh);
    };
    for (int r0 = wv * RPI; r0 < rows; r0 += nw * RPI) {
        uint32_t qa[NS][4], qb[NS][4], qh[NS][4], sc[NS][2], dw[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int o = voff + (int)((uint32_t)(r0 + RS * s) * row_bytes);
            ld5(o + 64 * n + 16 * hf, qa[s]);
            ld5(o + 64 * n + 32 + 16 * hf, qb[s]);
            ld5(o + 128 + 32 * n + 16 * hf, qh[s]);
            const uint2 c2 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, o + 192 + 8 * n, 0, 0));
            const uint32_t c3 = __builtin_amdgcn_raw_buffer_load_b32(wr, o + 200 + 8 * n, 0, 0);
            sc[s][0] = __builtin_amdgcn_alignbyte(c2.y, c2.x, sh);
            sc[s][1] = __builtin_amdgcn_alignbyte(c3, c2.y, sh);
            dw[s] = __builtin_amdgcn_raw_buffer_load_b32(wr, o + 208, 0, 0) >> (8 * sh);
        }
#pragma unroll
        for (int s = 0; s < NS; s++) {
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t a = qa[s][t], bq = qb[s][t], hq = qh[s][t];
                const uint32_t q[4] = {(a & 0x0F0F0F0Fu) | ((hq << 4) & 0x30303030u),
                                       (bq & 0x0F0F0F0Fu) | ((hq << 2) & 0x30303030u),
                                       ((a >> 4) & 0x0F0F0F0Fu) | (hq & 0x30303030u),
                                       ((bq >> 4) & 0x0F0F0F0Fu) | ((hq >> 2) & 0x30303030u)};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    acc[r] = __builtin_amdgcn_fdot2(
                        __builtin_bit_cast(qd_half2, __builtin_amdgcn_perm(0x64646464u, q[r], 0x04010400u)),
                        __builtin_bit_cast(qd_half2, xs[r][2 * t]), acc[r], false);
                    acc[r] = __builtin_amdgcn_fdot2(
                        __builtin_bit_cast(qd_half2, __builtin_amdgcn_perm(0x64646464u, q[r], 0x04030402u)),
                        __builtin_bit_cast(qd_half2, xs[r][2 * t + 1]), acc[r], false);
                }
            }
            float p = 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // scale byte hf + 2 r of the half's eight: bytes hf, hf+2 of
                // the first word, then of the second
                const int scv = (int)(int8_t)(sc[s][r >> 1] >> (8 * (hf + 2 * (r & 1))));
                p = fmaf((float)scv, fmaf(-1056.f, X[r], acc[r]), p);
            }
            p *= h2f(dw[s]);
            p = NBL == 1 ? sum32(p) : wave_sum(p);
            const int rr = r0 + RS * s + h;
            if ((lane & (32 * NBL - 1)) == 0 && rr < rows) store_y(y, rr, p);
        }
    }
}

// ---- bit-exact dequant: one thread per 8 consecutive output elements.
// Operation order and roundings of dequant_q4k_cpu.c:111-121 / :155-165;
// contraction is off so d1*q - m1 is a multiply then a subtract.

__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t *__restrict__ w, float *__restrict__ out,
                                                     uint64_t n_groups)
{
#pragma clang fp contract(off)
    for (uint64_t g = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; g < n_groups;
         g += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t sb = g >> 5;          // superblock (rows are packed)
        const uint32_t e0 = (uint32_t)(g & 31) * 8;
        const uint8_t *blk = w + sb * Q4K_BYTES;
        const uint32_t hdr = ld_b32(blk);
        const float d = h2f_exact(hdr);
        const float dmin = h2f_exact(hdr >> 16);
        const uint32_t s0 = ld_b32(blk + 4), s1 = ld_b32(blk + 8), s2 = ld_b32(blk + 12);
        const uint32_t j = e0 >> 6, sub = (e0 >> 5) & 1, l0 = e0 & 31;
        uint32_t sc, m;
        scale_min_k4(2 * j + sub, s0, s1, s2, sc, m);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        const uint2 q = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + l0);
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t byte = byte_of(k < 4 ? q.x : q.y, k & 3);
            const uint32_t nib = sub ? (byte >> 4) : (byte & 0xF);
            v[k] = d1 * (float)nib - m1;
        }
        float4 *o = reinterpret_cast<float4 *>(out + sb * QK + e0);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t *__restrict__ w, float *__restrict__ out,
                                                     uint64_t n_groups)
{
#pragma clang fp contract(off)
    for (uint64_t g = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; g < n_groups;
         g += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t sb = g >> 5;
        const uint32_t e0 = (uint32_t)(g & 31) * 8;
        const uint8_t *blk = w + sb * Q6K_BYTES;
        const float d = h2f_exact(ld16_a2(blk + 208));
        const uint32_t n = e0 >> 7, s = (e0 >> 5) & 3, l0 = e0 & 31;
        const uint32_t is = l0 >> 4;
        const float scf = (float)(int8_t)blk[192 + 8 * n + is + 2 * s];
        const uint8_t *ql = blk + 64 * n + ((s & 1) ? 32 : 0) + l0;
        const uint8_t *qh = blk + 128 + 32 * n + l0;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t lb = ql[k];
            const uint32_t nib = (s & 2) ? (lb >> 4) : (lb & 0xF);
            const uint32_t hb = ((uint32_t)qh[k] >> (2 * s)) & 3u;
            const int q = (int)(int8_t)(nib | (hb << 4)) - 32;
            v[k] = d * scf * (float)q;
        }
        float4 *o = reinterpret_cast<float4 *>(out + sb * QK + e0);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

__global__ __launch_bounds__(256) void k_dequant_q80(const uint8_t *__restrict__ w, float *__restrict__ out,
                                                     uint64_t n_blocks)
{
#pragma clang fp contract(off)
    for (uint64_t b = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; b < n_blocks;
         b += (uint64_t)gridDim.x * blockDim.x) {
        const uint8_t *blk = w + b * Q80_BYTES;
        const float d = h2f_exact(ld16_a2(blk));
        for (int i = 0; i < Q80_ELEMS; i++) out[b * Q80_ELEMS + i] = d * (float)(int8_t)blk[2 + i];
    }
}

int check_matvec_args(const void *w, const void *x, const void *y, int rows, int cols, int qtype)
{
    BREAD_REQUIRE(w && x && y, BREAD_ERR_ARG, "NULL pointer");
    BREAD_REQUIRE(rows >= 0 && cols > 0, BREAD_ERR_ARG, "rows must be >= 0 and cols > 0");
    BREAD_REQUIRE(qtype == BREAD_QTYPE_Q4_K || qtype == BREAD_QTYPE_Q6_K || qtype == BREAD_QTYPE_Q8_0,
                  BREAD_ERR_QTYPE, "qtype must be 12 (Q4_K), 14 (Q6_K) or 8 (Q8_0)");
    const int blk = qtype == BREAD_QTYPE_Q8_0 ? Q80_ELEMS : QK;
    BREAD_REQUIRE(cols % blk == 0, BREAD_ERR_SHAPE, "cols must be a multiple of the block size");
    BREAD_REQUIRE(((uintptr_t)w & 3) == 0, BREAD_ERR_ALIGN, "w must be 4-byte aligned");
    BREAD_REQUIRE(((uintptr_t)x & 15) == 0, BREAD_ERR_ALIGN, "x must be 16-byte aligned");
    return BREAD_OK;
}

uint64_t row_bytes_of(int qtype, int cols)
{
    switch (qtype) {
    case BREAD_QTYPE_Q4_K: return (uint64_t)(cols / QK) * Q4K_BYTES;
    case BREAD_QTYPE_Q6_K: return (uint64_t)(cols / QK) * Q6K_BYTES;
    case BREAD_QTYPE_Q8_0: return (uint64_t)(cols / Q80_ELEMS) * Q80_BYTES;
    }
    return 0;
}

template <typename XT, typename YT>
int launch_matvec(const void *w, const XT *x, YT *y, int rows, int cols, int qtype, hipStream_t st)
{
    int rc = check_matvec_args(w, x, y, rows, cols, qtype);
    if (rc) return rc;
    if (rows == 0) return BREAD_OK;
    const uint64_t rb = row_bytes_of(qtype, cols);
    bread_clear_stale_error();
    const int waves_per_block = 4;
    int blocks = (rows + waves_per_block - 1) / waves_per_block;
    if (blocks > 65536) blocks = 65536;
    const uint8_t *wb = (const uint8_t *)w;
    // long matvecs with 2048 or 4096 columns: x held in registers, >= 4 rows
    // per wave (16 waves per CU)
    constexpr int XR_WAVES = 256 * 16;
    if constexpr (std::is_same<XT, uint16_t>::value) {
        // fp16 x, Q4_K: the dot2 kernel (32-bit buffer offsets: the matrix
        // and the last iteration's rows past it below 4 GB)
        if (rows >= 4 * XR_WAVES && (cols == 2048 || cols == 4096) && qtype == BREAD_QTYPE_Q4_K &&
            ((uint64_t)rows + 16) * rb < (1ull << 32)) {
            const dim3 g(XR_WAVES / 4), b(256);
            if (cols == 2048) hipLaunchKernelGGL((k_matvec_q4h<YT, 1>), g, b, 0, st, wb, x, y, rows, (uint32_t)rb);
            else hipLaunchKernelGGL((k_matvec_q4h<YT, 2>), g, b, 0, st, wb, x, y, rows, (uint32_t)rb);
            BREAD_HIP(hipGetLastError());
            return BREAD_OK;
        }
        if (rows >= 4 * XR_WAVES && (cols == 2048 || cols == 4096) && qtype == BREAD_QTYPE_Q6_K &&
            ((uint64_t)rows + 16) * rb < (1ull << 32)) {
            const dim3 g(XR_WAVES / 4), b(256);
            if (cols == 2048) hipLaunchKernelGGL((k_matvec_q6h<YT, 1, 2>), g, b, 0, st, wb, x, y, rows, (uint32_t)rb);
            else hipLaunchKernelGGL((k_matvec_q6h<YT, 2, 2>), g, b, 0, st, wb, x, y, rows, (uint32_t)rb);
            BREAD_HIP(hipGetLastError());
            return BREAD_OK;
        }
    }
    if (rows >= 4 * XR_WAVES && (cols == 2048 || cols == 4096) && qtype != BREAD_QTYPE_Q8_0) {
        const dim3 g(XR_WAVES / 4), b(256);
        if (qtype == BREAD_QTYPE_Q4_K) {
            if (cols == 2048) hipLaunchKernelGGL((k_matvec_xr<BREAD_QTYPE_Q4_K, XT, YT, 1>), g, b, 0, st, wb, x, y, rows, rb);
            else hipLaunchKernelGGL((k_matvec_xr<BREAD_QTYPE_Q4_K, XT, YT, 2>), g, b, 0, st, wb, x, y, rows, rb);
        } else {
            if (cols == 2048) hipLaunchKernelGGL((k_matvec_xr<BREAD_QTYPE_Q6_K, XT, YT, 1>), g, b, 0, st, wb, x, y, rows, rb);
            else hipLaunchKernelGGL((k_matvec_xr<BREAD_QTYPE_Q6_K, XT, YT, 2>), g, b, 0, st, wb, x, y, rows, rb);
        }
        BREAD_HIP(hipGetLastError());
        return BREAD_OK;
    }
    switch (qtype) {
    case BREAD_QTYPE_Q4_K:
        hipLaunchKernelGGL((k_matvec<BREAD_QTYPE_Q4_K, XT, YT>), dim3(blocks), dim3(256), 0, st, wb, x, y, rows, cols, rb);
        break;
    case BREAD_QTYPE_Q6_K:
        hipLaunchKernelGGL((k_matvec<BREAD_QTYPE_Q6_K, XT, YT>), dim3(blocks), dim3(256), 0, st, wb, x, y, rows, cols, rb);
        break;
    default:
        hipLaunchKernelGGL((k_matvec<BREAD_QTYPE_Q8_0, XT, YT>), dim3(blocks), dim3(256), 0, st, wb, x, y, rows, cols, rb);
        break;
    }
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

} // namespace

extern "C" int bread_matvec(const void *w, const uint16_t *x, uint16_t *y, int rows, int cols, int qtype,
                            bread_stream_t stream)
{
    return launch_matvec<uint16_t, uint16_t>(w, x, y, rows, cols, qtype, to_hip(stream));
}

extern "C" int bread_matvec_f32(const void *w, const float *x, float *y, int rows, int cols, int qtype,
                                bread_stream_t stream)
{
    return launch_matvec<float, float>(w, x, y, rows, cols, qtype, to_hip(stream));
}

extern "C" int bread_dequant_rows(const void *w, int qtype, int rows, int cols, float *out,
                                  bread_stream_t stream)
{
    BREAD_REQUIRE(w && out, BREAD_ERR_ARG, "NULL pointer");
    BREAD_REQUIRE(rows >= 0 && cols > 0, BREAD_ERR_ARG, "rows must be >= 0 and cols > 0");
    BREAD_REQUIRE(qtype == BREAD_QTYPE_Q4_K || qtype == BREAD_QTYPE_Q6_K || qtype == BREAD_QTYPE_Q8_0,
                  BREAD_ERR_QTYPE, "qtype must be 12 (Q4_K), 14 (Q6_K) or 8 (Q8_0)");
    const int blk = qtype == BREAD_QTYPE_Q8_0 ? Q80_ELEMS : QK;
    BREAD_REQUIRE(cols % blk == 0, BREAD_ERR_SHAPE, "cols must be a multiple of the block size");
    BREAD_REQUIRE(((uintptr_t)w & 3) == 0, BREAD_ERR_ALIGN, "w must be 4-byte aligned");
    BREAD_REQUIRE(((uintptr_t)out & 15) == 0, BREAD_ERR_ALIGN, "out must be 16-byte aligned");
    if (rows == 0) return BREAD_OK;
    hipStream_t st = to_hip(stream);
    bread_clear_stale_error();
    const uint64_t n_blocks = (uint64_t)rows * (uint64_t)(cols / blk);
    const uint8_t *wb = (const uint8_t *)w;
    if (qtype == BREAD_QTYPE_Q8_0) {
        const uint64_t g = (n_blocks + 255) / 256;
        hipLaunchKernelGGL(k_dequant_q80, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(256), 0, st, wb, out, n_blocks);
    } else {
        const uint64_t n_groups = n_blocks * 32;
        const uint64_t g = (n_groups + 255) / 256;
        const dim3 grid((unsigned)(g < 65536 ? g : 65536));
        if (qtype == BREAD_QTYPE_Q4_K)
            hipLaunchKernelGGL(k_dequant_q4k, grid, dim3(256), 0, st, wb, out, n_groups);
        else
            hipLaunchKernelGGL(k_dequant_q6k, grid, dim3(256), 0, st, wb, out, n_groups);
    }
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}
