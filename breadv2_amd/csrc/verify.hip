// verify.hip — batched speculative verification at the MoE boundary.
//
// The reference verifies a draft of K tokens one token at a time: bread_step
// (main_speculative.cu:262-271) runs the whole model for one token, then
// greedy_sample (main.cu:326-335) takes the argmax of the fp16 logits, and
// the loop of main_speculative.cu:477-497 accepts drafts while the target's
// prediction equals them.  Here the B = K + 1 tokens of a round (the last
// confirmed token and the K drafts) go through each MoE layer together:
//   bread_moe_stack_forward  B tokens through a stack of MoE layers, one
//                            grouped bread_moe_forward per layer (one decode
//                            stack launch when B == 1);
//   bread_moe_greedy_head    output RMSNorm to fp16, the lm_head through
//                            bread_matvec (fp16 logits, main.cu:297-319) and
//                            the argmax of each token's logits on the device;
//   bread_spec_accept        the acceptance rule of :477-497 on the host.
#include <math.h>

#include <algorithm>

#include "bread_device.h"
#include "bread_internal.h"
#include "q4k_mfma.h"

namespace {

// Per token: out = x * inv_rms * w (w NULL: unit), inv_rms =
// 1/sqrt(mean(x^2) + eps), stored as fp32 or rounded to fp16.
template <typename OT>
__global__ __launch_bounds__(256) void k_norm_rows(const float *__restrict__ x, const float *__restrict__ w,
                                                   OT *__restrict__ out, int n, float eps)
{
    __shared__ float part[4];
    const float *xt = x + (size_t)blockIdx.x * n;
    OT *ot = out + (size_t)blockIdx.x * n;
    const int tid = (int)threadIdx.x;
    // rows up to NRK * 256 elements stay in registers between the two
    // passes (x and w requested together, one memory round trip); the
    // arithmetic and its order are the same either way
    constexpr int NRK = 8;
    const bool held = n <= NRK * 256;
    float xv[NRK], wv[NRK];
    float ss = 0.f;
    if (held) {
#pragma unroll
        for (int k = 0; k < NRK; k++) {
            const int i = tid + 256 * k;
            xv[k] = i < n ? xt[i] : 0.f;
            wv[k] = i < n && w ? w[i] : 1.0f;
        }
#pragma unroll
        for (int k = 0; k < NRK; k++)
            if (tid + 256 * k < n) ss = fmaf(xv[k], xv[k], ss);
    } else {
        for (int i = tid; i < n; i += 256) ss = fmaf(xt[i], xt[i], ss);
    }
    ss = wave_sum(ss);
    if (lane_id() == 0) part[tid / WAVE] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)n + eps);
    auto put = [&](int i, float v) {
        if constexpr (sizeof(OT) == 2) ot[i] = f2h(v);
        else ot[i] = v;
    };
    if (held) {
#pragma unroll
        for (int k = 0; k < NRK; k++)
            if (tid + 256 * k < n) put(tid + 256 * k, xv[k] * inv * wv[k]);
    } else {
        for (int i = tid; i < n; i += 256) put(i, xt[i] * inv * (w ? w[i] : 1.0f));
    }
}

// greedy_sample's rule (main.cu:326-335): best starts at logits[0] and moves
// to i only when logits[i] > best, so the result is the first index of the
// largest non-NaN value, and 0 when logits[0] is NaN.  Parallel form: each
// thread keeps (value, first index) over its strided subset, skipping NaN,
// and the block reduces with "larger value, then smaller index".
constexpr int AM_THREADS = 1024;

__device__ __forceinline__ void am_merge(float &bv, int &bi, float v, int i)
{
    if (i < 0) return;
    if (bi < 0 || v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__global__ __launch_bounds__(AM_THREADS) void k_argmax_f16(const uint16_t *__restrict__ logits, int n,
                                                            int32_t *__restrict__ out)
{
    __shared__ float sv[AM_THREADS / WAVE];
    __shared__ int si[AM_THREADS / WAVE];
    const uint16_t *lt = logits + (size_t)blockIdx.x * n;
    float bv = 0.f;
    int bi = -1;
    const int n8 = (n & 7) == 0 ? n / 8 : 0;  // rows are 16-byte aligned when n % 8 == 0
    for (int v = threadIdx.x; v < n8; v += AM_THREADS) {
        const uint4 q = reinterpret_cast<const uint4 *>(lt)[v];
        const uint32_t p[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float f = h2f(p[k / 2] >> (16 * (k & 1)));
            if (!isnan(f)) am_merge(bv, bi, f, 8 * v + k);
        }
    }
    for (int i = 8 * n8 + threadIdx.x; i < n; i += AM_THREADS) {
        const float f = h2f(lt[i]);
        if (!isnan(f)) am_merge(bv, bi, f, i);
    }
    for (int off = WAVE / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        am_merge(bv, bi, ov, oi);
    }
    if (lane_id() == 0) {
        sv[threadIdx.x / WAVE] = bv;
        si[threadIdx.x / WAVE] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int wv = 1; wv < AM_THREADS / WAVE; wv++) am_merge(bv, bi, sv[wv], si[wv]);
        out[blockIdx.x] = (bi < 0 || isnan(h2f(lt[0]))) ? 0 : bi;
    }
}

// ---------------------------------------------------------------------------
// Batched greedy head: the lm_head for T <= 32 tokens in one pass over its
// Q4_K weights (main.cu:297-319 runs one bread_matvec per token; a verify
// round of main_speculative.cu:477-497 runs B of them), with the argmax of
// each token's logits (greedy_sample, main.cu:326-335) folded in.
//
// A Q4_K weight is d sc_j q - dmin m_j in sub-block j (32 elements), so a
// superblock's dot product with x is d D - dmin M, D = sum sc_j q x and
// M = sum_j m_j X_j, X_j the sum of x over sub-block j.  D runs on
// v_mfma_f32_16x16x32_f16 with tokens as the M side and 16 weight rows as
// the N side: the B operand is sc q (exact in fp16, <= 945, from the nibble
// by a byte permutation and one packed fp16 fma), the A operand the fp16 x
// (exact), the products exact and the sums fp32.  M runs on two
// v_mfma_f32_16x16x4_f32 (X_j fp32, m_j exact).
//
// Lanes: lane l holds token / weight row c = l % 16 and quarter g = l / 16.
// From weight row c it reads the superblock's 16-byte head and qs bytes
// [32 g, 32 g + 32): the low nibbles are elements 64 g + e of the
// superblock (sub-block 2 g), the high nibbles 64 g + 32 + e (sub-block
// 2 g + 1).  Eight MFMAs take 8 of these elements each, so MFMA i covers
// elements 64 g + 8 i .. + 7 in quarter g; the x fragments follow the same
// order (a relabelling of K that A and B share), and so the lane also holds
// x over sub-blocks 2 g and 2 g + 1 of its token, whose sums are its X_j.
// The D layout puts tokens 4 g + i of row c in lane l, where the row's d
// and dmin are.
//
// Workgroup: HD_MAXSB compute waves, wave w owning superblock w (a K slice)
// of every row with its x fragments in registers for the whole launch, and
// HD_NRED reducing waves.  Workgroups take 16-row tiles in turn, one barrier
// a tile.  A compute wave keeps DEPTH tiles of its superblock column in a
// register ring, loading tile k + DEPTH - 1 while it computes tile k (the
// compiler's own vmcnt waits); its partial sums go to LDS, double-buffered.
// The reducing waves sum the partials, round to fp16, store the logits and
// keep a running argmax per token while the compute waves work on the next
// tile.  (Staging tiles in LDS with direct-to-LDS loads gave stale data now
// and then: a slot read right after the issuing wave's vmcnt drained and a
// barrier did not always hold the loaded bytes yet.)
// ---------------------------------------------------------------------------
constexpr int HD_MAXSB = 8;           // superblocks a row (H <= 2048): one compute wave each
constexpr int HD_MAXT = 32;           // tokens a launch (two 16-token tiles)
constexpr int HD_NRED = 4;            // reducing waves: one thread per (token, row) of a 16 x 16 tile
constexpr int HD_THREADS = 64 * (HD_MAXSB + HD_NRED);
// register ring slots a compute wave (tiles in flight + 1), for one and two
// 16-token tiles (two hold twice the x fragments)
constexpr int HD_DEPTH1 = 4, HD_DEPTH2 = 3;
constexpr int HD_GRID = 256;          // workgroups: one a CU (12 waves of up to 168 VGPRs)

template <int NTT, int DEPTH>
__global__ __launch_bounds__(HD_THREADS) void k_head_q4k(const uint8_t *__restrict__ w,
                                                         const uint16_t *__restrict__ x16,
                                                         uint16_t *__restrict__ logits, float *__restrict__ part_v,
                                                         int32_t *__restrict__ part_i, int vocab, int H, int T)
{
    __shared__ float part[2][HD_MAXSB][NTT * 16][17];  // [buffer][superblock][tt, token][row]
    const int NSB = H / 256;
    const int wv = wave_id(), l = lane_id();
    const size_t row_bytes = (size_t)NSB * Q4K_BYTES;
    const int ntile = vocab / 16;
    const int G = gridDim.x;
    const int niter = ((int)blockIdx.x < ntile) ? (ntile - 1 - (int)blockIdx.x) / G + 1 : 0;
    if (wv < HD_MAXSB) {
        if (wv >= NSB) {  // no superblock: keep the barrier count
            for (int it = 0; it < niter; it++) q4m_bar();
            return;
        }
        const int g = l >> 4, c = l & 15;
        // x fragments of token 16 tt + c (zero beyond T): MFMA i takes
        // elements 256 wv + 64 g + 8 i .. + 7; xm = the sums over sub-blocks
        // 2 g and 2 g + 1
        uint4 xf[NTT][8];
        float xm[NTT][2];
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) {
            const int t = 16 * tt + c;
            xm[tt][0] = xm[tt][1] = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xf[tt][i] = t < T ? *reinterpret_cast<const uint4 *>(x16 + (size_t)t * H + 256 * wv + 64 * g + 8 * i)
                                  : make_uint4(0u, 0u, 0u, 0u);
                const uint32_t v[4] = {xf[tt][i].x, xf[tt][i].y, xf[tt][i].z, xf[tt][i].w};
#pragma unroll
                for (int k = 0; k < 4; k++) xm[tt][i >> 2] += h2f(v[k] & 0xFFFFu) + h2f(v[k] >> 16);
            }
        }
        // tile it's column; past the workgroup's last tile that one again
        // (an L2 hit): loads without a condition keep the compiler's vmcnt
        // waits counted rather than draining
        const uint8_t *wcol = w + (size_t)c * row_bytes + (size_t)wv * Q4K_BYTES;  // row c of tile 0
        auto load = [&](Q4mRaw &r, int it) {
            const int ti = (int)blockIdx.x + std::min(it, niter - 1) * G;
            q4m_load(r, wcol + (size_t)16 * ti * row_bytes, g);
        };
        Q4mRaw ring[DEPTH];
#pragma unroll
        for (int k = 0; k < DEPTH - 1; k++) load(ring[k], k);
        for (int it0 = 0; it0 < niter; it0 += DEPTH) {
#pragma unroll
            for (int k = 0; k < DEPTH; k++) {
                const int it = it0 + k;
                if (it >= niter) break;
                load(ring[(k + DEPTH - 1) % DEPTH], it + DEPTH - 1);
                const Q4mRaw &b = ring[k];
                const float d = h2f(b.head.x & 0xFFFFu), dmin = h2f(b.head.x >> 16);
                uint32_t sc0, m0, sc1, m1;
                scale_min_k4(2 * g, b.head.y, b.head.z, b.head.w, sc0, m0);
                scale_min_k4(2 * g + 1, b.head.y, b.head.z, b.head.w, sc1, m1);
                const _Float16 s0 = (_Float16)(float)sc0, s1 = (_Float16)(float)sc1;
                const _Float16 n0 = (_Float16)(-1024.f * (float)sc0), n1 = (_Float16)(-1024.f * (float)sc1);
                const q4m_half2 S0{s0, s0}, N0{n0, n0}, S1{s1, s1}, N1{n1, n1};
                const q4m_half8 bq[8] = {q4m_b8(b.q0.x, b.q0.y, 0, S0, N0), q4m_b8(b.q0.z, b.q0.w, 0, S0, N0),
                                        q4m_b8(b.q1.x, b.q1.y, 0, S0, N0), q4m_b8(b.q1.z, b.q1.w, 0, S0, N0),
                                        q4m_b8(b.q0.x, b.q0.y, 1, S1, N1), q4m_b8(b.q0.z, b.q0.w, 1, S1, N1),
                                        q4m_b8(b.q1.x, b.q1.y, 1, S1, N1), q4m_b8(b.q1.z, b.q1.w, 1, S1, N1)};
#pragma unroll
                for (int tt = 0; tt < NTT; tt++) {
                    q4m_f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(q4m_half8, xf[tt][i]), bq[i],
                                                                     acc, 0, 0, 0);
                    accm = __builtin_amdgcn_mfma_f32_16x16x4f32(xm[tt][0], (float)m0, accm, 0, 0, 0);
                    accm = __builtin_amdgcn_mfma_f32_16x16x4f32(xm[tt][1], (float)m1, accm, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        part[it & 1][wv][16 * tt + 4 * g + i][c] = d * acc[i] - dmin * accm[i];
                }
                q4m_bar();
            }
        }
        return;
    }
    // reducing waves: thread r sums output (tt, token, row) = (r / 256 + k,
    // (r / 16) % 16, r % 16) for k = 0 .. NTT - 1
    const int r = (int)threadIdx.x - 64 * HD_MAXSB, row = r & 15, tok = r >> 4;
    float best[NTT];
    int besti[NTT];
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
        best[tt] = 0.f;
        besti[tt] = -1;
    }
    // the barrier after tile it's partials are in part[it & 1]; reduced
    // while the compute waves work on tile it + 1
    for (int it = 0; it < niter; it++) {
        q4m_bar();
        const int ti = (int)blockIdx.x + it * G;
#pragma unroll
        for (int tt = 0; tt < NTT; tt++) {
            const int t = 16 * tt + tok;
            if (t >= T) continue;  // uniform over each 16-lane row group
            float v = 0.f;
            for (int sbi = 0; sbi < NSB; sbi++) v += part[it & 1][sbi][16 * tt + tok][row];
            const uint16_t h = f2h(v);
            logits[(size_t)t * vocab + 16 * ti + row] = h;
            // greedy_sample's order: the largest non-NaN value, the lowest
            // index among equals; the lane's rows come in increasing order,
            // so a strictly larger value replaces its best
            const float vf = h2f(h);
            if (vf == vf && (besti[tt] < 0 || vf > best[tt])) {
                best[tt] = vf;
                besti[tt] = 16 * ti + row;
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
        // the 16 lanes of the token's row group: larger value, then lower index
        float bv = best[tt];
        int bi = besti[tt];
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 16);
            const int oi = __shfl_xor(bi, off, 16);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
        best[tt] = bv;
        besti[tt] = bi;
    }
#pragma unroll
    for (int tt = 0; tt < NTT; tt++) {
        const int t = 16 * tt + tok;
        if (row == 0 && t < T) {
            part_v[(size_t)t * G + blockIdx.x] = best[tt];
            part_i[(size_t)t * G + blockIdx.x] = besti[tt];
        }
    }
}

// Token t's argmax from the workgroups' partials: the largest value, the
// lowest index among equals; 0 when logits[t][0] is NaN (greedy_sample keeps
// index 0 then) or no value is a number.
__global__ __launch_bounds__(256) void k_head_argmax_merge(const float *__restrict__ part_v,
                                                           const int32_t *__restrict__ part_i, int nparts,
                                                           const uint16_t *__restrict__ logits, int vocab,
                                                           int32_t *__restrict__ out)
{
    __shared__ float sv[256 / WAVE];
    __shared__ int si[256 / WAVE];
    const int t = blockIdx.x;
    float bv = 0.f;
    int bi = -1;
    for (int p = threadIdx.x; p < nparts; p += 256) {
        const float v = part_v[(size_t)t * nparts + p];
        const int i = part_i[(size_t)t * nparts + p];
        if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) {
            bv = v;
            bi = i;
        }
    }
    for (int off = WAVE / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane_id() == 0) {
        sv[threadIdx.x / WAVE] = bv;
        si[threadIdx.x / WAVE] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 256 / WAVE; k++)
            if (si[k] >= 0 && (bi < 0 || sv[k] > bv || (sv[k] == bv && si[k] < bi))) {
                bv = sv[k];
                bi = si[k];
            }
        out[t] = (bi < 0 || isnan(h2f(logits[(size_t)t * vocab]))) ? 0 : bi;
    }
}

// The batched head over tokens [0, T) in chunks of HD_MAXT, each chunk one
// pass over the weights.  The workgroups' argmax partials live in the
// context's SwiGLU buffer (free between MoE calls on the stream).
int launch_head_q4k(bread_moe_ctx_t *c, const uint8_t *w, const uint16_t *x16, int vocab, int T, uint16_t *logits,
                    int32_t *tokens, hipStream_t st)
{
    const int H = c->shape.hidden;
    const int Imax = c->shape.expert_inter > c->shape.shared_inter ? c->shape.expert_inter : c->shape.shared_inter;
    const size_t h_floats = (size_t)c->max_tokens * (c->shape.top_k + 1) * Imax;
    const int tmax = std::min(T, HD_MAXT);
    const int grid = (int)std::min<size_t>((size_t)std::min(vocab / 16, HD_GRID), h_floats / (2 * (size_t)tmax));
    if (grid < 1) return bread_fail(BREAD_ERR_CAPACITY, "bread_moe_greedy_head", "no room for the argmax partials");
    for (int t0 = 0; t0 < T; t0 += HD_MAXT) {
        const int tn = std::min(HD_MAXT, T - t0);
        float *pv = c->h;
        int32_t *pi = reinterpret_cast<int32_t *>(c->h + (size_t)tn * grid);
        bread_clear_stale_error();
        if (tn > 16)
            hipLaunchKernelGGL((k_head_q4k<2, HD_DEPTH2>), dim3(grid), dim3(HD_THREADS), 0, st, w, x16 + (size_t)t0 * H,
                               logits + (size_t)t0 * vocab, pv, pi, vocab, H, tn);
        else
            hipLaunchKernelGGL((k_head_q4k<1, HD_DEPTH1>), dim3(grid), dim3(HD_THREADS), 0, st, w, x16 + (size_t)t0 * H,
                               logits + (size_t)t0 * vocab, pv, pi, vocab, H, tn);
        BREAD_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_head_argmax_merge, dim3(tn), dim3(256), 0, st, pv, pi, grid,
                           logits + (size_t)t0 * vocab, vocab, tokens + t0);
        BREAD_HIP(hipGetLastError());
    }
    return BREAD_OK;
}

}  // namespace

// One token through layers[0..n): each run of consecutive layers with the
// decode kernel's weight types is one persistent launch; any other layer
// (another mix of Q4_K and Q6_K) is the RMSNorm kernel followed by the
// per-token kernels.  Routing outputs go to record l * rstride of layer l,
// as in bread_launch_decode_layers.
int bread_launch_decode_runs(bread_moe_ctx_t *c, const bread_moe_layer_t *layers, int n, float *hidden,
                             int32_t *idx, float *w, float *gsh, hipStream_t st, int rstride)
{
    const int H = c->shape.hidden, K = c->shape.top_k;
    // Decide before launching anything: a run refused after earlier layers
    // had run would leave hidden part-way through the stack, and a caller
    // that falls back to another path on BREAD_ERR_SHAPE would apply those
    // layers twice.
    for (int l = 0, run = 0; l < n; l++) {
        if (!bread_standard_qtypes(&layers[l])) {
            run = 0;
            continue;
        }
        if (!bread_decode_accepts(c, &layers[l])) return BREAD_ERR_SHAPE;
        if (++run > c->max_layers) return BREAD_ERR_CAPACITY;
    }
    for (int l = 0; l < n;) {
        const size_t r = (size_t)l * rstride;
        if (bread_standard_qtypes(&layers[l])) {
            int m = l + 1;
            while (m < n && bread_standard_qtypes(&layers[m])) m++;
            const int rc = bread_launch_decode_layers(c, layers + l, m - l, hidden, idx ? idx + r * K : nullptr,
                                                      w ? w + r * K : nullptr, gsh ? gsh + r : nullptr, st, rstride);
            if (rc) return rc;
            l = m;
            continue;
        }
        bread_clear_stale_error();
        hipLaunchKernelGGL(k_norm_rows<float>, dim3(1), dim3(256), 0, st, hidden, layers[l].post_norm_w, c->x32, H,
                           c->shape.rms_eps);
        BREAD_HIP(hipGetLastError());
        const int rc = bread_launch_moe_multi(c, &layers[l], c->x32, hidden, 1, st);
        if (rc) return rc;
        if (idx) BREAD_HIP(hipMemcpyAsync(idx + r * K, c->idx, K * sizeof(int32_t), hipMemcpyDeviceToDevice, st));
        if (w) BREAD_HIP(hipMemcpyAsync(w + r * K, c->w, K * sizeof(float), hipMemcpyDeviceToDevice, st));
        if (gsh) BREAD_HIP(hipMemcpyAsync(gsh + r, c->gsh, sizeof(float), hipMemcpyDeviceToDevice, st));
        l++;
    }
    return BREAD_OK;
}

extern "C" int bread_moe_stack_forward(bread_moe_ctx_t *c, const bread_moe_layer_t *layers, int n, float *hidden,
                                       int T, int32_t *idx, float *w, float *gsh, bread_stream_t stream)
{
    BREAD_REQUIRE(c && layers && hidden, BREAD_ERR_ARG, "NULL context, layers or hidden");
    BREAD_REQUIRE(n >= 0 && T >= 0, BREAD_ERR_ARG, "n_layers and n_tokens must be >= 0");
    BREAD_REQUIRE(T <= c->max_tokens, BREAD_ERR_CAPACITY, "n_tokens > max_tokens of the context");
    BREAD_REQUIRE(((uintptr_t)hidden & 15) == 0, BREAD_ERR_ALIGN, "hidden must be 16-byte aligned");
    for (int l = 0; l < n; l++) {
        const int rc = bread_validate_layer(&c->shape, &layers[l]);
        if (rc) return rc;
        BREAD_REQUIRE(((uintptr_t)layers[l].post_norm_w & 15) == 0, BREAD_ERR_ALIGN,
                      "post_norm_w must be 16-byte aligned");
    }
    if (n == 0 || T == 0) return BREAD_OK;
    const int H = c->shape.hidden, K = c->shape.top_k;
    // one token, or up to bread_stack_loop_tokens() under the automatic
    // choice: the whole stack in one persistent launch per token, when the
    // shape allows it (token t's routing goes to record t of each layer)
    if ((T == 1 && (c->path == BREAD_PATH_AUTO || c->path == BREAD_PATH_DECODE)) ||
        (T <= bread_stack_loop_tokens() && c->path == BREAD_PATH_AUTO)) {
        if (n <= c->max_layers) {
            hipStream_t st = to_hip(stream);
            c->last_stream = st;
            int rc = BREAD_OK;
            for (int t = 0; t < T && rc == BREAD_OK; t++)
                rc = bread_launch_decode_runs(c, layers, n, hidden + (size_t)t * H, idx ? idx + (size_t)t * K : nullptr,
                                              w ? w + (size_t)t * K : nullptr, gsh ? gsh + t : nullptr, st, T);
            if (rc != BREAD_ERR_SHAPE || c->path == BREAD_PATH_DECODE) return rc;
            bread_clear_stale_error();
        }
    }
    hipStream_t st = to_hip(stream);
    for (int l = 0; l < n; l++) {
        bread_clear_stale_error();
        hipLaunchKernelGGL(k_norm_rows<float>, dim3(T), dim3(256), 0, st, hidden, layers[l].post_norm_w, c->x32, H,
                           c->shape.rms_eps);
        BREAD_HIP(hipGetLastError());
        const size_t o = (size_t)l * T;
        const int rc = bread_moe_forward(c, &layers[l], c->x32, hidden, T, idx ? idx + o * K : nullptr,
                                         w ? w + o * K : nullptr, gsh ? gsh + o : nullptr, stream);
        if (rc) return rc;
    }
    return BREAD_OK;
}

extern "C" int bread_moe_greedy_head(bread_moe_ctx_t *c, const float *hidden, const float *norm_w,
                                     const void *w_out, int qtype, int vocab, int T, uint16_t *logits,
                                     int32_t *tokens, bread_stream_t stream)
{
    BREAD_REQUIRE(c && hidden && w_out && logits && tokens, BREAD_ERR_ARG, "NULL argument");
    BREAD_REQUIRE(vocab > 0 && T >= 0, BREAD_ERR_ARG, "vocab must be > 0 and n_tokens >= 0");
    BREAD_REQUIRE(T <= c->max_tokens, BREAD_ERR_CAPACITY, "n_tokens > max_tokens of the context");
    BREAD_REQUIRE((((uintptr_t)hidden | (uintptr_t)norm_w | (uintptr_t)logits) & 15) == 0 && vocab % 8 == 0,
                  BREAD_ERR_ALIGN, "hidden, norm_w and logits must be 16-byte aligned and vocab a multiple of 8");
    if (T == 0) return BREAD_OK;
    const int H = c->shape.hidden;
    hipStream_t st = to_hip(stream);
    c->last_stream = st;
    // the fp16 normalised rows live in the context's fp32 input buffer
    uint16_t *x16 = reinterpret_cast<uint16_t *>(c->x32);
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_norm_rows<uint16_t>, dim3(T), dim3(256), 0, st, hidden, norm_w, x16, H, c->shape.rms_eps);
    BREAD_HIP(hipGetLastError());
    if (qtype == BREAD_QTYPE_Q4_K && H % 256 == 0 && H / 256 <= HD_MAXSB && vocab % 16 == 0 &&
        ((uintptr_t)w_out & 15) == 0)
        return launch_head_q4k(c, static_cast<const uint8_t *>(w_out), x16, vocab, T, logits, tokens, st);
    for (int t = 0; t < T; t++) {
        const int rc = bread_matvec(w_out, x16 + (size_t)t * H, logits + (size_t)t * vocab, vocab, H, qtype, stream);
        if (rc) return rc;
    }
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_argmax_f16, dim3(T), dim3(AM_THREADS), 0, st, logits, vocab, tokens);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

extern "C" int bread_argmax_f16(const uint16_t *logits, int n, int T, int32_t *out, bread_stream_t stream)
{
    BREAD_REQUIRE(logits && out, BREAD_ERR_ARG, "NULL argument");
    BREAD_REQUIRE(n > 0 && T >= 0, BREAD_ERR_ARG, "n must be > 0 and n_tokens >= 0");
    BREAD_REQUIRE((n % 8 != 0) || ((uintptr_t)logits & 15) == 0, BREAD_ERR_ALIGN,
                  "logits must be 16-byte aligned when n is a multiple of 8");
    if (T == 0) return BREAD_OK;
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_argmax_f16, dim3(T), dim3(AM_THREADS), 0, to_hip(stream), logits, n, out);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

extern "C" int bread_spec_accept(const int32_t *pred, const int32_t *draft, int n_draft, int32_t eos,
                                 int max_accept, int *n_accept, int32_t *next)
{
    BREAD_REQUIRE(pred && n_accept && next && (draft || n_draft == 0), BREAD_ERR_ARG, "NULL argument");
    BREAD_REQUIRE(n_draft >= 0 && max_accept >= 1, BREAD_ERR_ARG, "n_draft must be >= 0 and max_accept >= 1");
    // main_speculative.cu:477-497: the target's prediction after token i is
    // pred[i] (token 0 is the last confirmed one); draft i is accepted while
    // it equals the running prediction and is not EOS; the prediction at the
    // first mismatch (or after the last draft) is the next confirmed token.
    // Once the output budget is spent the reference stops stepping, so the
    // running prediction stays the last accepted draft.
    int a = 0;
    int32_t target = pred[0];
    while (a < n_draft && target == draft[a] && target != eos) {
        a++;
        if (a >= max_accept) break;
        target = pred[a];
    }
    *n_accept = a;
    *next = target;
    return BREAD_OK;
}
