// route.hip — routing for the multi-token paths, bit-identical to the
// reference's host routing (route_layer, one_layer.cu:964-985, with
// cpu_softmax / cpu_topk, layer_ops.cu:222-250).
//
// k_route_seq computes every router logit in the reference's own order:
//   logits[e] = ((0 + W[e][0] x[0]) + W[e][1] x[1]) + ... + W[e][H-1] x[H-1],
// each product rounded to fp32, then added, never fused (one_layer.cu:969-971),
// and the shared-gate score the same way with the fp16 gate widened
// (one_layer.cu:977-980).  The sum is inherently sequential, so the kernel
// gives each lane one token and each wave one router row (two beyond two
// workgroups per CU): a lane's 2048 dependent (product, add) pairs are the
// latency floor of exact routing, and route_seq.h keeps every other cost
// (activation staging, router weights by DPP broadcast) off that chain.

// k_topk_exact then runs softmax / top-k / renormalisation per token (one
// wave) with the host's arithmetic (softmax_keys_exact): given identical
// logits, indices and weights are bit-identical to the reference's.
#include <mutex>

#include "bread_internal.h"
#include "quant_dot.h"
#include "route_dev.h"
#include "route_seq.h"

// Logits workspace of bread_route_noalloc: n_tokens x n_experts floats at
// most (4 MiB; each GPU the library runs on holds one until the process
// ends).  Every entry a call reads is written by the same call first, so it
// is never cleared; calls that overlap on one GPU share it and race.
constexpr size_t SCRATCH_FLOATS = size_t(1) << 20;
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];

namespace {

using namespace route_seq;

// Device address of `scratch` per device, taken once with that device current.
constexpr int MAX_DEVICES = 64;
float *scratch_ptr[MAX_DEVICES];
std::mutex scratch_mu;

int scratch_for_current_device(float **out)
{
    int dev = 0;
    BREAD_HIP(hipGetDevice(&dev));
    BREAD_REQUIRE(dev >= 0 && dev < MAX_DEVICES, BREAD_ERR_ARG, "device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void *p = nullptr;
        BREAD_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        scratch_ptr[dev] = static_cast<float *>(p);
    }
    *out = scratch_ptr[dev];
    return BREAD_OK;
}

// Grid (ceil(E / (4 NE)) + shg_row, ceil(T / 64)): route_seq_block.
template <int NE>
__global__ __launch_bounds__(RS_WAVES * WAVE) void k_route_seq(const float *__restrict__ router,
                                                              const uint16_t *__restrict__ shg,
                                                              const float *__restrict__ x, float *__restrict__ logits,
                                                              float *__restrict__ gsh, int H, int E, int T,
                                                              int shg_row)
{
    __shared__ RsSmem S;
    route_seq_block<NE>(S, (int)blockIdx.x, (int)blockIdx.y, router, shg, x, logits, gsh, H, E, T, shg_row != 0);
}

// ---------------------------------------------------------------------------
// Certified fast routing for a few tokens.  The reference's sequential sums
// (one_layer.cu:969-971) are a 2048-step dependent chain per logit; for a
// few tokens the chain, not the data, sets the time of k_route_seq.  Here
// every logit is first summed in parallel with a rigorous radius R >=
// |fast - sequential|; the selection kernel then certifies each token from
// these (route_cert.h): a token whose top K, so widened, is strictly
// separated keeps its fast logits, which select the reference's experts in
// the reference's order; for the others only the rows that could reach the
// top K are summed again in the reference's order.  Indices are exact either
// way; the weights come from the fast logits (within the layer tolerance).
//
// k_route_fast: grid (ceil((E + 1) / NR), ceil(T / TT)); workgroup (b, g)
// takes router rows NR b .. NR b + NR - 1 (row E: the fp16 shared gate,
// widened; its fast sums are the shared-gate scores) for tokens TT g ..
// TT g + TT - 1, thread i the L = H / 256
// consecutive columns [L i, L i + L) of every token: a fused multiply-add
// chain gives the chunk sum p and a = sum |w x|; an inclusive scan of p over
// the threads (in column order) gives every chunk's exact prefix P_i to
// within gamma_{L+10} A, and the last prefix is the fast logit F.
//
// Radius.  With q_k = fl(w_k x_k), s*_k the reference's partial sums and S_k
// the exact ones (A = sum |w_k x_k|, n = H):
//   |s*_n - sum q| <= u sum |s*_k|,  |sum q - S_n| <= u A (+ n 2^-150),
//   sum |s*_k| <= sum |S_k| + n gamma_n A,
//   sum over chunk i of |S_k| <= L (|S_{Li}| + A_i),
//   |S_{Li}| <= |P_i| + gamma_{L+10} A,  |F - S_n| <= gamma_{L+10} A,
// so R = u (L SP + c A) with SP = sum_i |P_i| (exclusive prefixes) and
// c = 2 L + 12 + n^2 u (the gamma terms for n <= 2048, L <= 8), widened by
// 2^-10 for the fp32 evaluation and by 1e-37 for underflow.
constexpr int CF_TT = 16;        // tokens per workgroup at most (TT)
constexpr int CF_THREADS = 256;  // threads per router row
constexpr int CF_WAVES = CF_THREADS / WAVE;
constexpr int CF_MAX_T = 32;     // tokens per call (the small-batch path's limit)
constexpr int CF_MAX_K = 16;

template <int CTRL, int ROWS>
__device__ __forceinline__ float cf_dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF,
                                                                 true));
}

// Inclusive prefix sum over the wave in lane order: row_shr 1, 2, 4, 8
// inside the 16-lane rows (lanes without a source add 0), then each row's
// total into the rows after it (row_bcast 15 and 31).
__device__ __forceinline__ float cf_wave_scan(float v)
{
    v += cf_dpp<0x111, 0xF>(v);
    v += cf_dpp<0x112, 0xF>(v);
    v += cf_dpp<0x114, 0xF>(v);
    v += cf_dpp<0x118, 0xF>(v);
    v += cf_dpp<0x142, 0xA>(v);
    v += cf_dpp<0x143, 0xC>(v);
    return v;
}

template <int L, int TT, int NR>
__global__ __launch_bounds__(CF_THREADS, 2) void k_route_fast(const float *__restrict__ router,
                                                             const uint16_t *__restrict__ shg, int has_shg,
                                                             const float *__restrict__ x, float *__restrict__ logits,
                                                             float *__restrict__ radii, float *__restrict__ gsh,
                                                             int H, int E, int T, float coef_a,
                                                             uint8_t *__restrict__ xq)
{
    static_assert(L % 4 == 0 && L <= 8 && TT <= CF_TT && NR * TT <= CF_THREADS, "columns, tokens, rows");
    __shared__ float s_tot[NR][TT][CF_WAVES], s_sp[NR][TT][CF_WAVES], s_a[NR][TT][CF_WAVES];
    const int tid = (int)threadIdx.x, wv = tid / WAVE, lane = lane_id();
    const int r0 = NR * (int)blockIdx.x, t0 = (int)blockIdx.y * TT;
    const int nt = T - t0 < TT ? T - t0 : TT;
    const int c0 = L * tid;
    // every row's columns and the gate's are read (rows past E read row 0;
    // shg points at readable memory of H halves either way), so no load
    // waits on a branch
    float4 rv[NR][L / 4];
    uint2 hv[L / 4];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const int r = r0 + n < E ? r0 + n : 0;
#pragma unroll
        for (int j = 0; j < L / 4; j++) rv[n][j] = reinterpret_cast<const float4 *>(router + (size_t)r * H + c0)[j];
    }
#pragma unroll
    for (int j = 0; j < L / 4; j++) hv[j] = reinterpret_cast<const uint2 *>(shg + c0)[j];
    // every token's columns requested at once (positions past the last
    // token read the last token again and are not stored)
    float4 xv[TT][L / 4];
#pragma unroll
    for (int t = 0; t < TT; t++) {
        const float *xt = x + (size_t)(t0 + (t < nt ? t : nt - 1)) * H + c0;
#pragma unroll
        for (int j = 0; j < L / 4; j++) xv[t][j] = reinterpret_cast<const float4 *>(xt)[j];
    }
    // with xq (H = 2048 only): workgroup b < nt also writes token t0 + b's
    // activations in the small-batch gate/up kernel's fixed-point form
    if constexpr (L == 8) {
        if (xq && (int)blockIdx.x < nt) {
#pragma unroll
            for (int t = 0; t < TT; t++)
                if (t == (int)blockIdx.x) {
                    const float v[8] = {xv[t][0].x, xv[t][0].y, xv[t][0].z, xv[t][0].w,
                                        xv[t][1].x, xv[t][1].y, xv[t][1].z, xv[t][1].w};
                    xq16_store(v, tid, xq + (size_t)(t0 + t) * XQ_TOKEN_BYTES);
                }
        }
    }
    float inc[NR][TT], a[NR][TT];
#pragma unroll
    for (int n = 0; n < NR; n++) {
        const bool gate = r0 + n == E, hz = gate && !has_shg;
        float w[L];
#pragma unroll
        for (int j = 0; j < L / 4; j++) {
            w[4 * j] = gate ? (hz ? 0.f : h2f(hv[j].x)) : rv[n][j].x;
            w[4 * j + 1] = gate ? (hz ? 0.f : h2f(hv[j].x >> 16)) : rv[n][j].y;
            w[4 * j + 2] = gate ? (hz ? 0.f : h2f(hv[j].y)) : rv[n][j].z;
            w[4 * j + 3] = gate ? (hz ? 0.f : h2f(hv[j].y >> 16)) : rv[n][j].w;
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float p = 0.f, aa = 0.f;
#pragma unroll
            for (int j = 0; j < L / 4; j++) {
                p = fmaf(w[4 * j], xv[t][j].x, p);
                p = fmaf(w[4 * j + 1], xv[t][j].y, p);
                p = fmaf(w[4 * j + 2], xv[t][j].z, p);
                p = fmaf(w[4 * j + 3], xv[t][j].w, p);
                aa = fmaf(fabsf(w[4 * j]), fabsf(xv[t][j].x), aa);
                aa = fmaf(fabsf(w[4 * j + 1]), fabsf(xv[t][j].y), aa);
                aa = fmaf(fabsf(w[4 * j + 2]), fabsf(xv[t][j].z), aa);
                aa = fmaf(fabsf(w[4 * j + 3]), fabsf(xv[t][j].w), aa);
            }
            inc[n][t] = cf_wave_scan(p);  // inclusive prefix of p in the wave
            a[n][t] = aa;
            if (lane == WAVE - 1) s_tot[n][t][wv] = inc[n][t];
        }
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NR; n++) {
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float off = 0.f;  // the earlier waves' totals, in order
#pragma unroll
            for (int u = 0; u < CF_WAVES - 1; u++)
                if (u < wv) off += s_tot[n][t][u];
            // exclusive prefix P_i of this thread's chunk: the previous
            // lane's inclusive prefix (wave_shr 1; lane 0 reads 0) after the
            // waves before
            const float excl = off + cf_dpp<0x138, 0xF>(inc[n][t]);
            const float sp = wave_sum(fabsf(excl)), sa = wave_sum(a[n][t]);
            if (lane == 0) {
                s_sp[n][t][wv] = sp;
                s_a[n][t][wv] = sa;
            }
        }
    }
    __syncthreads();
    if (tid < NR * TT) {
        const int n = tid / TT, t = tid % TT, r = r0 + n;
        float f = 0.f, sp = 0.f, aa = 0.f;
#pragma unroll
        for (int u = 0; u < CF_WAVES; u++) {
            f += s_tot[n][t][u];
            sp += s_sp[n][t][u];
            aa += s_a[n][t][u];
        }
        if (t < nt && r == E) {
            gsh[t0 + t] = has_shg ? f : 0.f;
        } else if (t < nt && r < E) {
            logits[(size_t)(t0 + t) * E + r] = f;
            radii[(size_t)(t0 + t) * E + r] = (1.0f + 1.0f / 1024) * CERT_U * ((float)L * sp + coef_a * aa) + 1e-37f;
        }
    }
}

// One wave per token: softmax / top-k / renormalisation with the host's
// arithmetic on the logits of k_route_seq.
template <int MAXV>
__global__ __launch_bounds__(WAVE) void k_topk_exact(const float *__restrict__ logits, int E, int K,
                                                     int32_t *__restrict__ idx, float *__restrict__ w)
{
    __shared__ __attribute__((aligned(16))) float s_e[WAVE * MAXV];
    const int t = (int)blockIdx.x;
    int ik;
    float wk;
    topk_wave_exact<MAXV>(logits + (size_t)t * E, E, K, s_e, ik, wk);
    if (lane_id() < K) {
        idx[(size_t)t * K + lane_id()] = ik;
        w[(size_t)t * K + lane_id()] = wk;
    }
}

} // namespace

// Router rows per wave: one while the grid has at most two workgroups a CU
// (64 KB of LDS each, so both are resident and the latency of a lane's sum
// is the kernel's time), two beyond, where two rows sharing each activation
// read halve the LDS reads per product.
int bread_route_rows_per_wave(int T, int E)
{
    const int tiles = (T + RS_TT - 1) / RS_TT;
    return E < 2 || (size_t)tiles * ((E + RS_WAVES - 1) / RS_WAVES) <= 512 ? 1 : 2;
}

int bread_launch_route_logits(const float *router, const uint16_t *shg, const float *x, float *logits, float *gsh,
                              int H, int E, int T, bool shg_row, hipStream_t st)
{
    BREAD_REQUIRE(H % RS_CJ == 0, BREAD_ERR_SHAPE, "hidden must be a multiple of 128");
    const int ne = bread_route_rows_per_wave(T, E);
    const dim3 grid((E + RS_WAVES * ne - 1) / (RS_WAVES * ne) + (shg_row ? 1 : 0), (T + RS_TT - 1) / RS_TT);
    if (ne == 1)
        hipLaunchKernelGGL(k_route_seq<1>, grid, dim3(RS_WAVES * WAVE), 0, st, router, shg, x, logits, gsh, H, E, T,
                           shg_row ? 1 : 0);
    else
        hipLaunchKernelGGL(k_route_seq<2>, grid, dim3(RS_WAVES * WAVE), 0, st, router, shg, x, logits, gsh, H, E, T,
                           shg_row ? 1 : 0);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

// Certified fast routing of T <= CF_MAX_T tokens (see k_route_fast); false
// if the shape does not allow it (the caller then runs
// bread_launch_route_logits).  The radii live in c->h, which the layer's
// gate/up kernels only write afterwards.
bool bread_route_certified_ok(const bread_moe_ctx_t *c, int T)
{
    const bread_moe_shape_t &s = c->shape;
    const int H = s.hidden, E = s.n_experts, K = s.top_k;
    const int Imax = s.expert_inter > s.shared_inter ? s.expert_inter : s.shared_inter;
    const size_t hcap = (size_t)c->max_tokens * (K + 1) * Imax;
    return T >= 1 && T <= CF_MAX_T && (H == 4 * CF_THREADS || H == 8 * CF_THREADS) && E <= 16 * WAVE && K >= 1 &&
           K <= CF_MAX_K && K <= E && (size_t)T * E <= hcap;
}

int bread_launch_route_fast(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, int T, float *gsh,
                            float *radii, uint8_t *xq, hipStream_t st)
{
    BREAD_REQUIRE(!xq || (c->shape.hidden == XQ_H && T <= CF_TT), BREAD_ERR_SHAPE,
                  "fixed-point activations need hidden 2048 and at most 16 tokens");
    const bread_moe_shape_t &s = c->shape;
    const int H = s.hidden, E = s.n_experts;
    const double u = 5.9604644775390625e-8, n = (double)H;
    const float coef_a = (float)(2.0 * (H / CF_THREADS) + 12.0 + n * n * u * 1.01);
    // the gate workgroup reads H halves at shg; without a gate it reads the
    // router's first row instead (and stores zeros)
    const uint16_t *g = L->shexp_gate ? L->shexp_gate : reinterpret_cast<const uint16_t *>(L->router);
    const int has_g = L->shexp_gate ? 1 : 0;
    // tokens per workgroup: the fewest of 4, 8, 16 that hold T; beyond 16
    // tokens each workgroup takes 4 router rows (rows share every activation
    // read: each row workgroup reads all of its tokens' columns)
    const int L1 = H / CF_THREADS;
    const int tt = T <= 4 ? 4 : (T <= 8 || T > 16 ? 8 : 16);
    const int nr = T > 16 ? 4 : 1;
    const dim3 grid((E + 1 + nr - 1) / nr, (T + tt - 1) / tt), block(CF_THREADS);
#define BREAD_ROUTE_FAST(LL, TTT, NRR)                                                                       \
    hipLaunchKernelGGL((k_route_fast<LL, TTT, NRR>), grid, block, 0, st, L->router, g, has_g, x, c->logits, radii, \
                       gsh, H, E, T, coef_a, xq)
    switch (L1 * 1000 + tt * 10 + nr) {
    case 4041: BREAD_ROUTE_FAST(4, 4, 1); break;
    case 4081: BREAD_ROUTE_FAST(4, 8, 1); break;
    case 4161: BREAD_ROUTE_FAST(4, 16, 1); break;
    case 4084: BREAD_ROUTE_FAST(4, 8, 4); break;
    case 8041: BREAD_ROUTE_FAST(8, 4, 1); break;
    case 8081: BREAD_ROUTE_FAST(8, 8, 1); break;
    case 8161: BREAD_ROUTE_FAST(8, 16, 1); break;
    case 8084: BREAD_ROUTE_FAST(8, 8, 4); break;
    default:
        return bread_fail(BREAD_ERR_SHAPE, "bread_launch_route_fast", "hidden must be 1024 or 2048");
    }
#undef BREAD_ROUTE_FAST
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

int bread_launch_topk(const float *logits, int E, int K, int T, int32_t *idx, float *w, hipStream_t st)
{
    const int mv = (E + WAVE - 1) / WAVE;
    if (mv <= 4)
        hipLaunchKernelGGL(k_topk_exact<4>, dim3(T), dim3(WAVE), 0, st, logits, E, K, idx, w);
    else
        hipLaunchKernelGGL(k_topk_exact<16>, dim3(T), dim3(WAVE), 0, st, logits, E, K, idx, w);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

int bread_launch_route(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, int T, int32_t *idx,
                       float *w, float *gsh, hipStream_t st)
{
    const bread_moe_shape_t &s = c->shape;
    bread_clear_stale_error();
    int rc = bread_launch_route_logits(L->router, L->shexp_gate, x, c->logits, gsh, s.hidden, s.n_experts, T, true, st);
    if (rc) return rc;
    return bread_launch_topk(c->logits, s.n_experts, s.top_k, T, idx, w, st);
}

// bread_route without a context: the logits live in this file's static
// device workspace, so nothing is allocated on any call.
extern "C" int bread_route_noalloc(const bread_moe_shape_t *shape, const bread_moe_layer_t *L, const float *x, int T,
                                   int32_t *idx, float *w, float *gsh, bread_stream_t stream)
{
    int rc = bread_validate_shape(shape);
    if (rc) return rc;
    BREAD_REQUIRE(x && idx && w && gsh, BREAD_ERR_ARG, "NULL input or output");
    BREAD_REQUIRE(T >= 0, BREAD_ERR_ARG, "n_tokens < 0");
    BREAD_REQUIRE((size_t)T * (size_t)shape->n_experts <= SCRATCH_FLOATS, BREAD_ERR_CAPACITY,
                  "n_tokens * n_experts exceeds the 1048576-float routing workspace");
    BREAD_REQUIRE(((uintptr_t)x & 15) == 0, BREAD_ERR_ALIGN, "x must be 16-byte aligned");
    rc = bread_validate_layer(shape, L);
    if (rc) return rc;
    if (T == 0) return BREAD_OK;
    float *logits = nullptr;
    rc = scratch_for_current_device(&logits);
    if (rc) return rc;
    const hipStream_t st = to_hip(stream);
    bread_clear_stale_error();
    rc = bread_launch_route_logits(L->router, L->shexp_gate, x, logits, gsh, shape->hidden, shape->n_experts, T,
                                   true, st);
    if (rc) return rc;
    return bread_launch_topk(logits, shape->n_experts, shape->top_k, T, idx, w, st);
}
