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
