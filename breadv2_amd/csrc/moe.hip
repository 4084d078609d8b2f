// moe.hip — MoE context, routing, the multi-token path, RMSNorm and the
// C-ABI entry points of the MoE block.
//
// Multi-token path (any n_tokens, and the fallback for shapes the
// single-launch decode kernel is not built for): four stream-ordered kernels
//   router logits  -> softmax/top-k (one wave per token; route.hip, exact)
//   -> gate/up + SwiGLU (one wave per (token, slot, row))
//   -> down + combine (one wave per (token, row), slots in reference order).
// Slot 0 is the shared expert, slots 1..K the routed experts by rank.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <new>

#include "bread_internal.h"
#include "quant_dot.h"
#include "route_dev.h"

static int g_exit_on_error = 0;
static thread_local char g_last_error[256];

extern "C" void bread_set_exit_on_error(int enable)
{
    g_exit_on_error = enable;
}

extern "C" const char *bread_last_error(void)
{
    return g_last_error;
}

int bread_fail(int status, const char *where, const char *detail)
{
    snprintf(g_last_error, sizeof(g_last_error), "%s: %s (%s)", where, bread_status_str(status),
             detail ? detail : "");
    if (g_exit_on_error) {
        fprintf(stderr, "bread: %s: %s (%s)\n", where, bread_status_str(status), detail ? detail : "");
        exit(1);
    }
    return status;
}

extern "C" const char *bread_status_str(int status)
{
    switch (status) {
    case BREAD_OK: return "ok";
    case BREAD_ERR_ARG: return "invalid argument";
    case BREAD_ERR_QTYPE: return "unsupported qtype";
    case BREAD_ERR_SHAPE: return "unsupported shape";
    case BREAD_ERR_ALIGN: return "misaligned pointer";
    case BREAD_ERR_HIP: return "HIP runtime error";
    case BREAD_ERR_NOMEM: return "out of memory";
    case BREAD_ERR_CAPACITY: return "more tokens than the context holds";
    case BREAD_ERR_DEVICE: return "device-side fault flagged by a kernel";
    case BREAD_ERR_FORMAT: return "malformed model file";
    }
    return "unknown status";
}

extern "C" void bread_moe_shape_default(bread_moe_shape_t *s)
{
    if (!s) return;
    s->hidden = 2048;       // bread.h: hidden_dim
    s->expert_inter = 512;  // bread.h: expert_inter
    s->shared_inter = 512;  // bread.h: shared_inter
    s->n_experts = 256;     // bread.h: num_experts
    s->top_k = 8;           // bread.h: top_k
    s->rms_eps = 1e-6f;     // bread.h:68
}

int bread_validate_shape(const bread_moe_shape_t *s)
{
    BREAD_REQUIRE(s, BREAD_ERR_ARG, "NULL shape");
    BREAD_REQUIRE(s->hidden > 0 && s->expert_inter > 0 && s->shared_inter > 0 && s->n_experts > 0 &&
                      s->top_k > 0,
                  BREAD_ERR_ARG, "shape fields must be positive");
    BREAD_REQUIRE(s->top_k <= s->n_experts, BREAD_ERR_ARG, "top_k > n_experts");
    BREAD_REQUIRE(s->hidden % QK == 0 && s->expert_inter % QK == 0 && s->shared_inter % QK == 0,
                  BREAD_ERR_SHAPE, "hidden and intermediate sizes must be multiples of 256");
    BREAD_REQUIRE(s->n_experts <= 1024, BREAD_ERR_SHAPE, "n_experts > 1024");
    BREAD_REQUIRE(s->top_k <= 32, BREAD_ERR_SHAPE, "top_k > 32");
    return BREAD_OK;
}

int bread_validate_layer(const bread_moe_shape_t *s, const bread_moe_layer_t *L)
{
    BREAD_REQUIRE(L, BREAD_ERR_ARG, "NULL layer");
    BREAD_REQUIRE(L->gate_exps && L->up_exps && L->down_exps && L->gate_shexp && L->up_shexp &&
                      L->down_shexp && L->router,
                  BREAD_ERR_ARG, "NULL weight pointer in layer");
    // per tensor: pointer, expert stride (0: the shared expert), type
    const struct {
        const void *p;
        uint64_t stride;
        int type;
    } ts[6] = {{L->gate_exps, L->gate_expert_bytes, L->gate_type}, {L->up_exps, L->up_expert_bytes, L->up_type},
               {L->down_exps, L->down_expert_bytes, L->down_type}, {L->gate_shexp, 0, L->gate_shexp_type},
               {L->up_shexp, 0, L->up_shexp_type},                 {L->down_shexp, 0, L->down_shexp_type}};
    for (const auto &t : ts)
        BREAD_REQUIRE(bread_expert_qtype(t.type), BREAD_ERR_QTYPE, "expert tensors must be Q4_K or Q6_K");
    const int H = s->hidden, I = s->expert_inter;
    BREAD_REQUIRE(L->gate_expert_bytes >= (uint64_t)I * bread_expert_row_bytes(L->gate_type, H) &&
                      L->up_expert_bytes >= (uint64_t)I * bread_expert_row_bytes(L->up_type, H) &&
                      L->down_expert_bytes >= (uint64_t)H * bread_expert_row_bytes(L->down_type, I),
                  BREAD_ERR_SHAPE, "expert stride smaller than one expert");
    // Q4_K superblocks are read in 16-byte units, Q6_K ones in 4-byte units
    for (const auto &t : ts)
        BREAD_REQUIRE((((uintptr_t)t.p | t.stride) & (t.type == BREAD_QTYPE_Q4_K ? 15u : 3u)) == 0, BREAD_ERR_ALIGN,
                      "Q4_K tensors and strides must be 16-byte aligned, Q6_K ones 4-byte aligned");
    BREAD_REQUIRE(((uintptr_t)L->router & 15) == 0, BREAD_ERR_ALIGN, "router must be 16-byte aligned");
    BREAD_REQUIRE(((uintptr_t)L->shexp_gate & 7) == 0, BREAD_ERR_ALIGN, "shexp_gate must be 8-byte aligned");
    return BREAD_OK;
}

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------

extern "C" int bread_moe_ctx_create(const bread_moe_shape_t *shape, int max_tokens, bread_moe_ctx_t **out)
{
    int rc = bread_validate_shape(shape);
    if (rc) return rc;
    BREAD_REQUIRE(out && max_tokens > 0, BREAD_ERR_ARG, "out must be non-NULL and max_tokens > 0");
    *out = nullptr;
    bread_moe_ctx_t *c = new (std::nothrow) bread_moe_ctx_t();
    BREAD_REQUIRE(c, BREAD_ERR_NOMEM, "host allocation");
    c->shape = *shape;
    c->max_tokens = max_tokens;
    c->max_layers = 256;
    hipError_t e = hipGetDevice(&c->device);
    const int E = shape->n_experts, K = shape->top_k;
    const int Imax = shape->expert_inter > shape->shared_inter ? shape->expert_inter : shape->shared_inter;
    const size_t T = (size_t)max_tokens;
    if (e == hipSuccess) e = hipMalloc((void **)&c->logits, (T * E + E + 1) * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->idx, T * K * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&c->w, T * K * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->gsh, T * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->h, T * (K + 1) * Imax * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->x32, T * shape->hidden * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->h32, T * shape->hidden * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->tlogits, bread_decode_tlogit_words() * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc((void **)&c->xbuf, bread_decode_xbuf_floats() * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->hbuf, bread_decode_hbuf_floats() * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&c->dsync, sizeof(bread_decode_sync));
    if (e == hipSuccess && bread_decode_reset(c) != BREAD_OK) e = hipErrorUnknown;
    if (e == hipSuccess) e = hipMalloc(&c->d_layers, (size_t)c->max_layers * bread_decode_layer_record_bytes());
    if (e == hipSuccess) {
        c->h_layers = calloc((size_t)c->max_layers, bread_decode_layer_record_bytes());
        if (!c->h_layers) e = hipErrorOutOfMemory;
    }
    if (e == hipSuccess && bread_decode_max_blocks(&c->decode_max_blocks) != BREAD_OK) e = hipErrorUnknown;
    if (e == hipSuccess) {
        const int grc = bread_grouped_alloc(c);
        if (grc != BREAD_OK) e = grc == BREAD_ERR_NOMEM ? hipErrorOutOfMemory : hipErrorUnknown;
    }
    if (e == hipSuccess) {
        const int src = bread_small_alloc(c);
        if (src != BREAD_OK) e = src == BREAD_ERR_NOMEM ? hipErrorOutOfMemory : hipErrorUnknown;
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        bread_moe_ctx_destroy(c);
        return bread_fail(e == hipErrorOutOfMemory ? BREAD_ERR_NOMEM : BREAD_ERR_HIP, "bread_moe_ctx_create",
                          hipGetErrorString(e));
    }
    *out = c;
    return BREAD_OK;
}

extern "C" int bread_moe_ctx_destroy(bread_moe_ctx_t *c)
{
    if (!c) return BREAD_OK;
    (void)hipFree(c->logits);
    (void)hipFree(c->idx);
    (void)hipFree(c->w);
    (void)hipFree(c->gsh);
    (void)hipFree(c->h);
    (void)hipFree(c->x32);
    (void)hipFree(c->h32);
    (void)hipFree(c->tlogits);
    (void)hipFree(c->xbuf);
    (void)hipFree(c->hbuf);
    (void)hipFree(c->dsync);
    (void)hipFree(c->d_layers);
    bread_grouped_free(c);
    bread_small_free(c);
    free(c->h_layers);
    delete c;
    return BREAD_OK;
}

extern "C" int bread_moe_ctx_check(bread_moe_ctx_t *c, int *device_error)
{
    BREAD_REQUIRE(c, BREAD_ERR_ARG, "NULL context");
    BREAD_HIP(hipStreamSynchronize(c->last_stream));
    uint32_t err = 0;
    BREAD_HIP(hipMemcpy(&err, &c->dsync->error.v, sizeof(err), hipMemcpyDeviceToHost));
    if (device_error) *device_error = (int)err;
    if (err) {
        // a launch that gave up waiting may have left counters half-way: start
        // clean, counters, tags and epoch together
        if (bread_decode_reset(c) != BREAD_OK) return BREAD_ERR_HIP;
        BREAD_HIP(hipDeviceSynchronize());
        return bread_fail(BREAD_ERR_DEVICE, "bread_moe_ctx_check", "a kernel flagged an error");
    }
    return BREAD_OK;
}

extern "C" int bread_moe_ctx_route_stats(bread_moe_ctx_t *c, uint64_t *counts, int n, int reset)
{
    BREAD_REQUIRE(c && (counts || n == 0), BREAD_ERR_ARG, "NULL context or counts");
    BREAD_REQUIRE(n >= 0 && n <= BREAD_RSTAT_N, BREAD_ERR_ARG, "n outside [0, 8]");
    BREAD_HIP(hipStreamSynchronize(c->last_stream));
    uint32_t v[BREAD_RSTAT_N];
    BREAD_HIP(hipMemcpy(v, c->dsync->rstat.v, sizeof(v), hipMemcpyDeviceToHost));
    for (int i = 0; i < n; i++) counts[i] = v[i];
    if (reset) BREAD_HIP(hipMemset(c->dsync->rstat.v, 0, sizeof(v)));
    return BREAD_OK;
}

extern "C" int bread_moe_ctx_set_path(bread_moe_ctx_t *c, int path)
{
    BREAD_REQUIRE(c, BREAD_ERR_ARG, "NULL context");
    BREAD_REQUIRE(path >= BREAD_PATH_AUTO && path <= BREAD_PATH_SMALL, BREAD_ERR_ARG, "unknown path");
    c->path = path;
    return BREAD_OK;
}

extern "C" int bread_moe_ctx_set_spin_limit(bread_moe_ctx_t *c, long long n_sleeps)
{
    BREAD_REQUIRE(c, BREAD_ERR_ARG, "NULL context");
    BREAD_REQUIRE(n_sleeps <= (1ll << 24), BREAD_ERR_ARG, "spin limit above 2^24 sleeps");
    c->spin_limit = n_sleeps < 0 ? -1 : n_sleeps;
    return BREAD_OK;
}

extern "C" int bread_moe_ctx_set_trace(bread_moe_ctx_t *c, uint64_t *d_buf, size_t n_words, int *grid_out)
{
    BREAD_REQUIRE(c, BREAD_ERR_ARG, "NULL context");
    c->trace = d_buf;
    c->trace_words = d_buf ? n_words : 0;
    if (grid_out) *grid_out = bread_decode_grid(c->shape);
    return BREAD_OK;
}

// ---------------------------------------------------------------------------
// Per-token expert kernels (routing: route.hip)
// ---------------------------------------------------------------------------

// One wave's partial dot of a Q4_K or Q6_K row (nb superblocks) with x.
__device__ __forceinline__ float kq_row_partial(int type, const uint8_t *row, int nb, const float *x, int lane)
{
    return type == BREAD_QTYPE_Q4_K ? q4k_row_partial(row, nb, x, lane) : q6k_row_partial(row, nb, x, lane);
}

// Expert of an index the caller handed in: clamped to [0, E) so that no
// load leaves the tensor, with BREAD_DEV_ERR_INDEX set when it was outside.
__device__ __forceinline__ int checked_expert(int e, int E, uint32_t *err)
{
    if (e >= 0 && e < E) return e;
    __hip_atomic_fetch_or(err, BREAD_DEV_ERR_INDEX, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return e < 0 ? 0 : E - 1;
}

// One wave per (token, slot, row): gate and up rows, then SwiGLU.  Each
// tensor has its own type (Q4_K or Q6_K), as in the reference's
// cpu_tensor_matvec dispatch (one_layer.cu:1465-1468).  Slot 0 (the shared
// expert) only when `shared`.
__global__ __launch_bounds__(256) void k_gateup(bread_moe_layer_t L, const float *__restrict__ x,
                                                const int32_t *__restrict__ idx, float *__restrict__ h, int H,
                                                int I, int Ish, int K, int T, int E, int shared,
                                                uint32_t *__restrict__ err)
{
    const int Imax = I > Ish ? I : Ish;
    const int64_t v = (int64_t)((blockIdx.x * (uint64_t)blockDim.x + threadIdx.x) / WAVE);
    const int64_t per_tok = (int64_t)(K + 1) * Imax;
    if (v >= per_tok * T) return;
    const int t = (int)(v / per_tok);
    const int slot = (int)((v % per_tok) / Imax);
    const int r = (int)(v % Imax);
    if (r >= (slot ? I : Ish) || (slot == 0 && !shared)) return;
    const uint8_t *g, *u;
    int gt, ut;
    if (slot == 0) {
        g = (const uint8_t *)L.gate_shexp;
        u = (const uint8_t *)L.up_shexp;
        gt = L.gate_shexp_type;
        ut = L.up_shexp_type;
    } else {
        const int e = checked_expert(idx[(size_t)t * K + slot - 1], E, err);
        g = (const uint8_t *)L.gate_exps + (uint64_t)e * L.gate_expert_bytes;
        u = (const uint8_t *)L.up_exps + (uint64_t)e * L.up_expert_bytes;
        gt = L.gate_type;
        ut = L.up_type;
    }
    const float *xt = x + (size_t)t * H;
    const int lane = lane_id();
    const float gv = wave_sum(kq_row_partial(gt, g + r * bread_expert_row_bytes(gt, H), H / QK, xt, lane));
    const float uv = wave_sum(kq_row_partial(ut, u + r * bread_expert_row_bytes(ut, H), H / QK, xt, lane));
    if (lane == 0) h[((size_t)t * (K + 1) + slot) * Imax + r] = silu_mul(gv, uv);
}

// One wave per (token, output row): down rows of every slot, combined in the
// reference order (one_layer.cu:1447-1469): the shared expert (when
// `shared`), then the routed experts by rank.
__global__ __launch_bounds__(256) void k_down(bread_moe_layer_t L, const int32_t *__restrict__ idx,
                                              const float *__restrict__ w, const float *__restrict__ gsh,
                                              const float *__restrict__ h, float *__restrict__ hidden, int H,
                                              int I, int Ish, int K, int T, int E, int shared,
                                              uint32_t *__restrict__ err)
{
    const int Imax = I > Ish ? I : Ish;
    const int64_t v = (int64_t)((blockIdx.x * (uint64_t)blockDim.x + threadIdx.x) / WAVE);
    if (v >= (int64_t)H * T) return;
    const int t = (int)(v / H);
    const int r = (int)(v % H);
    const int lane = lane_id();
    const float *ht = h + (size_t)t * (K + 1) * Imax;
    const int st = L.down_shexp_type, dt = L.down_type;
    float acc = hidden[(size_t)t * H + r];
    if (shared) {
        const float sh = wave_sum(kq_row_partial(
            st, (const uint8_t *)L.down_shexp + (uint64_t)r * bread_expert_row_bytes(st, Ish), Ish / QK, ht, lane));
        acc += sigmoidf_ref(gsh[t]) * sh;
    }
    const uint64_t rb = bread_expert_row_bytes(dt, I);
    for (int k = 0; k < K; k++) {
        const int e = checked_expert(idx[(size_t)t * K + k], E, err);
        const uint8_t *d = (const uint8_t *)L.down_exps + (uint64_t)e * L.down_expert_bytes + r * rb;
        const float eo = wave_sum(kq_row_partial(dt, d, I / QK, ht + (size_t)(k + 1) * Imax, lane));
        acc += w[(size_t)t * K + k] * eo;
    }
    if (lane == 0) hidden[(size_t)t * H + r] = acc;
}

// fp32 RMSNorm, one 256-thread block per token (layer_ops.cu:203-212).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w,
                                                 float *__restrict__ out, int n, float eps)
{
    __shared__ float part[4];
    const float *xt = x + (size_t)blockIdx.x * n;
    float *ot = out + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(xt[i], xt[i], ss);
    ss = wave_sum(ss);
    if (lane_id() == 0) part[threadIdx.x / WAVE] = ss;
    __syncthreads();
    const float tot = part[0] + part[1] + part[2] + part[3];
    const float inv = 1.0f / sqrtf(tot / (float)n + eps);
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) ot[i] = xt[i] * inv * (w ? w[i] : 1.0f);
}

// The fp16 residual stream of one_layer_forward, in: per token, the fp32
// residual copy h32 = hidden and the MoE input x32.  With norm_w, x32 is the
// fp16-rounded post-attention RMSNorm output, also written to `normed` as
// one_layer.cu:1812-1815 writes d_normed2 (x * rms * w in that order,
// rms = 1/sqrt(mean(x^2) + eps)); without, `normed` is read.  H % 8 == 0.
__global__ __launch_bounds__(256) void k_f16_in(const uint16_t *__restrict__ hidden, uint16_t *__restrict__ normed,
                                                const float *__restrict__ norm_w, float *__restrict__ x32,
                                                float *__restrict__ h32, int H, float eps)
{
    __shared__ float part[4];
    const size_t base = (size_t)blockIdx.x * H;
    const uint4 *hv = reinterpret_cast<const uint4 *>(hidden + base);
    uint4 *nv = reinterpret_cast<uint4 *>(normed + base);
    float4 *xo = reinterpret_cast<float4 *>(x32 + base);
    float4 *ho = reinterpret_cast<float4 *>(h32 + base);
    const int n8 = H / 8;
    float inv = 1.0f;
    if (norm_w) {
        float ss = 0.f;
        for (int v = threadIdx.x; v < n8; v += 256) {
            const uint4 q = hv[v];
            const uint32_t p[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float a = h2f(p[k]), b = h2f(p[k] >> 16);
                ss = fmaf(a, a, ss);
                ss = fmaf(b, b, ss);
            }
        }
        ss = wave_sum(ss);
        if (lane_id() == 0) part[threadIdx.x / WAVE] = ss;
        __syncthreads();
        inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)H + eps);
    }
    for (int v = threadIdx.x; v < n8; v += 256) {
        const uint4 q = hv[v];
        const uint32_t p[4] = {q.x, q.y, q.z, q.w};
        float hf[8], xf[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            hf[2 * k] = h2f(p[k]);
            hf[2 * k + 1] = h2f(p[k] >> 16);
        }
        uint4 n;
        if (norm_w) {
            const float4 w0 = reinterpret_cast<const float4 *>(norm_w)[2 * v];
            const float4 w1 = reinterpret_cast<const float4 *>(norm_w)[2 * v + 1];
            const float wf[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo = f2h(hf[2 * k] * inv * wf[2 * k]);
                const uint32_t hi = f2h(hf[2 * k + 1] * inv * wf[2 * k + 1]);
                o[k] = lo | (hi << 16);
            }
            n = make_uint4(o[0], o[1], o[2], o[3]);
            nv[v] = n;
        } else {
            n = nv[v];
        }
        const uint32_t np[4] = {n.x, n.y, n.z, n.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            xf[2 * k] = h2f(np[k]);
            xf[2 * k + 1] = h2f(np[k] >> 16);
        }
        xo[2 * v] = make_float4(xf[0], xf[1], xf[2], xf[3]);
        xo[2 * v + 1] = make_float4(xf[4], xf[5], xf[6], xf[7]);
        ho[2 * v] = make_float4(hf[0], hf[1], hf[2], hf[3]);
        ho[2 * v + 1] = make_float4(hf[4], hf[5], hf[6], hf[7]);
    }
}

// fp16 bits -> fp32, 8 values a thread (exact): route_layer's widening of
// d_normed2 (vram_half_to_cpu_float, one_layer.cu:961) on the device.
__global__ __launch_bounds__(256) void k_widen_f16(const uint16_t *__restrict__ in, float *__restrict__ out,
                                                   size_t n8)
{
    const size_t v = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (v >= n8) return;
    const uint4 q = reinterpret_cast<const uint4 *>(in)[v];
    reinterpret_cast<float4 *>(out)[2 * v] = make_float4(h2f(q.x), h2f(q.x >> 16), h2f(q.y), h2f(q.y >> 16));
    reinterpret_cast<float4 *>(out)[2 * v + 1] = make_float4(h2f(q.z), h2f(q.z >> 16), h2f(q.w), h2f(q.w >> 16));
}

// ... and out: hidden = fp16(h32), round to nearest even, 8 values a thread.
__global__ __launch_bounds__(256) void k_f16_out(const float *__restrict__ h32, uint16_t *__restrict__ hidden,
                                                 size_t n8)
{
    const size_t v = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (v >= n8) return;
    const float4 a = reinterpret_cast<const float4 *>(h32)[2 * v];
    const float4 b = reinterpret_cast<const float4 *>(h32)[2 * v + 1];
    uint4 o;
    o.x = f2h(a.x) | ((uint32_t)f2h(a.y) << 16);
    o.y = f2h(a.z) | ((uint32_t)f2h(a.w) << 16);
    o.z = f2h(b.x) | ((uint32_t)f2h(b.y) << 16);
    o.w = f2h(b.z) | ((uint32_t)f2h(b.w) << 16);
    reinterpret_cast<uint4 *>(hidden)[v] = o;
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

int bread_launch_moe_multi(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, float *hidden, int T,
                           hipStream_t st)
{
    const bread_moe_shape_t &s = c->shape;
    int rc = bread_launch_route(c, L, x, T, c->idx, c->w, c->gsh, st);
    if (rc) return rc;
    const int Imax = s.expert_inter > s.shared_inter ? s.expert_inter : s.shared_inter;
    const uint64_t gu_waves = (uint64_t)T * (s.top_k + 1) * Imax;
    hipLaunchKernelGGL(k_gateup, dim3((unsigned)((gu_waves + 3) / 4)), dim3(256), 0, st, *L, x, c->idx, c->h,
                       s.hidden, s.expert_inter, s.shared_inter, s.top_k, T, s.n_experts, 1, &c->dsync->error.v);
    BREAD_HIP(hipGetLastError());
    const uint64_t dn_waves = (uint64_t)T * s.hidden;
    hipLaunchKernelGGL(k_down, dim3((unsigned)((dn_waves + 3) / 4)), dim3(256), 0, st, *L, c->idx, c->w, c->gsh,
                       c->h, hidden, s.hidden, s.expert_inter, s.shared_inter, s.top_k, T, s.n_experts, 1,
                       &c->dsync->error.v);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

// ---------------------------------------------------------------------------
// C-ABI entry points
// ---------------------------------------------------------------------------

static int check_tokens(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, int T)
{
    BREAD_REQUIRE(c && x, BREAD_ERR_ARG, "NULL context or input");
    BREAD_REQUIRE(T >= 0, BREAD_ERR_ARG, "n_tokens < 0");
    BREAD_REQUIRE(T <= c->max_tokens, BREAD_ERR_CAPACITY, "n_tokens > max_tokens of the context");
    BREAD_REQUIRE(((uintptr_t)x & 15) == 0, BREAD_ERR_ALIGN, "x must be 16-byte aligned");
    return bread_validate_layer(&c->shape, L);
}

extern "C" int bread_route(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, int T,
                           int32_t *idx, float *w, float *gsh, bread_stream_t stream)
{
    int rc = check_tokens(c, L, x, T);
    if (rc) return rc;
    BREAD_REQUIRE(idx && w && gsh, BREAD_ERR_ARG, "NULL output");
    if (T == 0) return BREAD_OK;
    c->last_stream = to_hip(stream);
    return bread_launch_route(c, L, x, T, idx, w, gsh, to_hip(stream));
}

extern "C" int bread_route_layer(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x,
                                 int *expert_indices, float *expert_weights, float *gsh_logit,
                                 bread_stream_t stream)
{
    BREAD_REQUIRE(expert_indices && expert_weights && gsh_logit, BREAD_ERR_ARG, "NULL host output");
    int rc = bread_route(c, L, x, 1, c ? c->idx : nullptr, c ? c->w : nullptr, c ? c->gsh : nullptr, stream);
    if (rc) return rc;
    hipStream_t st = to_hip(stream);
    const int K = c->shape.top_k;
    BREAD_HIP(hipMemcpyAsync(expert_indices, c->idx, K * sizeof(int32_t), hipMemcpyDeviceToHost, st));
    BREAD_HIP(hipMemcpyAsync(expert_weights, c->w, K * sizeof(float), hipMemcpyDeviceToHost, st));
    BREAD_HIP(hipMemcpyAsync(gsh_logit, c->gsh, sizeof(float), hipMemcpyDeviceToHost, st));
    BREAD_HIP(hipStreamSynchronize(st));
    return BREAD_OK;
}

extern "C" int bread_route_layer_f16(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const uint16_t *normed,
                                     int *expert_indices, float *expert_weights, float *gsh_logit,
                                     bread_stream_t stream)
{
    BREAD_REQUIRE(c && normed, BREAD_ERR_ARG, "NULL context or d_normed2");
    BREAD_REQUIRE(expert_indices && expert_weights && gsh_logit, BREAD_ERR_ARG, "NULL host output");
    BREAD_REQUIRE(((uintptr_t)normed & 15) == 0, BREAD_ERR_ALIGN, "d_normed2 must be 16-byte aligned");
    int rc = bread_validate_layer(&c->shape, L);
    if (rc) return rc;
    // x32 holds max_tokens >= 1 rows of H floats; H is a multiple of 256
    const size_t n8 = (size_t)c->shape.hidden / 8;
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_widen_f16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, to_hip(stream), normed,
                       c->x32, n8);
    BREAD_HIP(hipGetLastError());
    return bread_route_layer(c, L, c->x32, expert_indices, expert_weights, gsh_logit, stream);
}

// Up to this many tokens one decode-stack launch per token beats 40
// small-batch layers, measured on MI355X over 40 resident layers: 1597 /
// 2126 / 2680 us for 3 / 4 / 5 tokens one stack launch each, against
// 2271 / 2508 / 2610 us on the small-batch path (its exact router and
// selection cost ~27 us a layer).
extern "C" int bread_stack_loop_tokens(void)
{
    return 4;
}

extern "C" int bread_moe_forward(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, float *hidden,
                                 int T, int32_t *idx, float *w, float *gsh, bread_stream_t stream)
{
    int rc = check_tokens(c, L, x, T);
    if (rc) return rc;
    BREAD_REQUIRE(hidden, BREAD_ERR_ARG, "NULL hidden");
    if (T == 0) return BREAD_OK;
    hipStream_t st = to_hip(stream);
    c->last_stream = st;
    if (c->path == BREAD_PATH_DECODE || c->path == BREAD_PATH_GROUPED || c->path == BREAD_PATH_SMALL)
        BREAD_REQUIRE(bread_standard_qtypes(L), BREAD_ERR_QTYPE,
                      "the decode, small-batch and grouped kernels take Q4_K gate/up and Q6_K down "
                      "(BREAD_PATH_PER_TOKEN and BREAD_PATH_AUTO take any mix of Q4_K and Q6_K)");
    switch (c->path) {
    case BREAD_PATH_DECODE:
        BREAD_REQUIRE(T == 1, BREAD_ERR_SHAPE, "the decode path takes one token");
        rc = bread_launch_moe_decode(c, L, x, hidden, st);
        if (rc == BREAD_ERR_SHAPE) return bread_fail(rc, "bread_moe_forward", "shape not supported by the decode kernel");
        break;
    case BREAD_PATH_GROUPED:
        rc = bread_launch_moe_grouped(c, L, x, hidden, T, st);
        if (rc == BREAD_ERR_SHAPE) return bread_fail(rc, "bread_moe_forward", "shape not supported by the grouped path");
        break;
    case BREAD_PATH_PER_TOKEN:
        rc = bread_launch_moe_multi(c, L, x, hidden, T, st);
        break;
    case BREAD_PATH_SMALL:
        rc = bread_launch_moe_small(c, L, x, hidden, T, st);
        if (rc == BREAD_ERR_SHAPE) return bread_fail(rc, "bread_moe_forward", "shape not supported by the small-batch path");
        break;
    default:
        rc = (T == 1) ? bread_launch_moe_decode(c, L, x, hidden, st) : BREAD_ERR_SHAPE;
        if (rc == BREAD_ERR_SHAPE && T <= bread_small_auto_tokens()) rc = bread_launch_moe_small(c, L, x, hidden, T, st);
        if (rc == BREAD_ERR_SHAPE) rc = bread_launch_moe_grouped(c, L, x, hidden, T, st);
        if (rc == BREAD_ERR_SHAPE) rc = bread_launch_moe_multi(c, L, x, hidden, T, st);
    }
    if (rc) return rc;
    const int K = c->shape.top_k;
    if (idx) BREAD_HIP(hipMemcpyAsync(idx, c->idx, (size_t)T * K * sizeof(int32_t), hipMemcpyDeviceToDevice, st));
    if (w) BREAD_HIP(hipMemcpyAsync(w, c->w, (size_t)T * K * sizeof(float), hipMemcpyDeviceToDevice, st));
    if (gsh) BREAD_HIP(hipMemcpyAsync(gsh, c->gsh, (size_t)T * sizeof(float), hipMemcpyDeviceToDevice, st));
    return BREAD_OK;
}

// The routed experts with the caller's routing (the reference's expert-block
// harness, expert_bench.cu:123-151, and the routed loop of one_layer.cu:
// 1455-1470): per-token kernels without the shared slot.
extern "C" int bread_moe_expert_block(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x,
                                      float *hidden, int T, const int32_t *idx, const float *w,
                                      bread_stream_t stream)
{
    int rc = check_tokens(c, L, x, T);
    if (rc) return rc;
    BREAD_REQUIRE(hidden && idx && w, BREAD_ERR_ARG, "NULL hidden or routing");
    if (T == 0) return BREAD_OK;
    const hipStream_t st = to_hip(stream);
    c->last_stream = st;
    const bread_moe_shape_t &s = c->shape;
    const int Imax = s.expert_inter > s.shared_inter ? s.expert_inter : s.shared_inter;
    bread_clear_stale_error();
    const uint64_t gu_waves = (uint64_t)T * (s.top_k + 1) * Imax;
    hipLaunchKernelGGL(k_gateup, dim3((unsigned)((gu_waves + 3) / 4)), dim3(256), 0, st, *L, x, idx, c->h,
                       s.hidden, s.expert_inter, s.shared_inter, s.top_k, T, s.n_experts, 0, &c->dsync->error.v);
    BREAD_HIP(hipGetLastError());
    const uint64_t dn_waves = (uint64_t)T * s.hidden;
    hipLaunchKernelGGL(k_down, dim3((unsigned)((dn_waves + 3) / 4)), dim3(256), 0, st, *L, idx, w, c->gsh, c->h,
                       hidden, s.hidden, s.expert_inter, s.shared_inter, s.top_k, T, s.n_experts, 0,
                       &c->dsync->error.v);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

// The MoE block of one_layer_forward on its fp16 residual stream
// (one_layer.cu:1800-1986): norm in, bread_moe_forward in fp32, one rounding out.
extern "C" int bread_moe_forward_f16(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *norm_w,
                                     uint16_t *hidden, uint16_t *normed, int T, int32_t *idx, float *w,
                                     float *gsh, bread_stream_t stream)
{
    BREAD_REQUIRE(c && hidden && normed, BREAD_ERR_ARG, "NULL context, hidden or normed");
    BREAD_REQUIRE(T >= 0, BREAD_ERR_ARG, "n_tokens < 0");
    BREAD_REQUIRE(T <= c->max_tokens, BREAD_ERR_CAPACITY, "n_tokens > max_tokens of the context");
    BREAD_REQUIRE((((uintptr_t)hidden | (uintptr_t)normed | (uintptr_t)norm_w) & 15) == 0, BREAD_ERR_ALIGN,
                  "hidden, normed and norm_w must be 16-byte aligned");
    int rc = bread_validate_layer(&c->shape, L);
    if (rc) return rc;
    if (T == 0) return BREAD_OK;
    const int H = c->shape.hidden;
    hipStream_t st = to_hip(stream);
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_f16_in, dim3(T), dim3(256), 0, st, hidden, normed, norm_w, c->x32, c->h32, H,
                       c->shape.rms_eps);
    BREAD_HIP(hipGetLastError());
    rc = bread_moe_forward(c, L, c->x32, c->h32, T, idx, w, gsh, stream);
    if (rc) return rc;
    const size_t n8 = (size_t)T * H / 8;
    hipLaunchKernelGGL(k_f16_out, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, c->h32, hidden, n8);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

extern "C" int bread_moe_decode_layers(bread_moe_ctx_t *c, const bread_moe_layer_t *layers, int n,
                                       float *hidden, int32_t *idx, float *w, float *gsh, bread_stream_t stream)
{
    BREAD_REQUIRE(c && layers && hidden, BREAD_ERR_ARG, "NULL context, layers or hidden");
    BREAD_REQUIRE(n >= 0, BREAD_ERR_ARG, "n_layers < 0");
    BREAD_REQUIRE(((uintptr_t)hidden & 15) == 0, BREAD_ERR_ALIGN, "hidden must be 16-byte aligned");
    for (int l = 0; l < n; l++) {
        int rc = bread_validate_layer(&c->shape, &layers[l]);
        if (rc) return rc;
        BREAD_REQUIRE(((uintptr_t)layers[l].post_norm_w & 15) == 0, BREAD_ERR_ALIGN,
                      "post_norm_w must be 16-byte aligned");
    }
    if (n == 0) return BREAD_OK;
    hipStream_t st = to_hip(stream);
    c->last_stream = st;
    int rc = bread_launch_decode_runs(c, layers, n, hidden, idx, w, gsh, st, 1);
    if (rc == BREAD_ERR_SHAPE) return bread_fail(rc, "bread_moe_decode_layers", "shape not supported by the decode kernel");
    if (rc == BREAD_ERR_CAPACITY)
        return bread_fail(rc, "bread_moe_decode_layers", "a run of decode-kernel layers longer than the context's layer table");
    return rc;
}

extern "C" int bread_rmsnorm_f32(const float *x, const float *w, float *out, int n, int T, float eps,
                                 bread_stream_t stream)
{
    BREAD_REQUIRE(x && out, BREAD_ERR_ARG, "NULL pointer");
    BREAD_REQUIRE(n > 0 && T >= 0, BREAD_ERR_ARG, "n must be > 0 and n_tokens >= 0");
    if (T == 0) return BREAD_OK;
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(256), 0, to_hip(stream), x, w, out, n, eps);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}
