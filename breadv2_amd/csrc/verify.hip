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

#include "bread_device.h"
#include "bread_internal.h"

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
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(xt[i], xt[i], ss);
    ss = wave_sum(ss);
    if (lane_id() == 0) part[threadIdx.x / WAVE] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xt[i] * inv * (w ? w[i] : 1.0f);
        if constexpr (sizeof(OT) == 2) ot[i] = f2h(v);
        else ot[i] = v;
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
