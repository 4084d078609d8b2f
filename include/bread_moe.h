/* bread_moe.h — C ABI of the MI355X (gfx950) MoE feed-forward hot path.
 *
 * Drop-in for the reference's (arahe-dev/breadv2) MoE FFN path:
 *   - bread_matvec            replaces kernels.cu:289 (same name, argument
 *                             order and meaning; returns a status instead of
 *                             exit(1), kernels.cu:303-307)
 *   - bread_route_layer       replaces route_layer, one_layer.cu:937-992
 *   - bread_moe_forward       replaces the MoE block of one_layer_forward,
 *                             one_layer.cu:1800-1986 (GPU) and :1413-1471
 *                             (fp32 host order it reproduces)
 *   - bread_arena_*           replaces the expert residency of
 *                             weight_cache_load_experts, loader.c:628-693
 *
 * Every pointer argument named d_* or documented as "device" is a device
 * pointer; the caller owns it.  Every entry point is stream-ordered on the
 * given HIP stream (hipStream_t; NULL is the null stream) and returns a
 * bread_status_t.  Entry points that take a context are not reentrant for
 * the same context: two calls that overlap on one context race on its
 * scratch.  Use one context per stream.
 *
 * Weight layout is the native GGUF block layout, row-major, rows packed with
 * no padding: row stride = (cols / block_elems) * block_bytes
 * (gguf.c:60-95, 140-144).
 */
#ifndef BREAD_MOE_H
#define BREAD_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without the HIP headers: the same incomplete struct type. */
typedef struct ihipStream_t *bread_stream_t;

/* GGML type ids used on the path (gguf.h:31-37). */
#define BREAD_QTYPE_F32  0
#define BREAD_QTYPE_F16  1
#define BREAD_QTYPE_Q8_0 8
#define BREAD_QTYPE_Q4_K 12
#define BREAD_QTYPE_Q6_K 14

#define BREAD_QK_K            256 /* elements per K-quant superblock */
#define BREAD_Q4K_BLOCK_BYTES 144 /* d, dmin, 12 B scales, 128 B nibbles (kernels.cu:3-7) */
#define BREAD_Q6K_BLOCK_BYTES 210 /* 128 B ql, 64 B qh, 16 int8 sc, d (kernels.cu:9-13) */
#define BREAD_Q8_0_BLOCK_ELEMS 32
#define BREAD_Q8_0_BLOCK_BYTES 34 /* d, 32 int8 (kernels.cu:240-246) */

typedef enum {
    BREAD_OK = 0,
    BREAD_ERR_ARG = -1,        /* NULL pointer, negative size, bad shape field */
    BREAD_ERR_QTYPE = -2,      /* qtype not supported by this entry point */
    BREAD_ERR_SHAPE = -3,      /* cols not a multiple of the block size, etc. */
    BREAD_ERR_ALIGN = -4,      /* pointer alignment the kernels need is missing */
    BREAD_ERR_HIP = -5,        /* a HIP runtime call failed */
    BREAD_ERR_NOMEM = -6,      /* device or host allocation failed */
    BREAD_ERR_CAPACITY = -7,   /* more tokens than the context was created for */
    BREAD_ERR_DEVICE = -8,     /* a kernel reported a fault (see bread_moe_ctx_check) */
    BREAD_ERR_FORMAT = -9      /* a model file is malformed (bread_gguf_open) */
} bread_status_t;

/* Text for a status code (static storage). */
const char *bread_status_str(int status);

/* Where and why the last failing entry point on this thread failed,
 * including the HIP runtime's message for BREAD_ERR_HIP ("" if none). */
const char *bread_last_error(void);

/* When non-zero, every entry point that would return an error prints it and
 * calls exit(1), as the reference does (bread_utils.h:14-21,
 * kernels.cu:303-307).  Default 0. */
void bread_set_exit_on_error(int enable);

/* ------------------------------------------------------------------ */
/* Quantized matvec and dequant                                        */
/* ------------------------------------------------------------------ */

/* y[r] = sum_c dequant(W[r,c]) * x[c] for r < rows.  x and y are fp16 bits
 * (the reference's `half`), accumulation is fp32, y is rounded to nearest
 * fp16.  qtype is 12 (Q4_K), 14 (Q6_K) or 8 (Q8_0); cols must be a multiple
 * of 256 (K-quants) or 32 (Q8_0).  w must be 4-byte aligned and x 16-byte
 * aligned (BREAD_ERR_ALIGN otherwise).
 * Replaces kernels.cu:289-308 `void bread_matvec(void *w, half *x, half *y,
 * int rows, int cols, int qtype, cudaStream_t stream)`. */
int bread_matvec(const void *w, const uint16_t *x, uint16_t *y, int rows, int cols,
                 int qtype, bread_stream_t stream);

/* Same product with fp32 x and y (config 1 entry; the fp32 host path's
 * cpu_tensor_matvec, layer_ops.cu:169-189, on the device). */
int bread_matvec_f32(const void *w, const float *x, float *y, int rows, int cols,
                     int qtype, bread_stream_t stream);

/* Bit-exact dequant: out[r*cols + c] = the reference's fp32 value of W[r,c]
 * (dequant_q4k_cpu.c:90-172 with the subnormal-correct fp16 decode of
 * bread_utils.h:27-47; Q8_0 value = d*q, kernels.cu:246).  Same qtypes and
 * shape rules as bread_matvec. */
int bread_dequant_rows(const void *w, int qtype, int rows, int cols, float *out,
                       bread_stream_t stream);

/* ------------------------------------------------------------------ */
/* MoE layer                                                           */
/* ------------------------------------------------------------------ */

/* Model shape (bread.h:16-69 defaults: 2048, 512, 512, 256, 8, 1e-6). */
typedef struct {
    int hidden;        /* H */
    int expert_inter;  /* I: routed expert intermediate size */
    int shared_inter;  /* I_sh: shared expert intermediate size */
    int n_experts;     /* E */
    int top_k;         /* K */
    float rms_eps;
} bread_moe_shape_t;

void bread_moe_shape_default(bread_moe_shape_t *shape);

/* One layer's MoE weights, device pointers, native GGUF layout.
 * Routed expert e of a stacked tensor starts at base + e * expert_bytes, the
 * GGUF layout the reference slices (loader.h:35-47, loader.c:187-190); the
 * shared expert and router mirror wc_layer_t (loader.h:86-109) and the
 * tensors route_layer reads (one_layer.cu:964-980).
 * Types: each of the six expert tensors is BREAD_QTYPE_Q4_K or BREAD_QTYPE_Q6_K,
 * given per tensor as the reference records them (loader.c:191-193) and as its
 * fp32 path dispatches on them (one_layer.cu:1465-1468, layer_ops.cu:169-189).
 * Q4_K tensors and expert strides are 16-byte aligned, Q6_K ones 4-byte
 * aligned.  The decode, small-batch and grouped kernels take the mix the
 * reference GPU path hardcodes (gate/up Q4_K, down Q6_K, routed and shared,
 * one_layer.cu:1966-1977); any other mix runs on the per-token kernels.
 * router F32 [E][H]; shexp_gate F16 [H] or NULL (NULL means a zero logit,
 * sigmoid 0.5, as when the reference finds no tensor, one_layer.cu:974-976). */
typedef struct {
    const void *gate_exps;
    const void *up_exps;
    const void *down_exps;
    uint64_t gate_expert_bytes;
    uint64_t up_expert_bytes;
    uint64_t down_expert_bytes;
    int gate_type, up_type, down_type;
    const void *gate_shexp;
    const void *up_shexp;
    const void *down_shexp;
    int gate_shexp_type, up_shexp_type, down_shexp_type;
    const float *router;          /* ffn_gate_inp, fp32 [E][H] */
    const uint16_t *shexp_gate;   /* ffn_gate_inp_shexp, fp16 [H], may be NULL */
    const float *post_norm_w;     /* post_attention_norm, fp32 [H] (loader.h:88), may be
                                     NULL for unit weights; read by bread_moe_decode_layers
                                     only (bread_moe_forward takes the normalised input) */
} bread_moe_layer_t;

/* Scratch and synchronisation state for MoE calls on one stream.  Created
 * once (all allocation happens here, none on the call path). */
typedef struct bread_moe_ctx bread_moe_ctx_t;

int bread_moe_ctx_create(const bread_moe_shape_t *shape, int max_tokens,
                         bread_moe_ctx_t **out);
int bread_moe_ctx_destroy(bread_moe_ctx_t *ctx);

/* Which implementation bread_moe_forward runs.  AUTO picks by n_tokens and
 * shape as described there; the others force one path and make
 * bread_moe_forward return BREAD_ERR_SHAPE where it does not apply.  No
 * counterpart in the reference (which has one path); for tests and
 * benchmarks that compare the paths. */
typedef enum {
    BREAD_PATH_AUTO = 0,
    BREAD_PATH_DECODE = 1,     /* persistent single-token kernel */
    BREAD_PATH_GROUPED = 2,    /* expert-bucketed grouped GEMMs (MFMA) */
    BREAD_PATH_PER_TOKEN = 3,  /* one wave per (token, row) GEMV kernels */
    BREAD_PATH_SMALL = 4       /* 2..32 tokens: selected experts' rows over the whole GPU, fp32 dots */
} bread_moe_path_t;

int bread_moe_ctx_set_path(bread_moe_ctx_t *ctx, int path);
/* Bounds every wait of the decode and small-batch kernels on this context
 * at n_sleeps sleeps after the first look (n_sleeps < 0: each kernel's
 * default, 2^18 and 2^20; at most 2^24).  A wait that runs out sets its bit
 * of the error word (bread_moe_ctx_check) and the kernel exits normally.  No
 * reference counterpart: a small limit forces those error paths from the
 * host, for tests. */
int bread_moe_ctx_set_spin_limit(bread_moe_ctx_t *ctx, long long n_sleeps);
/* Largest n_tokens the automatic choice sends to the small-batch path. */
int bread_small_auto_tokens(void);
/* Largest n_tokens for which bread_moe_stack_forward's automatic choice runs
 * one launch of the whole decode stack per token.  No reference counterpart;
 * the crossover measured on MI355X against the small-batch path. */
int bread_stack_loop_tokens(void);

/* Synchronises the context's last stream and returns BREAD_ERR_DEVICE (and
 * the kernel's error word in *device_error, if given) when a kernel flagged
 * a fault.  Bits: 1 = the decode kernel's bounded wait for hidden or SwiGLU
 * values expired, 2 = its wait for router logits or their radii expired
 * (both: a launch that could not get every CU), 4 = the grouped path met a
 * weight superblock whose dequantised values exceed fp16's range (Q4_K
 * d >= 64 or dmin >= 1024, Q6_K |d*sc| >= 2047), 8 = the small-batch down
 * kernel's wait on a partner wave expired (the workgroup then writes none of
 * its rows of hidden), 16 = a decode workgroup's wait on another of its own
 * waves expired, 32 = bread_moe_expert_block met an expert index outside
 * [0, n_experts).  Outputs of a launch that set a bit are unspecified.  Clears
 * the word and resets the decode exchange state, so the context is usable
 * again. */
int bread_moe_ctx_check(bread_moe_ctx_t *ctx, int *device_error);

/* Routing outcomes counted on the device since the context was created (or
 * last reset), after synchronising its last stream: counts[0..n) (n <= 8)
 * receives, per decode-kernel layer, 0 = ranks certified by one radius,
 * 1 = by per-expert radii, 2 = two adjacent ranks recomputed in the
 * reference's order, 3 = every logit recomputed in the reference's order;
 * per multi-token token routed from fast logits (the small-batch path),
 * 4 = ranks certified from the fast logits, 5 = ranked by the
 * reference-order sums of the candidate rows, 6 = every logit recomputed in
 * the reference's order; 7 unused.  Counters wrap at
 * 2^32.  reset != 0 clears them; bread_moe_ctx_check clears them after a
 * flagged error.  No reference counterpart: it reports how often exact
 * routing needed the slow path. */
int bread_moe_ctx_route_stats(bread_moe_ctx_t *ctx, uint64_t *counts, int n, int reset);

/* Routing for n_tokens tokens on the device: router GEMV (fp32), softmax,
 * top-k with ties to the lower index, renormalised weights, and the raw
 * shared-gate logit (before the sigmoid).  d_x is fp32 [n_tokens][H];
 * outputs are device arrays d_idx int32 [n_tokens][K] (rank order),
 * d_w fp32 [n_tokens][K], d_gsh fp32 [n_tokens].
 * Device form of route_layer, one_layer.cu:937-992. */
int bread_route(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layer, const float *d_x,
                int n_tokens, int32_t *d_idx, float *d_w, float *d_gsh,
                bread_stream_t stream);

/* bread_route without a context, for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  The logits workspace is a static device
 * array of 1,048,576 floats in the library (4 MiB per GPU, held until the
 * process ends): n_tokens * n_experts above that returns BREAD_ERR_CAPACITY.
 * Results are bit-identical to bread_route's.  Calls that overlap on one GPU
 * share the workspace and race; serialise them (one stream, or events). */
int bread_route_noalloc(const bread_moe_shape_t *shape, const bread_moe_layer_t *layer, const float *d_x,
                        int n_tokens, int32_t *d_idx, float *d_w, float *d_gsh, bread_stream_t stream);

/* route_layer-compatible shim: one token, results copied to host arrays
 * (idx[K], w[K]) and the raw shared-gate logit returned in *gsh_logit.
 * Synchronises the stream (route_layer does a blocking copy,
 * one_layer.cu:319). */
int bread_route_layer(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layer, const float *d_x,
                      int *expert_indices, float *expert_weights, float *gsh_logit,
                      bread_stream_t stream);

/* route_layer with the reference's own input: d_normed2, the fp16
 * post-attention RMSNorm output of one token (fp16 bits [H], device,
 * 16-byte aligned), widened to fp32 on the device exactly as route_layer
 * widens it on the host (vram_half_to_cpu_float, one_layer.cu:961), then
 * routed as bread_route_layer.  Replaces `float route_layer(loader_t *L,
 * gguf_ctx_t *g, int layer_idx, const half *d_normed2, int *expert_indices,
 * float *expert_weights)` (one_layer.cu:937-939), whose callers are
 * one_layer.cu:1853 and :1998; the raw shared-gate logit that route_layer
 * returns lands in *gsh_logit. */
int bread_route_layer_f16(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layer, const uint16_t *d_normed2,
                          int *expert_indices, float *expert_weights, float *gsh_logit,
                          bread_stream_t stream);

/* The MoE FFN for n_tokens tokens, accumulated into the residual:
 *   hidden[t] += sigmoid(gsh_t) * shared(x_t) + sum_k w_tk * expert_{idx_tk}(x_t)
 * with expert(x) = down(silu(gate x) * (up x)), summed per element in the
 * reference order (shared first, then routed experts by rank).
 * d_x_normed fp32 [n_tokens][H] (the post-attention RMSNorm output),
 * d_hidden fp32 [n_tokens][H] in/out.  Optional outputs d_idx/d_w/d_gsh as in
 * bread_route (may be NULL).  Path (bread_moe_ctx_set_path, default
 * BREAD_PATH_AUTO): n_tokens == 1 runs the persistent decode kernel when the
 * shape allows it (see bread_moe_decode_layers); small batches (up to
 * bread_small_auto_tokens()) run the small-batch path (each selected expert's
 * rows streamed once over the whole GPU and dotted with the tokens that chose
 * it, fp32; H <= 2048, intermediate sizes 256 or 512); larger batches run the
 * grouped path (tokens bucketed by expert, expert GEMMs on the matrix cores
 * with fp16 operands and fp32 accumulation; intermediate sizes <= 512 and
 * 16-byte aligned Q6_K down weights); other shapes and weight-type mixes run
 * the per-token path.  A pinned path that cannot take the layer's weight
 * types returns BREAD_ERR_QTYPE. */
int bread_moe_forward(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layer,
                      const float *d_x_normed, float *d_hidden, int n_tokens,
                      int32_t *d_idx, float *d_w, float *d_gsh, bread_stream_t stream);

/* The routed experts of the MoE block with the caller's routing:
 *   hidden[t] += sum_k w[t][k] * expert_{idx[t][k]}(x_t)
 * in rank order, with no router and no shared expert: the block the
 * reference's expert benchmark times (bread_benchmark_expert_block,
 * expert_bench.cu:60-239, experts idx, weights w; its serial GPU loop of
 * :123-151) and the routed loop of one_layer.cu:1455-1470.  d_x fp32
 * [n_tokens][H], d_hidden fp32 [n_tokens][H] in/out, d_idx int32 and d_w
 * fp32 [n_tokens][K] on the device.  Runs the per-token kernels (any mix of
 * Q4_K and Q6_K).  An index outside [0, n_experts) is clamped and sets bit
 * 32 of the error word (bread_moe_ctx_check). */
int bread_moe_expert_block(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layer, const float *d_x,
                           float *d_hidden, int n_tokens, const int32_t *d_idx, const float *d_w,
                           bread_stream_t stream);

/* The MoE block of one_layer_forward on the reference's fp16 residual stream
 * (one_layer.cu:1800-1986, the d_hidden / d_normed2 interface of :1812-1815).
 * hidden and normed are fp16 [n_tokens][H], 16-byte aligned.
 *   norm_w != NULL (fp32 [H]): normed[t] = fp16(hidden[t] * rms * norm_w),
 *     rms = 1/sqrt(mean(hidden[t]^2) + shape.rms_eps), written to `normed` as
 *     the reference writes d_normed2;  norm_w == NULL: `normed` is the input.
 *   hidden[t] = fp16(float(hidden[t]) + MoE(float(normed[t])))
 * The block runs in fp32 exactly as bread_moe_forward (same paths) and is
 * rounded to fp16 once; the reference rounds after the shared expert and
 * after each routed expert, and keeps gate/up/SwiGLU/down results in fp16.
 * Values beyond fp16's range become +-Inf, as in the reference.  Optional
 * routing outputs as in bread_moe_forward. */
int bread_moe_forward_f16(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layer, const float *norm_w,
                          uint16_t *hidden, uint16_t *normed, int n_tokens,
                          int32_t *d_idx, float *d_w, float *d_gsh, bread_stream_t stream);

/* ------------------------------------------------------------------ */
/* Batched speculative verification                                     */
/* ------------------------------------------------------------------ */

/* n_tokens tokens through a stack of MoE layers:
 *   for l < n_layers:  x = RMSNorm(hidden) * layers[l].post_norm_w  (NULL: unit);
 *                      hidden += MoE_l(x)
 * one bread_moe_forward per layer for all tokens (the grouped path), or, for
 * a single token or up to bread_stack_loop_tokens() tokens under the automatic
 * choice, one bread_moe_decode_layers launch per token.  Replaces the
 * token-by-token verification of main_speculative.cu:477-497 (one
 * bread_step per draft token) at the MoE boundary: the B = K + 1 tokens of a
 * round share each layer's expert reads.  d_hidden fp32 [n_tokens][H] in/out;
 * optional routing outputs [n_layers][n_tokens][K] / [n_layers][n_tokens]. */
int bread_moe_stack_forward(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layers, int n_layers,
                            float *d_hidden, int n_tokens, int32_t *d_idx, float *d_w, float *d_gsh,
                            bread_stream_t stream);

/* Greedy prediction per token (main.cu:282-335, bc_output_norm / bc_logits /
 * bc_greedy): x = fp16(RMSNorm(hidden) * norm_w), logits = bread_matvec(w_out,
 * x) as fp16 [n_tokens][vocab], tokens[t] = greedy_sample's argmax (first
 * index of the largest logit; NaN logits skipped; 0 when logits[0] is NaN).
 * hidden fp32 [n_tokens][H]; vocab a multiple of 8; all device buffers. */
int bread_moe_greedy_head(bread_moe_ctx_t *ctx, const float *d_hidden, const float *d_norm_w,
                          const void *d_w_out, int qtype, int vocab, int n_tokens, uint16_t *d_logits,
                          int32_t *d_tokens, bread_stream_t stream);

/* greedy_sample's argmax (main.cu:326-335) over n_tokens rows of n fp16
 * logits, on the device. */
int bread_argmax_f16(const uint16_t *d_logits, int n, int n_tokens, int32_t *d_out, bread_stream_t stream);

/* The acceptance rule of main_speculative.cu:477-497, on host arrays.
 * pred[i] is the target's greedy prediction after token i of the round
 * (i = 0: the last confirmed token, i >= 1: draft i-1), n_draft + 1 entries.
 * Drafts are accepted while equal to the running prediction and not eos, at
 * most max_accept (>= 1: the tokens the caller may still output).  *next is
 * the prediction at the first mismatch or after the last draft (the bonus
 * token and the next round's seed); when the budget ends the run it is the
 * last accepted draft, since the reference stops stepping there. */
int bread_spec_accept(const int32_t *pred, const int32_t *draft, int n_draft, int32_t eos, int max_accept,
                      int *n_accept, int32_t *next);

/* One decode token through a stack of MoE layers in a single launch:
 *   for l < n_layers:  x = RMSNorm(hidden) * layers[l].post_norm_w  (eps = shape.rms_eps);
 *                      hidden += MoE_l(x)
 * the MoE part of the reference's per-layer loop (main.cu:685 ->
 * one_layer.cu:1812-1983, with the fp32 order of :1413-1471).  d_hidden is
 * fp32 [H] in/out.  Optional per-layer routing outputs d_idx int32
 * [n_layers][K], d_w fp32 [n_layers][K], d_gsh fp32 [n_layers] (raw
 * shared-gate logits); NULL skips them.  Needs the shape the persistent
 * kernel is built for (H 2048, I = I_sh = 512, E <= 256, K <= 8), 16-byte
 * aligned weights and n_layers <= 256; returns BREAD_ERR_SHAPE otherwise.
 * Layers with another weight-type mix than the kernel's (see
 * bread_moe_layer_t) split the stack: each run of the kernel's layers is one
 * launch, each other layer the RMSNorm and per-token kernels.
 * For n_layers > 1 the host layer array is copied into the context; a
 * different array than the previous call's costs one synchronous upload.
 * The kernel runs one 1024-thread workgroup per CU and every workgroup waits
 * on the others, so it needs the whole device: launches that overlap on one
 * device (any context or stream) are not allowed, and one that cannot get
 * all CUs times out and flags a device error (bread_moe_ctx_check). */
int bread_moe_decode_layers(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layers, int n_layers,
                            float *d_hidden, int32_t *d_idx, float *d_w, float *d_gsh,
                            bread_stream_t stream);

/* Timeline of the decode kernel: when d_buf is non-NULL, every launch with
 * grid * n_layers * 18 <= n_words records 64-bit wall-clock stamps (100 MHz)
 * at d_buf[(workgroup * n_layers + layer) * 18 + point], points 0 layer
 * start, 1 input normalised, 2 own logit published, 3 every logit seen,
 * 4 rank-1 expert known, 5 routing done, 6 own down dots done, 7 every down
 * dot done, 8 every SwiGLU output seen, 9 output rows stored, 10 the last
 * routed slot's SwiGLU outputs stored, 11 every routed down band loaded,
 * 12 last selection pass done, 13 ranks final (certified or recomputed),
 * 14 and 15 (uncertified layers only) own logit in the reference's order
 * done and every such logit seen, 16 the certificate's radii and maxima
 * settled, 17 every selection pass seen by the certificate.  Points a
 * layer does not reach keep their old value (clear the buffer first).
 * *grid_out receives the launch's workgroup count.  NULL turns it off. */
int bread_moe_ctx_set_trace(bread_moe_ctx_t *ctx, uint64_t *d_buf, size_t n_words, int *grid_out);

/* out[t] = x[t] * (1/sqrt(mean(x[t]^2) + eps)) * w, fp32, n_tokens rows of n
 * (layer_ops.cu:203-212; the device kernel one_layer.cu:158-181 in fp32).
 * w may be NULL for unit weights.  out may alias x. */
int bread_rmsnorm_f32(const float *d_x, const float *d_w, float *d_out, int n, int n_tokens,
                      float eps, bread_stream_t stream);

/* ------------------------------------------------------------------ */
/* HBM-resident expert arena                                           */
/* ------------------------------------------------------------------ */

/* All experts of n_layers layers resident in HBM: one allocation per layer
 * holding gate/up/down stacked tensors, the shared expert, the fp32 router
 * and the fp16 shared gate, each 256-byte aligned.  Replaces the reference's
 * 3 x 256 x 40 separate cudaMalloc calls (loader.c:628-693) and its LRU
 * (loader.c:325-505). */
typedef struct bread_arena bread_arena_t;

int bread_arena_create(const bread_moe_shape_t *shape, int n_layers, bread_arena_t **out);
int bread_arena_destroy(bread_arena_t *arena);
/* Descriptor of layer `layer` (device pointers into the arena); shexp_gate
 * and post_norm_w are NULL when the layer holds no such tensor (a layer
 * loaded from a file without them). */
int bread_arena_layer(const bread_arena_t *arena, int layer, bread_moe_layer_t *out);
/* Bytes of the largest layer allocation. */
uint64_t bread_arena_layer_bytes(const bread_arena_t *arena);
/* Weight types of layer `layer` (each BREAD_QTYPE_Q4_K or BREAD_QTYPE_Q6_K;
 * a new arena's layers are Q4_K, Q4_K, Q6_K for gate, up, down, routed and
 * shared).  A change re-lays out the layer and reallocates it when its size
 * changes (synchronous); its contents are then undefined until written.
 * The reference keeps each tensor's type per layer (loader.c:191-193). */
int bread_arena_set_layer_types(bread_arena_t *arena, int layer, int gate_type, int up_type, int down_type,
                                int gate_shexp_type, int up_shexp_type, int down_shexp_type);

/* ------------------------------------------------------------------ */
/* GGUF model files                                                    */
/* ------------------------------------------------------------------ */

/* A parsed GGUF v2/v3 file: header, metadata and tensor index over a
 * read-only mapping of the file (weights are not read until loaded).
 * Replaces gguf_open / gguf_find_tensor / gguf_tensor_by_idx (gguf.c:306-411,
 * gguf.h:100-127); a malformed file (bad magic or version, truncated
 * records, tensor data beyond the end) returns BREAD_ERR_FORMAT instead of
 * exiting. */
typedef struct bread_gguf bread_gguf_t;

typedef struct {
    const char *name;     /* owned by the file handle */
    uint32_t type;        /* ggml type id (0 F32, 1 F16, 8 Q8_0, 12 Q4_K, 14 Q6_K, ...) */
    uint32_t n_dims;
    uint64_t dims[4];     /* dims[0] innermost (columns) */
    uint64_t offset;      /* from the start of the data section */
    uint64_t size;        /* bytes (0 for a type this build has no size for) */
    uint64_t n_elems;
    const void *data;     /* host pointer into the mapping */
} bread_gguf_tensor_t;

int bread_gguf_open(const char *path, bread_gguf_t **out);
int bread_gguf_close(bread_gguf_t *file);
int bread_gguf_info(const bread_gguf_t *file, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv,
                    uint64_t *data_offset, uint32_t *alignment);
int bread_gguf_tensor(const bread_gguf_t *file, uint64_t index, bread_gguf_tensor_t *out);
/* BREAD_ERR_ARG (without recording an error) when no tensor has this name. */
int bread_gguf_find(const bread_gguf_t *file, const char *name, bread_gguf_tensor_t *out);
/* Scalar metadata: integers and bools (any width, signed sign-extended),
 * floats (f32/f64) and strings (copied NUL-terminated, cut to buf_len - 1
 * bytes); BREAD_ERR_ARG when absent or of another kind.  Arrays are parsed
 * and skipped. */
int bread_gguf_kv_int(const bread_gguf_t *file, const char *key, int64_t *value);
int bread_gguf_kv_float(const bread_gguf_t *file, const char *key, double *value);
int bread_gguf_kv_str(const bread_gguf_t *file, const char *key, char *buf, size_t buf_len);
/* Bytes of n_elems elements of a ggml type (ggml_tensor_nbytes, gguf.c:140);
 * 0 for unknown types or a count that is not a whole number of blocks. */
uint64_t bread_ggml_type_size(uint32_t type, uint64_t n_elems);

/* MoE shape of block `layer` from its tensors (loader.c:160-206): hidden and
 * expert intermediate from ffn_gate_exps [H, I, E], shared intermediate from
 * ffn_gate_shexp, top_k from <arch>.expert_used_count and rms_eps from
 * <arch>.attention.layer_norm_rms_epsilon when present (else 8 and 1e-6,
 * bread.h). */
int bread_gguf_moe_shape(const bread_gguf_t *file, int layer, bread_moe_shape_t *shape);

/* Copies block `gguf_layer`'s MoE tensors into arena layer `arena_layer`:
 * blk.N.ffn_{gate,up,down}_exps (each Q4_K or Q6_K; experts at stride
 * tensor.size / n_experts, loader.c:188-190), ffn_{gate,up,down}_shexp (each
 * Q4_K or Q6_K), ffn_gate_inp (F32 router) and, when present,
 * ffn_gate_inp_shexp (F16) and post_attention_norm (F32), which
 * bread_arena_layer then exposes as shexp_gate and post_norm_w.  The arena
 * layer takes the file's expert types (bread_arena_set_layer_types).  Other
 * types return BREAD_ERR_QTYPE, dimensions other than the arena's shape
 * BREAD_ERR_SHAPE.  Synchronous. */
int bread_arena_load_gguf(bread_arena_t *arena, int arena_layer, const bread_gguf_t *file, int gguf_layer);

/* ------------------------------------------------------------------ */
/* Seeded synthetic weights (bench and test inputs)                    */
/* ------------------------------------------------------------------ */

/* Counter-based generator (SplitMix64 of seed + i * 0x9E3779B97F4A7C15),
 * so every byte depends only on (seed, position): the same bytes on any
 * device or host.  Q4_K: d and dmin fp16 of U(1e-3, 1e-2), scale bytes and
 * nibbles uniform.  Q6_K: ql, qh uniform, sc int8 uniform in [-32, 31], d
 * fp16 of U(1e-3, 1e-2).  n_blocks superblocks are written to d_dst. */
int bread_synth_q4k(void *d_dst, uint64_t n_blocks, uint64_t seed, bread_stream_t stream);
int bread_synth_q6k(void *d_dst, uint64_t n_blocks, uint64_t seed, bread_stream_t stream);
/* n values ~ N(mean, std) (Box-Muller over the same counter generator), as
 * fp32 or as fp16 bits. */
int bread_synth_normal_f32(float *d_dst, uint64_t n, uint64_t seed, float mean, float std,
                           bread_stream_t stream);
int bread_synth_normal_f16(uint16_t *d_dst, uint64_t n, uint64_t seed, float mean, float std,
                           bread_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* BREAD_MOE_H */
