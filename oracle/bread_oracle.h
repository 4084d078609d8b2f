/* bread_oracle.h — CPU restatement of the reference's MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library (breadv2_amd) never links or calls it.
 *
 * Every function follows the reference's source text (cited file:line under
 * /root/reference, repo arahe-dev/breadv2) in operation order, compiled with
 * -ffp-contract=off so no multiply-add is fused where the reference has none.
 */
#ifndef BREAD_ORACLE_H
#define BREAD_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_QTYPE_F32  0
#define ORACLE_QTYPE_F16  1
#define ORACLE_QTYPE_Q8_0 8
#define ORACLE_QTYPE_Q4_K 12
#define ORACLE_QTYPE_Q6_K 14

/* fp16 bits -> fp32 with subnormals (bread_utils.h:27-47). */
float oracle_h2f(uint16_t h);
/* fp32 -> fp16 bits, round to nearest even (IEEE 754 convertFormat). */
uint16_t oracle_f2h(float f);

/* 6-bit (scale, min) unpack (dequant_q4k_cpu.c:70-79). */
void oracle_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *d, uint8_t *m);

/* One superblock -> 256 floats (dequant_q4k_cpu.c:90-123 / :141-172 with
 * the subnormal-correct converter as used by layer_ops.cu:44-105). */
void oracle_dequant_q4k_block(const uint8_t *block, float *out);
void oracle_dequant_q6k_block(const uint8_t *block, float *out);
/* One 34-byte Q8_0 block -> 32 floats, value = d * q (kernels.cu:246, :275-278). */
void oracle_dequant_q8_0_block(const uint8_t *block, float *out);

/* Bytes per row of `cols` elements (gguf.c:140-144 with the type table at
 * gguf.c:60-95); 0 for an unsupported type or a ragged column count. */
uint64_t oracle_row_bytes(int qtype, int cols);

/* rows x cols dequant, row-major, native GGUF row stride.  Returns 0 or -1. */
int oracle_dequant_rows(const void *w, int qtype, int rows, int cols, float *out);

/* y = W x, fp32, each row summed sequentially (layer_ops.cu:133-189). */
int oracle_matvec(const void *w, int qtype, const float *x, float *y, int rows, int cols);
/* Same with the row loop split over `nthreads` OpenMP threads; each row is
 * still summed sequentially, so the result is bit-identical to oracle_matvec. */
int oracle_matvec_mt(const void *w, int qtype, const float *x, float *y,
                     int rows, int cols, int nthreads);
/* bread_matvec semantics with fp16 I/O (kernels.cu:150-193): x widened to
 * fp32, fp32 sequential sum, y rounded to fp16. */
int oracle_matvec_f16io(const void *w, int qtype, const uint16_t *x, uint16_t *y,
                        int rows, int cols);

/* Elementwise primitives (layer_ops.cu:203-255). */
void  oracle_rms_norm_weighted(const float *x, const float *w, float *out, int n, float eps);
void  oracle_swiglu(const float *gate, const float *up, float *out, int n);
void  oracle_softmax(float *x, int n);
void  oracle_topk(const float *probs, int n, int k, int *indices, float *weights);
float oracle_sigmoid(float x);
/* The C library's expf, which cpu_softmax / cpu_swiglu / cpu_sigmoid call
 * (layer_ops.cu:214-255); the array form for checks in bulk. */
float oracle_expf(float x);
void  oracle_expf_array(const float *x, float *out, uint64_t n);

/* One MoE layer's weights on the host, native GGUF layout.  Expert e of a
 * stacked tensor starts at base + e * expert_bytes (loader.h:35-47,
 * loader.c:187-190). */
typedef struct {
    const uint8_t *gate_exps, *up_exps, *down_exps;
    uint64_t gate_expert_bytes, up_expert_bytes, down_expert_bytes;
    int gate_type, up_type, down_type;
    const uint8_t *gate_shexp, *up_shexp, *down_shexp;
    int gate_shexp_type, up_shexp_type, down_shexp_type;
    const float *router;          /* [n_experts][hidden] fp32 */
    const uint16_t *shexp_gate;   /* [hidden] fp16, may be NULL */
} oracle_layer_t;

typedef struct {
    int hidden, expert_inter, shared_inter, n_experts, top_k;
} oracle_shape_t;

/* Routing for one token (one_layer.cu:964-985): sequential router GEMV,
 * F16 shared-gate dot, softmax, top-k with renorm.  Returns the raw shared
 * gate logit (before the sigmoid), as route_layer does.  `logits` may be
 * NULL; when given it receives the pre-softmax logits. */
float oracle_route(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                   int *idx, float *w, float *logits);

/* oracle_route for n_tokens tokens (x [T][H]; idx/w [T][K], gsh [T], logits
 * [T][E] or NULL), tokens spread over `nthreads` OpenMP threads; each token
 * is exactly oracle_route. */
void oracle_route_batch(const oracle_shape_t *s, const oracle_layer_t *L, const float *x, int n_tokens,
                        int *idx, float *w, float *gsh, float *logits, int nthreads);

/* One token through the MoE block in the reference's fp32 order
 * (one_layer.cu:1416-1471): hidden += sigmoid(gsh)*shared(x), then
 * hidden += w_k * expert_k(x) for k in rank order.  idx/w/gsh are optional
 * outputs (may be NULL). */
void oracle_moe_token(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                      float *hidden, int *idx, float *w, float *gsh);

/* Same result, threaded: router rows, then (expert, row-chunk) work items,
 * in the shape of expert_bench.cu:126-144.  Bit-identical to
 * oracle_moe_token because every row is still summed sequentially and the
 * combine keeps the reference order. */
void oracle_moe_token_mt(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                         float *hidden, int *idx, float *w, float *gsh, int nthreads);

/* B tokens: the per-token block applied B times (x and hidden are [B][H]). */
void oracle_moe_forward(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                        float *hidden, int n_tokens, int *idx, float *w, float *gsh,
                        int nthreads);

/* greedy_sample (main.cu:326-335): argmax over n fp16 logits, best starts at
 * logits[0] and moves only on a strictly greater value. */
int oracle_greedy_f16(const uint16_t *logits, int n);

/* One verification round of main_speculative.cu:468-510 with bread_step
 * replaced by a lookup: pred[i] is the target's prediction after token i of
 * the round (0: the confirmed token, i >= 1: draft i-1).  total_gen and
 * max_tokens are the loop's counters; returns the accepted count, sets
 * *next (confirmed_tok after the round) and *out_gen (total_gen after it,
 * bonus token included). */
int oracle_spec_round(const int32_t *pred, const int32_t *draft, int n_drafted, int32_t eos, int total_gen,
                      int max_tokens, int32_t *next, int *out_gen);

/* Online core count and affinity-mask size, for the baseline report. */
int oracle_online_cores(void);
int oracle_affinity_cores(void);

#ifdef __cplusplus
}
#endif
#endif
