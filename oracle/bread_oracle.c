/* bread_oracle.c — CPU restatement of the reference's MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library.  The product library never links or calls it.
 *
 * Each function restates the reference's algorithm from its source text
 * (arahe-dev/breadv2, cited as file:line) in the same operation order.
 * Build with -ffp-contract=off: the reference multiplies and adds as separate
 * roundings (MSVC /fp:precise), and so must the restatement.
 *
 * Pinning (each function is checked by tests/test_oracle.py):
 *   oracle_h2f                exhaustive over all 65,536 patterns against the
 *                             F16C hardware conversion (numpy float16)
 *   oracle_f2h                exhaustive round trip over all finite halfs and
 *                             numpy's RNE float16 cast on random floats
 *   oracle_get_scale_min_k4   exhaustive over every byte value in each of the
 *                             12 positions against a bit-field pack/unpack
 *   oracle_dequant_q4k/q6k    the reference's known-answer blocks
 *                             (dequant_q4k_cpu.c:181-283), the reference's own
 *                             compiled dequant (oracle/_ref) on seeded blocks,
 *                             and an independent numpy formula
 *   oracle_dequant_q8_0       closed form d*q on seeded blocks (numpy)
 *   oracle_matvec             known-answer row dots 1792 / 2048
 *                             (kernels.cu:460-571) and an fp64 brute force
 *   oracle_softmax/topk       stable sort on (-p, index), constructed ties,
 *                             NaN rule, sum-to-one invariant
 *   oracle_route              fp64 brute force + a Python sequential loop on
 *                             small shapes
 *   oracle_moe_token(_mt)     one-hot routing (K=1) reduces to a single
 *                             expert; a numpy fp64 re-derivation; the
 *                             threaded form is bit-identical to the serial one
 */
#define _GNU_SOURCE
#include "bread_oracle.h"

#include <math.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210
#define Q80_BYTES 34
#define Q80_ELEMS 32

/* bread_utils.h:27-47: subnormals are mantissa * 2^-24; Inf/NaN keep the
 * payload bits (no quieting). */
float oracle_h2f(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exponent = (h >> 10) & 0x1F;
    uint32_t mantissa = h & 0x03FF;
    uint32_t bits;
    if (exponent == 0) {
        float val = (float)mantissa * (1.0f / 16777216.0f);
        return (h >> 15) ? -val : val;
    } else if (exponent == 31) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even.  NaNs stay
 * NaN (quiet bit set, top payload bits kept). */
uint16_t oracle_f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t mant = x & 0x7FFFFFu;
    if (exp == 0xFFu)
        return (uint16_t)(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    int e = (int)exp - 112; /* half exponent field */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        /* half subnormal: h = M * 2^(e-14), M the 24-bit significand */
        if (exp == 0) return (uint16_t)sign; /* float subnormals are < 2^-126 */
        uint32_t M = mant | 0x800000u;
        int shift = 14 - e;
        if (shift > 24) return (uint16_t)sign;
        uint32_t h = M >> shift;
        uint32_t rem = M & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* may carry to Inf */
    return (uint16_t)(sign | h);
}

/* dequant_q4k_cpu.c:70-79 */
void oracle_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m)
{
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static uint16_t rd16(const uint8_t *p)
{
    return (uint16_t)(p[0] | (p[1] << 8));
}

/* dequant_q4k_cpu.c:90-123, fp16 via bread_h2f as in layer_ops.cu:44-75.
 * Three roundings per element: d*sc, (d*sc)*q, then minus dmin*m. */
void oracle_dequant_q4k_block(const uint8_t *block, float *out)
{
    const float d = oracle_h2f(rd16(block + 0));
    const float dmin = oracle_h2f(rd16(block + 2));
    const uint8_t *scales = block + 4;
    const uint8_t *q = block + 16;
    float *y = out;
    int is = 0;
    for (int j = 0; j < QK; j += 64) {
        uint8_t sc, m;
        oracle_get_scale_min_k4(is + 0, scales, &sc, &m);
        const float d1 = d * sc;
        const float m1 = dmin * m;
        oracle_get_scale_min_k4(is + 1, scales, &sc, &m);
        const float d2 = d * sc;
        const float m2 = dmin * m;
        for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
        q += 32;
        is += 2;
    }
}

/* dequant_q4k_cpu.c:141-172 with bread_h2f (layer_ops.cu:77-105).
 * y = (d * sc) * q: two roundings. */
void oracle_dequant_q6k_block(const uint8_t *block, float *out)
{
    const float d = oracle_h2f(rd16(block + 208));
    const uint8_t *ql = block;
    const uint8_t *qh = block + 128;
    const int8_t *sc = (const int8_t *)(block + 192);
    float *y = out;
    for (int n = 0; n < QK; n += 128) {
        for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 0] = d * sc[is + 0] * q1;
            y[l + 32] = d * sc[is + 2] * q2;
            y[l + 64] = d * sc[is + 4] * q3;
            y[l + 96] = d * sc[is + 6] * q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

/* kernels.cu:246 (value = d * q) and :275-278 (the GPU kernel's product). */
void oracle_dequant_q8_0_block(const uint8_t *block, float *out)
{
    const float d = oracle_h2f(rd16(block));
    const int8_t *q = (const int8_t *)(block + 2);
    for (int i = 0; i < Q80_ELEMS; i++) out[i] = d * (float)q[i];
}

/* gguf.c:140-144 over the type table gguf.c:60-95. */
uint64_t oracle_row_bytes(int qtype, int cols)
{
    if (cols <= 0) return 0;
    switch (qtype) {
    case ORACLE_QTYPE_F32: return (uint64_t)cols * 4;
    case ORACLE_QTYPE_F16: return (uint64_t)cols * 2;
    case ORACLE_QTYPE_Q8_0: return (cols % Q80_ELEMS) ? 0 : (uint64_t)(cols / Q80_ELEMS) * Q80_BYTES;
    case ORACLE_QTYPE_Q4_K: return (cols % QK) ? 0 : (uint64_t)(cols / QK) * Q4K_BYTES;
    case ORACLE_QTYPE_Q6_K: return (cols % QK) ? 0 : (uint64_t)(cols / QK) * Q6K_BYTES;
    default: return 0;
    }
}

/* Dequantize one row into `out` (cols floats). */
static void dequant_row(const uint8_t *row, int qtype, int cols, float *out)
{
    switch (qtype) {
    case ORACLE_QTYPE_F32:
        memcpy(out, row, (size_t)cols * 4);
        break;
    case ORACLE_QTYPE_F16:
        for (int c = 0; c < cols; c++) out[c] = oracle_h2f(rd16(row + 2 * (size_t)c));
        break;
    case ORACLE_QTYPE_Q8_0:
        for (int b = 0; b < cols / Q80_ELEMS; b++)
            oracle_dequant_q8_0_block(row + (size_t)b * Q80_BYTES, out + b * Q80_ELEMS);
        break;
    case ORACLE_QTYPE_Q4_K:
        for (int b = 0; b < cols / QK; b++)
            oracle_dequant_q4k_block(row + (size_t)b * Q4K_BYTES, out + b * QK);
        break;
    case ORACLE_QTYPE_Q6_K:
        for (int b = 0; b < cols / QK; b++)
            oracle_dequant_q6k_block(row + (size_t)b * Q6K_BYTES, out + b * QK);
        break;
    }
}

int oracle_dequant_rows(const void *w, int qtype, int rows, int cols, float *out)
{
    uint64_t rb = oracle_row_bytes(qtype, cols);
    if (!w || !out || rows < 0 || rb == 0) return -1;
    for (int r = 0; r < rows; r++)
        dequant_row((const uint8_t *)w + (size_t)r * rb, qtype, cols, out + (size_t)r * cols);
    return 0;
}

/* One row of layer_ops.cu:133-167: dequantize a superblock into a scratch
 * array, then `sum += block[i] * x[b*256 + i]`, sequential over the row. */
static float row_dot(const uint8_t *row, int qtype, const float *x, int cols)
{
    float blk[QK];
    float sum = 0.0f;
    switch (qtype) {
    case ORACLE_QTYPE_F32: {
        const float *rf = (const float *)row;
        for (int c = 0; c < cols; c++) sum += rf[c] * x[c];
        return sum;
    }
    case ORACLE_QTYPE_F16:
        for (int c = 0; c < cols; c++) sum += oracle_h2f(rd16(row + 2 * (size_t)c)) * x[c];
        return sum;
    case ORACLE_QTYPE_Q8_0:
        for (int b = 0; b < cols / Q80_ELEMS; b++) {
            oracle_dequant_q8_0_block(row + (size_t)b * Q80_BYTES, blk);
            for (int i = 0; i < Q80_ELEMS; i++) sum += blk[i] * x[b * Q80_ELEMS + i];
        }
        return sum;
    case ORACLE_QTYPE_Q4_K:
        for (int b = 0; b < cols / QK; b++) {
            oracle_dequant_q4k_block(row + (size_t)b * Q4K_BYTES, blk);
            for (int i = 0; i < QK; i++) sum += blk[i] * x[b * QK + i];
        }
        return sum;
    case ORACLE_QTYPE_Q6_K:
        for (int b = 0; b < cols / QK; b++) {
            oracle_dequant_q6k_block(row + (size_t)b * Q6K_BYTES, blk);
            for (int i = 0; i < QK; i++) sum += blk[i] * x[b * QK + i];
        }
        return sum;
    }
    return sum;
}

int oracle_matvec(const void *w, int qtype, const float *x, float *y, int rows, int cols)
{
    uint64_t rb = oracle_row_bytes(qtype, cols);
    if (!w || !x || !y || rows < 0 || rb == 0) return -1;
    for (int r = 0; r < rows; r++)
        y[r] = row_dot((const uint8_t *)w + (size_t)r * rb, qtype, x, cols);
    return 0;
}

int oracle_matvec_mt(const void *w, int qtype, const float *x, float *y,
                     int rows, int cols, int nthreads)
{
    uint64_t rb = oracle_row_bytes(qtype, cols);
    if (!w || !x || !y || rows < 0 || rb == 0) return -1;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int r = 0; r < rows; r++)
        y[r] = row_dot((const uint8_t *)w + (size_t)r * rb, qtype, x, cols);
    return 0;
}

int oracle_matvec_f16io(const void *w, int qtype, const uint16_t *x, uint16_t *y,
                        int rows, int cols)
{
    uint64_t rb = oracle_row_bytes(qtype, cols);
    if (!w || !x || !y || rows < 0 || rb == 0) return -1;
    float *xf = (float *)malloc((size_t)cols * sizeof(float));
    if (!xf) return -1;
    for (int c = 0; c < cols; c++) xf[c] = oracle_h2f(x[c]);
    for (int r = 0; r < rows; r++)
        y[r] = oracle_f2h(row_dot((const uint8_t *)w + (size_t)r * rb, qtype, xf, cols));
    free(xf);
    return 0;
}

/* layer_ops.cu:203-212 */
void oracle_rms_norm_weighted(const float *x, const float *w, float *out, int n, float eps)
{
    float sum_sq = 0.0f;
    for (int i = 0; i < n; i++) sum_sq += x[i] * x[i];
    const float inv_rms = 1.0f / sqrtf(sum_sq / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv_rms * w[i];
}

/* layer_ops.cu:214-220 */
void oracle_swiglu(const float *gate, const float *up, float *out, int n)
{
    for (int i = 0; i < n; i++) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* layer_ops.cu:222-229: max is the first occurrence, the sum is sequential
 * and there is no epsilon in the division. */
void oracle_softmax(float *x, int n)
{
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float s = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        s += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= s;
}

/* layer_ops.cu:231-250: K passes of a strict '>' argmax scan from i = 0, so
 * equal probabilities go to the lower index; output in rank order; renorm
 * by the rank-order sum when it is positive.
 * Defined here where the reference is undefined (a pass that finds no entry
 * above -1e30 writes used[-1], layer_ops.cu:238-246): such entries (NaN) rank
 * below every number, so the pass takes the lowest unused index and its
 * value. */
void oracle_topk(const float *probs, int n, int K, int *indices, float *weights)
{
    unsigned char *used = (unsigned char *)calloc((size_t)(n > 0 ? n : 1), 1);
    float w_sum = 0.0f;
    for (int k = 0; k < K; k++) {
        int best = -1;
        float bv = -1e30f;
        for (int i = 0; i < n; i++)
            if (!used[i] && probs[i] > bv) {
                bv = probs[i];
                best = i;
            }
        if (best < 0) {
            for (int i = 0; i < n; i++)
                if (!used[i]) {
                    best = i;
                    break;
                }
            bv = probs[best];
        }
        indices[k] = best;
        weights[k] = bv;
        w_sum += bv;
        used[best] = 1;
    }
    if (w_sum > 0.0f)
        for (int k = 0; k < K; k++) weights[k] /= w_sum;
    free(used);
}

/* layer_ops.cu:252-255 */
float oracle_expf(float x)
{
    return expf(x);
}

void oracle_expf_array(const float *x, float *out, uint64_t n)
{
    for (uint64_t i = 0; i < n; i++) out[i] = expf(x[i]);
}

float oracle_sigmoid(float x)
{
    return 1.0f / (1.0f + expf(-x));
}

/* one_layer.cu:964-971 router GEMV (logits start at 0, j sequential),
 * :974-980 F16 shared-gate dot, :983-985 softmax and top-k. */
float oracle_route(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                   int *idx, float *w, float *logits_out)
{
    const int H = s->hidden, E = s->n_experts;
    float *logits = (float *)malloc((size_t)E * sizeof(float));
    for (int i = 0; i < E; i++) {
        float acc = 0.0f;
        const float *row = L->router + (size_t)i * H;
        for (int j = 0; j < H; j++) acc += row[j] * x[j];
        logits[i] = acc;
    }
    if (logits_out) memcpy(logits_out, logits, (size_t)E * sizeof(float));
    float gsh = 0.0f;
    if (L->shexp_gate)
        for (int j = 0; j < H; j++) gsh += oracle_h2f(L->shexp_gate[j]) * x[j];
    oracle_softmax(logits, E);
    oracle_topk(logits, E, s->top_k, idx, w);
    free(logits);
    return gsh;
}

void oracle_route_batch(const oracle_shape_t *s, const oracle_layer_t *L, const float *x, int n_tokens,
                        int *idx, float *w, float *gsh, float *logits, int nthreads)
{
    const int H = s->hidden, E = s->n_experts, K = s->top_k;
#pragma omp parallel for schedule(dynamic, 16) num_threads(nthreads)
    for (int t = 0; t < n_tokens; t++)
        gsh[t] = oracle_route(s, L, x + (size_t)t * H, idx + (size_t)t * K, w + (size_t)t * K,
                              logits ? logits + (size_t)t * E : NULL);
}

static const uint8_t *expert_ptr(const uint8_t *base, uint64_t stride, int e)
{
    return base + (uint64_t)e * stride;
}

void oracle_moe_token(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                      float *hidden, int *idx_out, float *w_out, float *gsh_out)
{
    const int H = s->hidden, I = s->expert_inter, Ish = s->shared_inter, K = s->top_k;
    float *sg = (float *)malloc((size_t)Ish * sizeof(float));
    float *su = (float *)malloc((size_t)Ish * sizeof(float));
    float *sh = (float *)malloc((size_t)H * sizeof(float));
    float *eg = (float *)malloc((size_t)I * sizeof(float));
    float *eu = (float *)malloc((size_t)I * sizeof(float));
    float *eo = (float *)malloc((size_t)H * sizeof(float));
    int *idx = (int *)malloc((size_t)K * sizeof(int));
    float *w = (float *)malloc((size_t)K * sizeof(float));

    /* one_layer.cu:1416-1420 shared gate/up */
    oracle_matvec(L->gate_shexp, L->gate_shexp_type, x, sg, Ish, H);
    oracle_matvec(L->up_shexp, L->up_shexp_type, x, su, Ish, H);
    /* :1422-1441 routing */
    const float gsh = oracle_route(s, L, x, idx, w, NULL);
    /* :1443-1449 shared SwiGLU, down, sigmoid-gated accumulate */
    oracle_swiglu(sg, su, sg, Ish);
    oracle_matvec(L->down_shexp, L->down_shexp_type, sg, sh, H, Ish);
    const float sw = oracle_sigmoid(gsh);
    for (int i = 0; i < H; i++) hidden[i] += sw * sh[i];
    /* :1451-1471 routed experts in rank order */
    for (int k = 0; k < K; k++) {
        const int e = idx[k];
        oracle_matvec(expert_ptr(L->gate_exps, L->gate_expert_bytes, e), L->gate_type, x, eg, I, H);
        oracle_matvec(expert_ptr(L->up_exps, L->up_expert_bytes, e), L->up_type, x, eu, I, H);
        oracle_swiglu(eg, eu, eg, I);
        oracle_matvec(expert_ptr(L->down_exps, L->down_expert_bytes, e), L->down_type, eg, eo, H, I);
        for (int i = 0; i < H; i++) hidden[i] += w[k] * eo[i];
    }
    if (idx_out) memcpy(idx_out, idx, (size_t)K * sizeof(int));
    if (w_out) memcpy(w_out, w, (size_t)K * sizeof(float));
    if (gsh_out) *gsh_out = gsh;
    free(sg); free(su); free(sh); free(eg); free(eu); free(eo); free(idx); free(w);
}

/* Work item of the threaded form: `slot` 0 is the shared expert, 1..K the
 * routed experts in rank order; rows [r0, r1). */
void oracle_moe_token_mt(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                         float *hidden, int *idx_out, float *w_out, float *gsh_out, int nthreads)
{
    const int H = s->hidden, I = s->expert_inter, Ish = s->shared_inter;
    const int E = s->n_experts, K = s->top_k, S = K + 1;
    const int Imax = I > Ish ? I : Ish;
    if (nthreads < 1) nthreads = 1;
    float *logits = (float *)malloc((size_t)E * sizeof(float));
    float *h = (float *)malloc((size_t)S * Imax * sizeof(float));
    float *eo = (float *)malloc((size_t)S * H * sizeof(float));
    int *idx = (int *)malloc((size_t)K * sizeof(int));
    float *w = (float *)malloc((size_t)K * sizeof(float));

    /* Router rows in parallel; each row summed sequentially (one_layer.cu:969-971). */
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int i = 0; i < E; i++) {
        float acc = 0.0f;
        const float *row = L->router + (size_t)i * H;
        for (int j = 0; j < H; j++) acc += row[j] * x[j];
        logits[i] = acc;
    }
    float gsh = 0.0f;
    if (L->shexp_gate)
        for (int j = 0; j < H; j++) gsh += oracle_h2f(L->shexp_gate[j]) * x[j];
    oracle_softmax(logits, E);
    oracle_topk(logits, E, K, idx, w);

    /* gate/up + SwiGLU per (slot, 32-row chunk) */
    const int CH = 32;
    const int nch_i = (Imax + CH - 1) / CH;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int item = 0; item < S * nch_i; item++) {
        const int slot = item / nch_i;
        const int rows = slot ? I : Ish;
        const int r0 = (item % nch_i) * CH;
        const int r1 = r0 + CH < rows ? r0 + CH : rows;
        const uint8_t *g, *u;
        int gt, ut;
        if (slot == 0) {
            g = L->gate_shexp; u = L->up_shexp; gt = L->gate_shexp_type; ut = L->up_shexp_type;
        } else {
            const int e = idx[slot - 1];
            g = expert_ptr(L->gate_exps, L->gate_expert_bytes, e);
            u = expert_ptr(L->up_exps, L->up_expert_bytes, e);
            gt = L->gate_type; ut = L->up_type;
        }
        const uint64_t gb = oracle_row_bytes(gt, H), ub = oracle_row_bytes(ut, H);
        for (int r = r0; r < r1; r++) {
            const float gv = row_dot(g + (size_t)r * gb, gt, x, H);
            const float uv = row_dot(u + (size_t)r * ub, ut, x, H);
            h[(size_t)slot * Imax + r] = (gv / (1.0f + expf(-gv))) * uv;
        }
    }

    /* down per (slot, 256-row chunk) */
    const int CD = 256;
    const int nch_h = (H + CD - 1) / CD;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int item = 0; item < S * nch_h; item++) {
        const int slot = item / nch_h;
        const int cols = slot ? I : Ish;
        const int r0 = (item % nch_h) * CD;
        const int r1 = r0 + CD < H ? r0 + CD : H;
        const uint8_t *d;
        int dt;
        if (slot == 0) {
            d = L->down_shexp; dt = L->down_shexp_type;
        } else {
            d = expert_ptr(L->down_exps, L->down_expert_bytes, idx[slot - 1]);
            dt = L->down_type;
        }
        const uint64_t db = oracle_row_bytes(dt, cols);
        for (int r = r0; r < r1; r++)
            eo[(size_t)slot * H + r] = row_dot(d + (size_t)r * db, dt, h + (size_t)slot * Imax, cols);
    }

    /* combine in the reference order, per element (one_layer.cu:1447-1469) */
    const float sw = oracle_sigmoid(gsh);
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int i = 0; i < H; i++) {
        float v = hidden[i];
        v += sw * eo[i];
        for (int k = 0; k < K; k++) v += w[k] * eo[(size_t)(k + 1) * H + i];
        hidden[i] = v;
    }
    if (idx_out) memcpy(idx_out, idx, (size_t)K * sizeof(int));
    if (w_out) memcpy(w_out, w, (size_t)K * sizeof(float));
    if (gsh_out) *gsh_out = gsh;
    free(logits); free(h); free(eo); free(idx); free(w);
}

void oracle_moe_forward(const oracle_shape_t *s, const oracle_layer_t *L, const float *x,
                        float *hidden, int n_tokens, int *idx, float *w, float *gsh,
                        int nthreads)
{
    for (int t = 0; t < n_tokens; t++) {
        const float *xt = x + (size_t)t * s->hidden;
        float *ht = hidden + (size_t)t * s->hidden;
        int *it = idx ? idx + (size_t)t * s->top_k : NULL;
        float *wt = w ? w + (size_t)t * s->top_k : NULL;
        float *gt = gsh ? gsh + t : NULL;
        if (nthreads > 1)
            oracle_moe_token_mt(s, L, xt, ht, it, wt, gt, nthreads);
        else
            oracle_moe_token(s, L, xt, ht, it, wt, gt);
    }
}

/* main.cu:326-335 */
int oracle_greedy_f16(const uint16_t *logits, int n)
{
    int best_id = 0;
    float best_val = oracle_h2f(logits[0]);
    for (int i = 1; i < n; i++) {
        const float v = oracle_h2f(logits[i]);
        if (v > best_val) {
            best_val = v;
            best_id = i;
        }
    }
    return best_id;
}

/* main_speculative.cu:474-510, the body of the verification loop. */
int oracle_spec_round(const int32_t *pred, const int32_t *draft, int n_drafted, int32_t eos, int total_gen,
                      int max_tokens, int32_t *next, int *out_gen)
{
    int step = 0;                       /* bread_step calls made so far */
    int32_t target_pred = pred[step++]; /* bread_step(confirmed_tok) */
    int n_accept = 0;
    for (int i = 0; i < n_drafted; i++) {
        if (target_pred == draft[i] && target_pred != eos) {
            n_accept++;
            total_gen++;
            if (total_gen >= max_tokens) break;
            target_pred = pred[step++]; /* bread_step(draft[i]) */
        } else {
            break;
        }
    }
    if (total_gen < max_tokens && target_pred != eos) total_gen++; /* bonus token */
    *next = target_pred;
    *out_gen = total_gen;
    return n_accept;
}

int oracle_online_cores(void)
{
    return (int)sysconf(_SC_NPROCESSORS_ONLN);
}

int oracle_affinity_cores(void)
{
    cpu_set_t set;
    CPU_ZERO(&set);
    if (sched_getaffinity(0, sizeof(set), &set) != 0) return -1;
    return CPU_COUNT(&set);
}
