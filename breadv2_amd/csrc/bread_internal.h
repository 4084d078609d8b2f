// bread_internal.h — host-side internals of libbread_moe: status helpers,
// the MoE context and the HBM arena.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bread_moe.h"

// Records and returns a status; with exit-on-error set it prints and exits
// like the reference's CUDA_CHECK (bread_utils.h:14-21).
int bread_fail(int status, const char *where, const char *detail);

#define BREAD_HIP(call)                                                       \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) return bread_fail(BREAD_ERR_HIP, #call, hipGetErrorString(e_)); \
    } while (0)

#define BREAD_REQUIRE(cond, status, detail)                                   \
    do {                                                                      \
        if (!(cond)) return bread_fail((status), __func__, (detail));         \
    } while (0)

// hipGetLastError reports the last error of any earlier HIP call on this
// thread, including calls made by other libraries in the process.  Entry
// points clear it before launching so the check after the launch reports
// their own launch only.
static inline void bread_clear_stale_error()
{
    (void)hipGetLastError();
}

static inline hipStream_t to_hip(bread_stream_t s)
{
    return reinterpret_cast<hipStream_t>(s);
}

// One counter on its own 128-byte line (atomics to one line serialise).
struct alignas(128) bread_line {
    uint32_t v;
    uint32_t pad[31];
};

// Bits of the context's device error word (bread_moe_ctx_check).
enum : uint32_t {
    BREAD_DEV_ERR_HWAIT = 1u,   // decode: a wait for hidden or SwiGLU values ran out
    BREAD_DEV_ERR_LWAIT = 2u,   // decode: a wait for router logits or their radii ran out
    BREAD_DEV_ERR_RANGE = 4u,   // grouped: a weight superblock's values exceed fp16's range
    BREAD_DEV_ERR_PAIR = 8u,    // small batch: a wait on the partner wave ran out
    BREAD_DEV_ERR_LOCAL = 16u,  // decode: a wait on another wave of the workgroup ran out
    BREAD_DEV_ERR_INDEX = 32u,  // expert block: a caller's expert index outside [0, n_experts)
};

// Routing outcomes counted on the device (bread_moe_ctx_route_stats).
enum : int {
    BREAD_RSTAT_RADIUS = 0,     // decode layers whose fast ranks one radius certified
    BREAD_RSTAT_PER_EXPERT = 1, // decode layers certified by per-expert radii
    BREAD_RSTAT_PAIR = 2,       // decode layers with two adjacent ranks recomputed in reference order
    BREAD_RSTAT_EXACT = 3,      // decode layers with every logit recomputed in reference order
    BREAD_RSTAT_MT_CERT = 4,    // multi-token tokens whose fast ranks the certificate vouched for
    BREAD_RSTAT_MT_CAND = 5,    // ... ranked by the reference-order sums of their candidate rows
    BREAD_RSTAT_MT_EXACT = 6,   // ... with every row summed in reference order
    BREAD_RSTAT_N = 8,
};

// Device-side status of the persistent decode kernel.
struct bread_decode_sync {
    bread_line error;  // non-zero: a bounded wait expired (sticky until checked)
    struct alignas(128) {
        uint32_t v[BREAD_RSTAT_N];
    } rstat;           // routing outcomes, wrapping at 2^32
};

// Workspace of the grouped (multi-token) path, sized for max_tokens.
struct bread_grouped_ws {
    void *xhi = nullptr, *xlo = nullptr;  // activations as hi/lo fp16 [max_tokens][H]
    int *xexp = nullptr;                  // row scale exponents [max_tokens]
    int *pair_tok = nullptr;              // token of each expert-sorted pair [max_tokens*(K+1)]
    int *pos_of = nullptr;                // sorted position of pair (t, k) [max_tokens*K]
    void *tiles = nullptr;                // M-tiles of the expert GEMMs
    int *n_tiles = nullptr;
    int *work = nullptr;                  // per-XCD work lists of the two expert GEMMs
    int *n_work = nullptr;                // their lengths [2][8]
    float *eo = nullptr;                  // expert outputs by pair [max_tokens*(K+1)][H]
};

struct bread_small_ws {
    int32_t *slot_expert = nullptr;  // expert of each slot (-1: shared)
    int32_t *slot_cnt = nullptr;     // pairs of each slot (at most 4)
    int32_t *slot_pair = nullptr;    // pair ids of each slot in token order [slots][4]
    int32_t *n_slots = nullptr;
    float *eo = nullptr;             // expert outputs by pair [T (K+1)][H]
    uint8_t *xq = nullptr;           // activations in fixed point for k_sw_gateup [16][XQ_TOKEN_BYTES]
};

struct bread_moe_ctx {
    bread_moe_shape_t shape;
    int path;          // BREAD_PATH_*
    int max_tokens;
    int max_layers;
    int device;
    int decode_max_blocks;  // co-resident workgroups of the decode kernel
    hipStream_t last_stream;
    // device scratch
    float *logits;     // [max_tokens][E] (+1: the decode kernel's shared-gate logit)
    int32_t *idx;      // [max_tokens][K]
    float *w;          // [max_tokens][K]
    float *gsh;        // [max_tokens]
    float *h;          // [max_tokens][K+1][Imax] SwiGLU outputs, slot 0 = shared
    float *x32, *h32;  // [max_tokens][H] fp32 input and residual of the fp16-stream entry
    uint64_t *tlogits; // decode router logits, (epoch tag << 32) | fp32 bits, one per 64 B
    float *xbuf;       // decode layer outputs by parity, one 128 B record per workgroup
    float *hbuf;       // decode SwiGLU outputs by layer mod 3, one 128 B record per workgroup
    uint32_t epoch;    // layers run by the decode kernel on this context
    int hphase;        // epoch mod 3
    bread_decode_sync *dsync;
    void *d_layers;    // device layer table of the decode kernel [max_layers]
    void *h_layers;    // host copy of the last uploaded table
    int n_layers_uploaded;
    uint64_t *trace;   // optional decode timeline (device), trace_words entries
    size_t trace_words;
    bread_grouped_ws gws;
    bread_small_ws sws;
    int64_t spin_limit = -1;  // sleeps a bounded wait allows; < 0: each kernel's default
};

// Per-layer arena flags: which optional tensors the layer holds.
enum : int {
    BREAD_ARENA_HAS_SHGATE = 1,  // fp16 shared-gate vector (otherwise logit 0)
    BREAD_ARENA_HAS_NORM = 2,    // fp32 post-attention norm weight (otherwise unit)
};

// Where one arena layer's tensors sit in its allocation, for its weight types.
struct bread_arena_layout {
    int types[6];  // gate, up, down, gate_sh, up_sh, down_sh: BREAD_QTYPE_Q4_K or _Q6_K
    uint64_t layer_bytes;
    uint64_t off_gate, off_up, off_down, off_gate_sh, off_up_sh, off_down_sh, off_router, off_shgate, off_norm;
    uint64_t gate_expert_bytes, up_expert_bytes, down_expert_bytes;
};

struct bread_arena {
    bread_moe_shape_t shape;
    int n_layers;
    int device;
    bread_arena_layout *lay;  // n_layers layouts
    uint8_t **layers;         // n_layers device allocations
    int *flags;               // n_layers x BREAD_ARENA_HAS_*
};

// Layout of a layer with the given types; re-lays out (and reallocates)
// layer l of the arena when its types differ (synth.hip).
bread_arena_layout bread_arena_plan(const bread_moe_shape_t &s, const int types[6]);
int bread_arena_relayout(bread_arena_t *a, int l, const int types[6]);

// Expert tensor types: each of gate, up and down, routed and shared, is
// Q4_K or Q6_K (loader.c:191-193 records them per tensor; the fp32 path
// dispatches on them, one_layer.cu:1465-1468 and layer_ops.cu:169-189).
__host__ __device__ inline bool bread_expert_qtype(int t)
{
    return t == BREAD_QTYPE_Q4_K || t == BREAD_QTYPE_Q6_K;
}

// Bytes of one row of `cols` columns (a multiple of 256) of a Q4_K or Q6_K tensor.
__host__ __device__ inline uint64_t bread_expert_row_bytes(int t, int cols)
{
    return (uint64_t)(cols / 256) * (t == BREAD_QTYPE_Q4_K ? 144u : 210u);
}

// The layout the specialised kernels (decode, small-batch, grouped) take:
// Q4_K gate and up, Q6_K down, for the routed experts and the shared one.
// Other mixes run on the per-token kernels.
inline bool bread_standard_qtypes(const bread_moe_layer_t *L)
{
    return L->gate_type == BREAD_QTYPE_Q4_K && L->up_type == BREAD_QTYPE_Q4_K && L->down_type == BREAD_QTYPE_Q6_K &&
           L->gate_shexp_type == BREAD_QTYPE_Q4_K && L->up_shexp_type == BREAD_QTYPE_Q4_K &&
           L->down_shexp_type == BREAD_QTYPE_Q6_K;
}

int bread_validate_shape(const bread_moe_shape_t *s);
int bread_validate_layer(const bread_moe_shape_t *s, const bread_moe_layer_t *L);

// Launchers implemented in the .hip translation units.
int bread_launch_route(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x,
                       int n_tokens, int32_t *idx, float *w, float *gsh, hipStream_t st);
int bread_launch_moe_multi(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x,
                           float *hidden, int n_tokens, hipStream_t st);
int bread_launch_topk(const float *logits, int E, int K, int T, int32_t *idx, float *w, hipStream_t st);
// Router logits in the reference's sequential order (route.hip): logits
// [T][E]; with shg_row also the shared-gate score of every token into gsh.
int bread_route_rows_per_wave(int T, int E);
int bread_launch_route_logits(const float *router, const uint16_t *shg, const float *x, float *logits, float *gsh,
                              int H, int E, int T, bool shg_row, hipStream_t st);
// Certified fast routing for a few tokens (route.hip): fast logits with
// radii for every token into c->logits and radii (T x E floats in c->h);
// the certificate and the exact sums it asks for run in the caller's
// selection kernel (route_cert.h).
bool bread_route_certified_ok(const bread_moe_ctx_t *c, int T);
int bread_launch_route_fast(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, int T, float *gsh,
                            float *radii, uint8_t *xq, hipStream_t st);
int bread_grouped_alloc(bread_moe_ctx_t *ctx);
void bread_grouped_free(bread_moe_ctx_t *ctx);
bool bread_grouped_supported(const bread_moe_shape_t &s, const bread_moe_layer_t *L);
int bread_launch_moe_grouped(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x, float *hidden,
                             int n_tokens, hipStream_t st);
int bread_small_alloc(bread_moe_ctx_t *ctx);
void bread_small_free(bread_moe_ctx_t *ctx);
bool bread_small_supported(const bread_moe_shape_t &s, const bread_moe_layer_t *L);
int bread_small_max_tokens();
int bread_launch_moe_small(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x, float *hidden,
                           int n_tokens, hipStream_t st);
// One token (token index tok of the call: its routing lands at record tok
// of the context's routing buffers).
int bread_launch_moe_decode(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x,
                            float *hidden, hipStream_t st, int tok = 0);
// Routing outputs of layer l at idx + l * rstride * K (w alike, gsh + l * rstride).
int bread_launch_decode_layers(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layers, int n, float *hidden,
                               int32_t *idx, float *w, float *gsh, hipStream_t st, int rstride = 1);
// The same for any mix of weight types (verify.hip): runs of layers with the
// decode kernel's types in one launch each, other layers on the per-token kernels.
int bread_launch_decode_runs(bread_moe_ctx_t *ctx, const bread_moe_layer_t *layers, int n, float *hidden,
                             int32_t *idx, float *w, float *gsh, hipStream_t st, int rstride);
// true if bread_launch_decode_layers takes this layer on this context (shape,
// types, alignment, a grid that fits the device)
bool bread_decode_accepts(const bread_moe_ctx_t *ctx, const bread_moe_layer_t *L);
int bread_decode_max_blocks(int *out);
int bread_decode_grid(const bread_moe_shape_t &s);
int bread_decode_trace_points();
int bread_decode_reset(bread_moe_ctx_t *ctx);
size_t bread_decode_xbuf_floats();
size_t bread_decode_hbuf_floats();
size_t bread_decode_tlogit_words();
size_t bread_decode_layer_record_bytes();
