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

static inline hipStream_t to_hip(bread_stream_t s)
{
    return reinterpret_cast<hipStream_t>(s);
}

// Device-side synchronisation block of the single-launch decode kernel.
// Every field returns to its reset value when a launch ends (the last
// workgroup out restores it), so launches need no host-side memset and can
// be captured in a graph.
struct bread_sync {
    uint32_t router_done;  // router workgroups finished
    uint32_t h_done;       // gate/up workgroups finished
    uint32_t exit_count;   // workgroups finished
    uint32_t error;        // non-zero: a bounded wait expired (sticky until checked)
    int32_t route_idx[64]; // published top-k (-1 = not yet published)
};

struct bread_moe_ctx {
    bread_moe_shape_t shape;
    int max_tokens;
    int device;
    hipStream_t last_stream;
    // device scratch
    float *logits;     // [max_tokens][E]
    float *lbound;     // [max_tokens][E] error bound of each logit
    int32_t *idx;      // [max_tokens][K]
    float *w;          // [max_tokens][K]
    float *gsh;        // [max_tokens]
    float *h;          // [max_tokens][K+1][Imax] SwiGLU outputs, slot 0 = shared
    bread_sync *sync;  // decode kernel synchronisation
};

struct bread_arena {
    bread_moe_shape_t shape;
    int n_layers;
    int device;
    uint64_t layer_bytes;
    uint64_t off_gate, off_up, off_down, off_gate_sh, off_up_sh, off_down_sh, off_router, off_shgate;
    uint64_t gate_expert_bytes, up_expert_bytes, down_expert_bytes;
    uint8_t **layers;  // n_layers device allocations
};

int bread_validate_layer(const bread_moe_shape_t *s, const bread_moe_layer_t *L);

// Launchers implemented in the .hip translation units.
int bread_launch_route(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x,
                       int n_tokens, int32_t *idx, float *w, float *gsh, hipStream_t st);
int bread_launch_moe_multi(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x,
                           float *hidden, int n_tokens, hipStream_t st);
int bread_launch_moe_decode(bread_moe_ctx_t *ctx, const bread_moe_layer_t *L, const float *x,
                            float *hidden, hipStream_t st);
