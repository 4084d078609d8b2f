// moe_decode.hip — single-launch MoE layer for one decode token (B = 1) on
// gfx950, for the Qwen3.5-35B-A3B shape (H 2048, I = I_sh = 512, E <= 256,
// K <= 11).
//
// One grid, three workgroup roles by blockIdx (dispatched in index order):
//   [0, R)        router: one wave per router row (plus one for the shared
//                 gate dot); the last router workgroup to finish runs
//                 softmax/top-k and publishes the K expert indices.
//   [R, R+G)      gate/up: each wave owns UPW (slot, row) units and streams
//                 the gate and up rows (2 x 1152 B) with 16-byte loads, 8
//                 lanes per 144-byte superblock; x lives in registers; SwiGLU
//                 is fused.  Shared-expert units start at once, routed units
//                 as soon as the indices are published.
//   [R+G, R+G+D)  down: DR output rows x all K+1 slots per workgroup; weight
//                 loads are issued as soon as the indices are known, then the
//                 workgroup waits for every gate/up workgroup and combines in
//                 the reference order (shared, then ranks 0..K-1).
// Producers only ever wait on lower-indexed workgroups, so in-order dispatch
// guarantees progress; every wait is also bounded (SPIN_LIMIT) and flags
// sync->error instead of hanging.  The last workgroup out restores the sync
// block, so no host-side reset is needed between launches.
//
// Replaces the reference's 45 launches per layer and its host routing round
// trip (one_layer.cu:1812-1983, route_layer :937-992).
#include "bread_internal.h"
#include "quant_dot.h"
#include "route_dev.h"

namespace {

constexpr int DH = 2048;
constexpr int DI = 512;
constexpr int NBH = DH / QK;              // Q4_K superblocks per gate/up row
constexpr int NBI = DI / QK;              // Q6_K superblocks per down row
constexpr int GU_ROW = NBH * Q4K_BYTES;   // 1152 B
constexpr int DN_ROW = NBI * Q6K_BYTES;   // 420 B
constexpr int UPW = 2;                    // gate/up units per wave
constexpr int DR = 4;                     // output rows per down workgroup
constexpr int SPW = 3;                    // slots per down wave: K + 1 <= 4 * SPW
constexpr int MAXK = 4 * SPW - 1;
constexpr uint32_t SPIN_LIMIT = 1u << 20;

static_assert(NBH == 8, "gate/up lane layout covers exactly 8 superblocks per row");
static_assert(NBI == 2, "down lane layout covers exactly 2 superblocks per row");

struct DecodeArgs {
    const uint8_t *gate_exps, *up_exps, *down_exps;
    uint64_t gate_eb, up_eb, down_eb;
    const uint8_t *gate_sh, *up_sh, *down_sh;
    const float *router;
    const uint16_t *shg;
    const float *x;
    float *hidden;
    float *logits, *gsh, *w_out, *h;
    int32_t *idx_out;
    bread_sync *sync;
    int E, K;
    int n_router, n_gu, n_down;
};

__device__ __forceinline__ uint32_t ld_acq_u32(const uint32_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void flag_error(bread_sync *s, uint32_t code)
{
    __hip_atomic_fetch_or(&s->error, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-wide: wait until all K published indices are set; lane k < K returns
// index k clamped into [0, E) (a clamp flags an error).  Returns false when
// the bounded wait expired.
__device__ bool wait_routes(bread_sync *s, int K, int E, int &my_e)
{
    const int lane = lane_id();
    int v = 0;
    bool ok = false;
    for (uint32_t it = 0; it < SPIN_LIMIT; it++) {
        v = lane < K ? (int)__hip_atomic_load(&s->route_idx[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
        if (__all(v >= 0)) {
            ok = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (!ok || v < 0 || v >= E) {
        if (lane == 0 || (v < 0 || v >= E)) flag_error(s, ok ? 2u : 1u);
        v = 0;
    }
    my_e = v;
    return ok;
}

// Wave-wide bounded wait for *p >= target, then an acquire fence.
__device__ bool wait_count(bread_sync *s, const uint32_t *p, uint32_t target)
{
    for (uint32_t it = 0; it < SPIN_LIMIT; it++) {
        const uint32_t v = __builtin_amdgcn_readfirstlane(ld_acq_u32(p));
        if (v >= target) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            return true;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane_id() == 0) flag_error(s, 4u);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return false;
}

__global__ __launch_bounds__(256) void k_moe_decode(DecodeArgs a)
{
    __shared__ int s_last;
    __shared__ float s_dot[MAXK + 1][DR];
    const int bid = (int)blockIdx.x;
    const int wid = (int)(threadIdx.x / WAVE);
    const int lane = lane_id();
    bread_sync *sy = a.sync;

    if (bid < a.n_router) {
        // ---------------- router ----------------
        const int v = bid * 4 + wid;
        if (v < a.E) {
            const float s = router_row_dot(a.router + (size_t)v * DH, a.x, DH);
            if (lane == 0) a.logits[v] = s;
        } else if (v == a.E) {
            const float s = a.shg ? shgate_dot(a.shg, a.x, DH) : 0.f;
            if (lane == 0) a.gsh[0] = s;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t old =
                __hip_atomic_fetch_add(&sy->router_done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            s_last = (old == (uint32_t)a.n_router - 1);
        }
        __syncthreads();
        if (s_last && wid == 0) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            int ik;
            float wk;
            topk_wave<4>(a.logits, a.E, a.K, ik, wk);
            if (lane < a.K) {
                a.w_out[lane] = wk;
                a.idx_out[lane] = ik;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            if (lane < a.K) __hip_atomic_store(&sy->route_idx[lane], ik, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if (bid < a.n_router + a.n_gu) {
        // ---------------- gate/up + SwiGLU ----------------
        const int gw = (bid - a.n_router) * 4 + wid;
        const int c = lane & 7;
        const int sbl = lane >> 3;
        const uint32_t j = (uint32_t)c >> 1;
        const int base = sbl * QK + 64 * (int)j + 16 * (c & 1);
        float xl[16], xh[16];
        load_x16(a.x, base, xl);
        load_x16(a.x, base + 32, xh);
        float sxl = 0.f, sxh = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sxl += xl[i];
            sxh += xh[i];
        }
        const int total = (a.K + 1) * DI;
        const int u0 = gw * UPW;
        int my_e = 0;
        if (u0 < total && (u0 + UPW - 1) / DI >= 1) wait_routes(sy, a.K, a.E, my_e);
        uint4 hg[UPW], qg[UPW], hu[UPW], qu[UPW];
#pragma unroll
        for (int i = 0; i < UPW; i++) {
            const int u = u0 + i;
            if (u < total) {
                const int slot = u / DI, r = u % DI;
                const uint8_t *gp, *up;
                if (slot == 0) {
                    gp = a.gate_sh;
                    up = a.up_sh;
                } else {
                    const int e = __shfl(my_e, slot - 1);
                    gp = a.gate_exps + (uint64_t)e * a.gate_eb;
                    up = a.up_exps + (uint64_t)e * a.up_eb;
                }
                const uint8_t *gb = gp + (size_t)r * GU_ROW + sbl * Q4K_BYTES;
                const uint8_t *ub = up + (size_t)r * GU_ROW + sbl * Q4K_BYTES;
                hg[i] = ld_b128(gb);
                qg[i] = ld_b128(gb + 16 + 16 * c);
                hu[i] = ld_b128(ub);
                qu[i] = ld_b128(ub + 16 + 16 * c);
            }
        }
#pragma unroll
        for (int i = 0; i < UPW; i++) {
            const int u = u0 + i;
            if (u < total) {
                const float g = wave_sum(q4k_chunk_dot_sx(hg[i], qg[i], j, xl, xh, sxl, sxh));
                const float uu = wave_sum(q4k_chunk_dot_sx(hu[i], qu[i], j, xl, xh, sxl, sxh));
                if (lane == 0) a.h[u] = silu_mul(g, uu);  // u = slot * DI + r
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_fetch_add(&sy->h_done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        // ---------------- down + combine ----------------
        const int r0 = (bid - a.n_router - a.n_gu) * DR;
        const int q = lane >> 4;          // row r0 + q
        const int b = (lane >> 3) & 1;    // superblock of the row
        const int uu = lane & 7;
        const int n = uu >> 2, t = uu & 3;
        const uint32_t i2 = (uint32_t)t >> 1;
        int my_e = 0;
        wait_routes(sy, a.K, a.E, my_e);
        uint2 ql0[SPW], ql1[SPW], qh[SPW], scw[SPW];
        uint32_t d16[SPW];
#pragma unroll
        for (int si = 0; si < SPW; si++) {
            const int slot = wid + 4 * si;
            if (slot <= a.K) {
                const uint8_t *base;
                if (slot == 0) {
                    base = a.down_sh;
                } else {
                    const int e = __shfl(my_e, slot - 1);
                    base = a.down_exps + (uint64_t)e * a.down_eb;
                }
                const uint8_t *blk = base + (size_t)(r0 + q) * DN_ROW + b * Q6K_BYTES;
                ql0[si] = ld8_a2(blk + 64 * n + 8 * t);
                ql1[si] = ld8_a2(blk + 64 * n + 32 + 8 * t);
                qh[si] = ld8_a2(blk + 128 + 32 * n + 8 * t);
                scw[si] = ld8_a2(blk + 192 + 8 * n);
                d16[si] = ld16_a2(blk + 208);
            }
        }
        wait_count(sy, &sy->h_done, (uint32_t)a.n_gu);
#pragma unroll
        for (int si = 0; si < SPW; si++) {
            const int slot = wid + 4 * si;
            if (slot <= a.K) {
                const float *hs = a.h + (size_t)slot * DI + b * QK + 128 * n + 8 * t;
                float xs[4][8];
#pragma unroll
                for (int s = 0; s < 4; s++) load_x8(hs, 32 * s, xs[s]);
                const float dv = sum16(q6k_unit_dot(ql0[si], ql1[si], qh[si], scw[si], i2, h2f(d16[si]), xs));
                if ((lane & 15) == 0) s_dot[slot][q] = dv;
            }
        }
        __syncthreads();
        if (wid == 0 && lane < DR) {
            const int r = r0 + lane;
            float v = a.hidden[r];
            v += sigmoidf_ref(a.gsh[0]) * s_dot[0][lane];
            for (int k = 0; k < a.K; k++) v += a.w_out[k] * s_dot[k + 1][lane];
            a.hidden[r] = v;
        }
    }

    // ---------------- exit: the last workgroup restores the sync block ----------------
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t total = (uint32_t)(a.n_router + a.n_gu + a.n_down);
        const uint32_t old = __hip_atomic_fetch_add(&sy->exit_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (old == total - 1) {
            __hip_atomic_store(&sy->router_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&sy->h_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int k = 0; k < a.K; k++)
                __hip_atomic_store(&sy->route_idx[k], -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&sy->exit_count, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

} // namespace

int bread_launch_moe_decode(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, float *hidden,
                            hipStream_t st)
{
    const bread_moe_shape_t &s = c->shape;
    if (s.hidden != DH || s.expert_inter != DI || s.shared_inter != DI || s.n_experts > 256 || s.top_k > MAXK)
        return BREAD_ERR_SHAPE;  // caller falls back to the multi-kernel path
    DecodeArgs a;
    a.gate_exps = (const uint8_t *)L->gate_exps;
    a.up_exps = (const uint8_t *)L->up_exps;
    a.down_exps = (const uint8_t *)L->down_exps;
    a.gate_eb = L->gate_expert_bytes;
    a.up_eb = L->up_expert_bytes;
    a.down_eb = L->down_expert_bytes;
    a.gate_sh = (const uint8_t *)L->gate_shexp;
    a.up_sh = (const uint8_t *)L->up_shexp;
    a.down_sh = (const uint8_t *)L->down_shexp;
    a.router = L->router;
    a.shg = L->shexp_gate;
    a.x = x;
    a.hidden = hidden;
    a.logits = c->logits;
    a.gsh = c->gsh;
    a.w_out = c->w;
    a.h = c->h;
    a.idx_out = c->idx;
    a.sync = c->sync;
    a.E = s.n_experts;
    a.K = s.top_k;
    a.n_router = (s.n_experts + 1 + 3) / 4;
    a.n_gu = ((s.top_k + 1) * DI / UPW + 3) / 4;
    a.n_down = DH / DR;
    const int grid = a.n_router + a.n_gu + a.n_down;
    hipLaunchKernelGGL(k_moe_decode, dim3(grid), dim3(256), 0, st, a);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}
