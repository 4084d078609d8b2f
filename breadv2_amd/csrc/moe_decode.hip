// moe_decode.hip — persistent single-launch MoE decode (one token, B = 1) for
// gfx950 at the Qwen3.5-35B-A3B shape (H 2048, I = I_sh = 512, E <= 256,
// K <= 11), over one layer or a stack of layers per launch.
//
// For each layer l of the launch:  x = RMSNorm(h) * w_l  (or the given x for
// a single pre-normalised layer),  h += MoE_l(x).  One cooperative grid with
// four workgroup roles that stay fixed across layers:
//   router  (R): one wave per router row plus one for the shared-gate dot;
//                router rows are loaded before h is ready; router workgroup 0
//                also publishes the normalised x.
//   shared  (S): shared-expert gate/up + SwiGLU (weights loaded before h is
//                ready; they do not depend on routing).
//   routed  (G): routed-expert gate/up + SwiGLU; each workgroup runs
//                softmax/top-k itself from the published logits (no publish
//                hop), then streams its rows.
//   down    (D): down projection of all K+1 slots for DR output rows; weight
//                loads are issued as soon as the routing is known, then the
//                combine runs in the reference order (shared, then ranks).
// Layer-to-layer and phase-to-phase dependencies are device counters, each
// spread over 8 cache lines (one contended line costs ~10 ns per atomic on
// MI355X).  Data that crosses workgroups (h, x, logits, SwiGLU outputs) is
// written and read with device-coherent (sc1) accesses, so no L2-wide
// writeback or invalidate is needed.  Every wait is bounded and flags an
// error instead of hanging; the last workgroup out resets the counters, so
// launches need no host-side reset.
//
// Replaces the reference's 45 launches per layer and its host routing round
// trip (one_layer.cu:1812-1983, route_layer :937-992), and the per-layer host
// loop over layers (main.cu:685).
#include <string.h>

#include "bread_internal.h"
#include "quant_dot.h"
#include "route_dev.h"

namespace {

constexpr int DH = 2048;
constexpr int DI = 512;
constexpr int NBH = DH / QK;             // Q4_K superblocks per gate/up row
constexpr int NBI = DI / QK;             // Q6_K superblocks per down row
constexpr int GU_ROW = NBH * Q4K_BYTES;  // 1152 B
constexpr int DN_ROW = NBI * Q6K_BYTES;  // 420 B
constexpr int UPW = 2;                   // gate/up (slot, row) units per wave
constexpr int UPB = 4 * UPW;             // units per gate/up workgroup
constexpr int DR = 4;                    // output rows per down workgroup
constexpr int SPW = 3;                   // slots per down wave: K + 1 <= 4 * SPW
constexpr int MAXK = 4 * SPW - 1;
constexpr int NLINES = 8;
constexpr uint32_t SPIN_LIMIT = 1u << 18;
constexpr uint32_t BUF_WORD3 = 0x00020000u;  // raw buffer descriptor word 3 (gfx9)
constexpr int AUX_COHERENT = 16;             // sc1: device-coherent access

static_assert(NBH == 8 && NBI == 2, "lane layouts assume H = 2048 and I = 512");
static_assert(DI % UPB == 0, "a gate/up workgroup must stay inside one slot");

// Trace points recorded per (workgroup, layer) when a trace buffer is given.
enum { TP_START = 0, TP_READY = 1, TP_ROUTED = 2, TP_LOADS = 3, TP_HREADY = 4, TP_DONE = 5, TP_N = 8 };

struct DecLayer {
    const uint8_t *gate_exps, *up_exps, *down_exps;
    const uint8_t *gate_sh, *up_sh, *down_sh;
    const float *router;
    const uint16_t *shg;
    const float *norm_w;
    uint64_t gate_eb, up_eb, down_eb;
};

struct DecArgs {
    const DecLayer *layers;  // device table, or NULL: use `one`
    DecLayer one;
    int L;
    const float *x0;         // non-NULL: layer 0 input given (already normalised)
    float *hidden;
    float eps;
    float *logits;           // [E + 1]: logits, then the shared-gate logit
    float *xnorm;            // [H]
    float *hbuf;             // [(K + 1) * I]
    int32_t *idx_out;        // [L][K] or NULL
    float *w_out;            // [L][K] or NULL
    float *gsh_out;          // [L] or NULL
    bread_decode_sync *sync;
    uint64_t *trace;         // [grid][L][TP_N] or NULL
    int E, K;
    int nR, nS, nG, nD;
};

// ---------------------------------------------------------------- memory helpers

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, (int)BUF_WORD3);
}

// 16-byte buffer load at voff (per lane) + soff (wave-uniform constant)
template <int AUX>
__device__ __forceinline__ float4 bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0)
{
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, AUX));
}

template <int AUX>
__device__ __forceinline__ uint4 bload4u(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, AUX));
}

__device__ __forceinline__ uint32_t bload1u(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

template <int AUX>
__device__ __forceinline__ void bstore4(float4 v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0)
{
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v),
                                           r, (int)voff, (int)soff, AUX);
}

// 8 bytes at a 2-byte aligned buffer offset, from aligned dword loads (the
// buffer-load form of ld8_a2: every dword read holds a wanted byte).
__device__ __forceinline__ uint2 bld8_a2(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    const uint32_t a = off & ~3u, sh = off & 3u;
    const uint32_t w0 = bload1u(r, a), w1 = bload1u(r, a + 4), w2 = bload1u(r, (off + 7) & ~3u);
    uint2 o;
    o.x = __builtin_amdgcn_alignbyte(w1, w0, sh);
    o.y = __builtin_amdgcn_alignbyte(w2, w1, sh);
    return o;
}

__device__ __forceinline__ uint32_t bld16_a2(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return (bload1u(r, off & ~3u) >> (8u * (off & 3u))) & 0xFFFFu;
}

__device__ __forceinline__ float cload(const float *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void cstore(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void trace_point(const DecArgs &a, int l, int tp)
{
    if (a.trace && threadIdx.x == 0)
        a.trace[((size_t)blockIdx.x * a.L + l) * TP_N + tp] = wall_clock64();
}

// The layer record is the same for the whole grid: keep it in scalar registers.
__device__ __forceinline__ DecLayer load_layer(const DecArgs &a, int l)
{
    DecLayer d = a.layers ? a.layers[l] : a.one;
    d.gate_exps = uniform_ptr(d.gate_exps);
    d.up_exps = uniform_ptr(d.up_exps);
    d.down_exps = uniform_ptr(d.down_exps);
    d.gate_sh = uniform_ptr(d.gate_sh);
    d.up_sh = uniform_ptr(d.up_sh);
    d.down_sh = uniform_ptr(d.down_sh);
    d.router = uniform_ptr(d.router);
    d.shg = uniform_ptr(d.shg);
    d.norm_w = uniform_ptr(d.norm_w);
    d.gate_eb = uniform64(d.gate_eb);
    d.up_eb = uniform64(d.up_eb);
    d.down_eb = uniform64(d.down_eb);
    return d;
}

// ---------------------------------------------------------------- synchronisation

__device__ __forceinline__ bool has_error(const bread_decode_sync *s)
{
    return __hip_atomic_load(&s->error.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

__device__ __forceinline__ void flag_error(bread_decode_sync *s, uint32_t code)
{
    __hip_atomic_fetch_or(&s->error.v, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-wide bounded wait until the sum of a counter's 8 lines reaches target.
__device__ __forceinline__ bool wait_lines(bread_decode_sync *s, const bread_line *lines, uint32_t target)
{
    const int lane = lane_id();
    for (uint32_t it = 0; it < SPIN_LIMIT; it++) {
        const uint32_t v =
            lane < NLINES ? __hip_atomic_load(&lines[lane].v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        uint32_t tot = 0;
#pragma unroll
        for (int k = 0; k < NLINES; k++) tot += __builtin_amdgcn_readlane(v, k);
        if (tot >= target) return true;
        if ((it & 63) == 63 && has_error(s)) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0) flag_error(s, 1u);
    return false;
}

// Workgroup-wide wait: wave 0 polls (one poller per workgroup keeps the
// counter lines' traffic low), the others wait at the barrier.
__device__ __forceinline__ void wait_lines_wg(bread_decode_sync *s, const bread_line *lines, uint32_t target)
{
    if (wave_id() == 0) wait_lines(s, lines, target);
    __syncthreads();
}

// Workgroup-wide: every memory access of every wave has completed (s_waitcnt
// 0 before the barrier), then one counter line is bumped.  Every write that
// another workgroup reads is a device-coherent (sc1) store, complete once it
// is acknowledged, so no cache writeback is needed: an agent-scope release or
// acquire fence here (an L2 writeback / invalidate) costs ~5-30 ns per
// workgroup, serialised, on MI355X.
__device__ __forceinline__ void signal_line(bread_line *lines)
{
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(&lines[blockIdx.x % NLINES].v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Softmax/top-k over the published logits (coherent loads) by one wave;
// lane k < K gets (idx_k, w_k); also returns the raw shared-gate logit.
__device__ __forceinline__ void route_from_logits(const DecArgs &a, int &ik, float &wk, float &gsh)
{
    const int lane = lane_id();
    float p[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int i = lane + WAVE * v;
        p[v] = i < a.E ? cload(a.logits + i) : -__builtin_inff();
    }
    gsh = cload(a.logits + a.E);
    topk_wave_vals<4>(p, a.E, a.K, ik, wk);
}

// ---------------------------------------------------------------- router role

// A router wave holds columns 4*lane + 256*m (m < 8) of its row and of x.
__device__ void router_role(const DecArgs &a)
{
    const int wid = wave_id(), lane = lane_id();
    const int v = (int)blockIdx.x * 4 + wid;
    const bool row = v < a.E, gate = v == a.E;
    const uint32_t vo = 16u * (uint32_t)lane;
    for (int l = 0; l < a.L; l++) {
        const DecLayer Ly = load_layer(a, l);
        trace_point(a, l, TP_START);
        float4 wr[8];
        if (row) {
            const auto r = rsrc(Ly.router + (size_t)v * DH, DH * 4);
#pragma unroll
            for (int m = 0; m < 8; m++) wr[m] = bload4<0>(r, vo, 1024u * m);
        } else if (gate && Ly.shg) {
            const auto r = rsrc(Ly.shg, DH * 2);
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const uint2 g = __builtin_bit_cast(
                    uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)(8 * lane), (int)(512 * m), 0));
                wr[m] = make_float4(h2f(g.x), h2f(g.x >> 16), h2f(g.y), h2f(g.y >> 16));
            }
        } else {
#pragma unroll
            for (int m = 0; m < 8; m++) wr[m] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (l > 0) wait_lines_wg(a.sync, a.sync->out_done, (uint32_t)(l * a.nD));
        trace_point(a, l, TP_READY);
        float4 xv[8];
        if (l == 0 && a.x0) {
            const auto xr = rsrc(a.x0, DH * 4);
#pragma unroll
            for (int m = 0; m < 8; m++) xv[m] = bload4<0>(xr, vo, 1024u * m);
        } else {
            const auto hr = rsrc(a.hidden, DH * 4);
            float ss = 0.f;
#pragma unroll
            for (int m = 0; m < 8; m++) {
                xv[m] = bload4<AUX_COHERENT>(hr, vo, 1024u * m);
                ss = fmaf(xv[m].x, xv[m].x, ss);
                ss = fmaf(xv[m].y, xv[m].y, ss);
                ss = fmaf(xv[m].z, xv[m].z, ss);
                ss = fmaf(xv[m].w, xv[m].w, ss);
            }
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)DH + a.eps);  // layer_ops.cu:209
            if (Ly.norm_w) {
                const auto nr = rsrc(Ly.norm_w, DH * 4);
#pragma unroll
                for (int m = 0; m < 8; m++) {
                    const float4 nw = bload4<0>(nr, vo, 1024u * m);
                    xv[m] = make_float4(xv[m].x * inv * nw.x, xv[m].y * inv * nw.y, xv[m].z * inv * nw.z,
                                        xv[m].w * inv * nw.w);
                }
            } else {
#pragma unroll
                for (int m = 0; m < 8; m++)
                    xv[m] = make_float4(xv[m].x * inv, xv[m].y * inv, xv[m].z * inv, xv[m].w * inv);
            }
        }
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            acc = fmaf(wr[m].x, xv[m].x, acc);
            acc = fmaf(wr[m].y, xv[m].y, acc);
            acc = fmaf(wr[m].z, xv[m].z, acc);
            acc = fmaf(wr[m].w, xv[m].w, acc);
        }
        acc = wave_sum(acc);
        if ((row || gate) && lane == 0) cstore(a.logits + v, acc);  // v == E: the shared-gate logit
        if (blockIdx.x == 0 && wid == 0) {
            const auto xr = rsrc(a.xnorm, DH * 4);
#pragma unroll
            for (int m = 0; m < 8; m++) bstore4<AUX_COHERENT>(xv[m], xr, vo, 1024u * m);
        }
        trace_point(a, l, TP_DONE);
        signal_line(a.sync->router_done);
    }
}

// ---------------------------------------------------------------- gate/up roles

// A gate/up lane owns qs chunk c = lane%8 of superblock sbl = lane/8 of a row:
// x columns base + [0,16) (low nibbles) and base + 32 + [0,16) (high nibbles),
// base = sbl*256 + 64*(c/2) + 16*(c%2).  The 64 lanes cover all H columns once.
__device__ __forceinline__ int gu_base(int lane)
{
    const int c = lane & 7;
    return (lane >> 3) * QK + 64 * (c >> 1) + 16 * (c & 1);
}

__device__ __forceinline__ void load_x32(__amdgpu_buffer_rsrc_t r, int base, float (&xl)[16], float (&xh)[16])
{
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 lo = bload4<AUX_COHERENT>(r, (uint32_t)(4 * base), (uint32_t)(16 * q));
        const float4 hi = bload4<AUX_COHERENT>(r, (uint32_t)(4 * base), (uint32_t)(128 + 16 * q));
        xl[4 * q] = lo.x; xl[4 * q + 1] = lo.y; xl[4 * q + 2] = lo.z; xl[4 * q + 3] = lo.w;
        xh[4 * q] = hi.x; xh[4 * q + 1] = hi.y; xh[4 * q + 2] = hi.z; xh[4 * q + 3] = hi.w;
    }
}

// x = RMSNorm(h) * w (or the given x of a single pre-normalised layer).
__device__ __forceinline__ void gu_x_from_hidden(const DecArgs &a, const DecLayer &Ly, int l, int base,
                                                 float (&xl)[16], float (&xh)[16])
{
    if (l == 0 && a.x0) {
        load_x16(a.x0, base, xl);
        load_x16(a.x0, base + 32, xh);
        return;
    }
    load_x32(rsrc(a.hidden, DH * 4), base, xl, xh);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        ss = fmaf(xl[i], xl[i], ss);
        ss = fmaf(xh[i], xh[i], ss);
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)DH + a.eps);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float wl = Ly.norm_w ? Ly.norm_w[base + i] : 1.f;
        const float wh = Ly.norm_w ? Ly.norm_w[base + 32 + i] : 1.f;
        xl[i] = xl[i] * inv * wl;
        xh[i] = xh[i] * inv * wh;
    }
}

__device__ __forceinline__ void gu_issue(const uint8_t *gbase, const uint8_t *ubase, int r0, uint4 (&hg)[UPW],
                                         uint4 (&qg)[UPW], uint4 (&hu)[UPW], uint4 (&qu)[UPW])
{
    const int lane = lane_id();
    const uint32_t oh = (uint32_t)((lane >> 3) * Q4K_BYTES);
    const uint32_t oq = oh + 16u + 16u * (uint32_t)(lane & 7);
    const auto gr = rsrc(gbase + (size_t)r0 * GU_ROW, UPW * GU_ROW);
    const auto ur = rsrc(ubase + (size_t)r0 * GU_ROW, UPW * GU_ROW);
#pragma unroll
    for (int i = 0; i < UPW; i++) {
        hg[i] = bload4u<0>(gr, oh, (uint32_t)(i * GU_ROW));
        qg[i] = bload4u<0>(gr, oq, (uint32_t)(i * GU_ROW));
        hu[i] = bload4u<0>(ur, oh, (uint32_t)(i * GU_ROW));
        qu[i] = bload4u<0>(ur, oq, (uint32_t)(i * GU_ROW));
    }
}

// Gate/up + SwiGLU for UPW consecutive rows of one slot by one wave.
__device__ __forceinline__ void gu_compute(const DecArgs &a, int slot, int r0, const float (&xl)[16],
                                           const float (&xh)[16], const uint4 (&hg)[UPW], const uint4 (&qg)[UPW],
                                           const uint4 (&hu)[UPW], const uint4 (&qu)[UPW])
{
    const int lane = lane_id();
    const uint32_t j = (uint32_t)(lane & 7) >> 1;
    float sxl = 0.f, sxh = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        sxl += xl[i];
        sxh += xh[i];
    }
#pragma unroll
    for (int i = 0; i < UPW; i++) {
        const float g = wave_sum(q4k_chunk_dot_sx(hg[i], qg[i], j, xl, xh, sxl, sxh));
        const float u = wave_sum(q4k_chunk_dot_sx(hu[i], qu[i], j, xl, xh, sxl, sxh));
        if (lane == 0) cstore(a.hbuf + slot * DI + r0 + i, silu_mul(g, u));
    }
}

__device__ void shared_role(const DecArgs &a)
{
    const int wid = wave_id(), lane = lane_id();
    const int r0 = (((int)blockIdx.x - a.nR) * 4 + wid) * UPW;  // rows of the shared expert
    const int base = gu_base(lane);
    for (int l = 0; l < a.L; l++) {
        const DecLayer Ly = load_layer(a, l);
        trace_point(a, l, TP_START);
        uint4 hg[UPW], qg[UPW], hu[UPW], qu[UPW];
        gu_issue(Ly.gate_sh, Ly.up_sh, r0, hg, qg, hu, qu);
        if (l > 0) wait_lines_wg(a.sync, a.sync->out_done, (uint32_t)(l * a.nD));
        trace_point(a, l, TP_READY);
        float xl[16], xh[16];
        gu_x_from_hidden(a, Ly, l, base, xl, xh);
        gu_compute(a, 0, r0, xl, xh, hg, qg, hu, qu);
        trace_point(a, l, TP_DONE);
        signal_line(a.sync->h_done);
    }
}

__device__ void routed_role(const DecArgs &a)
{
    __shared__ int s_e;
    const int wid = wave_id(), lane = lane_id();
    const int u0 = DI + ((int)blockIdx.x - a.nR - a.nS) * UPB;  // first (slot, row) unit
    const int slot = u0 / DI;                                   // 1..K: rank slot - 1
    const int r0 = u0 % DI + wid * UPW;
    const int base = gu_base(lane);
    for (int l = 0; l < a.L; l++) {
        const DecLayer Ly = load_layer(a, l);
        trace_point(a, l, TP_START);
        wait_lines_wg(a.sync, a.sync->router_done, (uint32_t)((l + 1) * a.nR));
        trace_point(a, l, TP_READY);
        float xl[16], xh[16];
        load_x32(rsrc(a.xnorm, DH * 4), base, xl, xh);
        if (wid == 0) {
            int ik;
            float wk, g;
            route_from_logits(a, ik, wk, g);
            const int e = __shfl(ik, slot - 1);
            if (lane == 0) s_e = (e >= 0 && e < a.E) ? e : 0;
        }
        __syncthreads();
        const int e = uniform(s_e);
        trace_point(a, l, TP_ROUTED);
        uint4 hg[UPW], qg[UPW], hu[UPW], qu[UPW];
        gu_issue(Ly.gate_exps + (uint64_t)e * Ly.gate_eb, Ly.up_exps + (uint64_t)e * Ly.up_eb, r0, hg, qg, hu, qu);
        gu_compute(a, slot, r0, xl, xh, hg, qg, hu, qu);
        trace_point(a, l, TP_DONE);
        signal_line(a.sync->h_done);
    }
}

// ---------------------------------------------------------------- down role

// A down lane owns row r0 + lane/16, superblock b = (lane/8)%2 of it and the
// Q6_K unit (half n, l in [8t, 8t+8)) of that superblock; wave w handles
// slots w, w+4, w+8 for the workgroup's DR rows.
__device__ void down_role(const DecArgs &a)
{
    __shared__ int s_idx[MAXK];
    __shared__ float s_w[MAXK];
    __shared__ float s_gsh;
    __shared__ float s_dot[MAXK + 1][DR];
    const int wid = wave_id(), lane = lane_id();
    const int dwg = (int)blockIdx.x - a.nR - a.nS - a.nG;
    const int r0 = dwg * DR;
    const int q = lane >> 4;
    const int b = (lane >> 3) & 1;
    const int n = (lane >> 2) & 1, t = lane & 3;
    const uint32_t i2 = (uint32_t)t >> 1;
    // byte offsets of this lane's fields inside the workgroup's DR rows
    const uint32_t ob = (uint32_t)(q * DN_ROW + b * Q6K_BYTES);
    const uint32_t o_ql0 = ob + 64 * n + 8 * t, o_ql1 = o_ql0 + 32;
    const uint32_t o_qh = ob + 128 + 32 * n + 8 * t, o_sc = ob + 192 + 8 * n, o_d = ob + 208;
    const uint32_t o_h = (uint32_t)(4 * (b * QK + 128 * n + 8 * t));
    for (int l = 0; l < a.L; l++) {
        const DecLayer Ly = load_layer(a, l);
        trace_point(a, l, TP_START);
        wait_lines_wg(a.sync, a.sync->router_done, (uint32_t)((l + 1) * a.nR));
        trace_point(a, l, TP_READY);
        if (wid == 0) {
            int ik;
            float wk, g;
            route_from_logits(a, ik, wk, g);
            if (lane < a.K) {
                s_idx[lane] = (ik >= 0 && ik < a.E) ? ik : 0;
                s_w[lane] = wk;
            }
            if (lane == 0) s_gsh = g;
            if (dwg == 0 && lane < a.K) {
                if (a.idx_out) a.idx_out[l * a.K + lane] = ik;
                if (a.w_out) a.w_out[l * a.K + lane] = wk;
                if (a.gsh_out && lane == 0) a.gsh_out[l] = g;
            }
        }
        __syncthreads();
        trace_point(a, l, TP_ROUTED);
        uint2 ql0[SPW], ql1[SPW], qh[SPW], scw[SPW];
        uint32_t d16[SPW];
#pragma unroll
        for (int si = 0; si < SPW; si++) {
            const int slot = wid + 4 * si;
            if (slot <= a.K) {
                const uint8_t *base =
                    slot == 0 ? Ly.down_sh : Ly.down_exps + (uint64_t)uniform(s_idx[slot - 1]) * Ly.down_eb;
                const auto r = rsrc(base + (size_t)r0 * DN_ROW, DR * DN_ROW);
                ql0[si] = bld8_a2(r, o_ql0);
                ql1[si] = bld8_a2(r, o_ql1);
                qh[si] = bld8_a2(r, o_qh);
                scw[si] = bld8_a2(r, o_sc);
                d16[si] = bld16_a2(r, o_d);
            }
        }
        trace_point(a, l, TP_LOADS);
        wait_lines_wg(a.sync, a.sync->h_done, (uint32_t)((l + 1) * (a.nS + a.nG)));
        trace_point(a, l, TP_HREADY);
        const auto hr = rsrc(a.hbuf, (uint32_t)((a.K + 1) * DI * 4));
#pragma unroll
        for (int si = 0; si < SPW; si++) {
            const int slot = wid + 4 * si;
            if (slot <= a.K) {
                float xs[4][8];
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const float4 v0 = bload4<AUX_COHERENT>(hr, o_h, (uint32_t)(4 * slot * DI + 128 * s));
                    const float4 v1 = bload4<AUX_COHERENT>(hr, o_h, (uint32_t)(4 * slot * DI + 128 * s + 16));
                    xs[s][0] = v0.x; xs[s][1] = v0.y; xs[s][2] = v0.z; xs[s][3] = v0.w;
                    xs[s][4] = v1.x; xs[s][5] = v1.y; xs[s][6] = v1.z; xs[s][7] = v1.w;
                }
                const float dv = sum16(q6k_unit_dot(ql0[si], ql1[si], qh[si], scw[si], i2, h2f(d16[si]), xs));
                if ((lane & 15) == 0) s_dot[slot][q] = dv;
            }
        }
        __syncthreads();
        if (wid == 0 && lane < DR) {
            const int r = r0 + lane;
            float v = cload(a.hidden + r);
            v += sigmoidf_ref(s_gsh) * s_dot[0][lane];                      // one_layer.cu:1447-1449
            for (int k = 0; k < a.K; k++) v += s_w[k] * s_dot[k + 1][lane];  // :1469
            cstore(a.hidden + r, v);
        }
        trace_point(a, l, TP_DONE);
        signal_line(a.sync->out_done);
    }
}

// ---------------------------------------------------------------- kernel

__global__ __launch_bounds__(256, 4) void k_decode(DecArgs a)
{
    const int bid = (int)blockIdx.x;
    if (bid < a.nR)
        router_role(a);
    else if (bid < a.nR + a.nS)
        shared_role(a);
    else if (bid < a.nR + a.nS + a.nG)
        routed_role(a);
    else
        down_role(a);
    // exit: the last workgroup out (two levels of 8 lines) resets every counter
    __syncthreads();
    if (threadIdx.x == 0) {
        bread_decode_sync *s = a.sync;
        const int total = a.nR + a.nS + a.nG + a.nD;
        const int grp = bid % NLINES;
        const uint32_t members = (uint32_t)((total - grp + NLINES - 1) / NLINES);
        const uint32_t o1 = __hip_atomic_fetch_add(&s->exit1[grp].v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (o1 == members - 1) {
            const uint32_t o2 = __hip_atomic_fetch_add(&s->exit2.v, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (o2 == (uint32_t)NLINES - 1) {
                for (int k = 0; k < NLINES; k++) {
                    __hip_atomic_store(&s->router_done[k].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&s->h_done[k].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&s->out_done[k].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&s->exit1[k].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __hip_atomic_store(&s->exit2.v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

DecLayer to_dec(const bread_moe_layer_t &L)
{
    DecLayer d;
    d.gate_exps = (const uint8_t *)L.gate_exps;
    d.up_exps = (const uint8_t *)L.up_exps;
    d.down_exps = (const uint8_t *)L.down_exps;
    d.gate_sh = (const uint8_t *)L.gate_shexp;
    d.up_sh = (const uint8_t *)L.up_shexp;
    d.down_sh = (const uint8_t *)L.down_shexp;
    d.router = L.router;
    d.shg = L.shexp_gate;
    d.norm_w = L.post_norm_w;
    d.gate_eb = L.gate_expert_bytes;
    d.up_eb = L.up_expert_bytes;
    d.down_eb = L.down_expert_bytes;
    return d;
}

bool decode_shape_ok(const bread_moe_shape_t &s)
{
    return s.hidden == DH && s.expert_inter == DI && s.shared_inter == DI && s.n_experts <= 256 &&
           s.n_experts >= s.top_k && s.top_k <= MAXK;
}

void fill_roles(const bread_moe_shape_t &s, DecArgs &a)
{
    a.E = s.n_experts;
    a.K = s.top_k;
    a.nR = (s.n_experts + 1 + 3) / 4;
    a.nS = DI / UPB;
    a.nG = s.top_k * DI / UPB;
    a.nD = DH / DR;
}

int launch(bread_moe_ctx_t *c, DecArgs &a, hipStream_t st)
{
    const int grid = a.nR + a.nS + a.nG + a.nD;
    // One layer: every wait is on lower-indexed workgroups, which in-order
    // dispatch starts first, so the grid need not be co-resident.  Several
    // layers: later layers wait on higher-indexed workgroups too, so the whole
    // grid must be resident at once (a cooperative launch checks it).
    if (a.L > 1 && grid > c->decode_max_blocks) return BREAD_ERR_SHAPE;
    a.logits = c->logits;
    a.xnorm = c->xnorm;
    a.hbuf = c->h;
    a.sync = c->dsync;
    a.trace = (c->trace && (size_t)grid * a.L * TP_N <= c->trace_words) ? c->trace : nullptr;
    a.eps = c->shape.rms_eps;
    bread_clear_stale_error();
    if (a.L == 1) {
        hipLaunchKernelGGL(k_decode, dim3(grid), dim3(256), 0, st, a);
        BREAD_HIP(hipGetLastError());
    } else {
        void *args[] = {&a};
        BREAD_HIP(hipLaunchCooperativeKernel((const void *)k_decode, dim3(grid), dim3(256), args, 0, st));
    }
    return BREAD_OK;
}

} // namespace

int bread_decode_max_blocks(int *out)
{
    int dev = 0, cus = 0, per_cu = 0;
    BREAD_HIP(hipGetDevice(&dev));
    BREAD_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    BREAD_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_decode, 256, 0));
    *out = cus * per_cu;
    return BREAD_OK;
}

int bread_launch_moe_decode(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, float *hidden,
                            hipStream_t st)
{
    if (!decode_shape_ok(c->shape)) return BREAD_ERR_SHAPE;
    DecArgs a;
    memset(&a, 0, sizeof(a));
    fill_roles(c->shape, a);
    a.layers = nullptr;
    a.one = to_dec(*L);
    a.L = 1;
    a.x0 = x;
    a.hidden = hidden;
    a.idx_out = c->idx;
    a.w_out = c->w;
    a.gsh_out = c->gsh;
    return launch(c, a, st);
}

int bread_launch_decode_layers(bread_moe_ctx_t *c, const bread_moe_layer_t *layers, int n, float *hidden,
                               int32_t *idx, float *w, float *gsh, hipStream_t st)
{
    if (!decode_shape_ok(c->shape)) return BREAD_ERR_SHAPE;
    BREAD_REQUIRE(n <= c->max_layers, BREAD_ERR_CAPACITY, "more layers than the context holds");
    // the device layer table is re-uploaded only when it changes
    DecLayer *tab = (DecLayer *)c->h_layers;
    bool same = c->n_layers_uploaded == n;
    for (int l = 0; l < n; l++) {
        const DecLayer d = to_dec(layers[l]);
        if (same && memcmp(&tab[l], &d, sizeof(d)) != 0) same = false;
        tab[l] = d;
    }
    if (!same) {
        BREAD_HIP(hipMemcpyAsync(c->d_layers, tab, (size_t)n * sizeof(DecLayer), hipMemcpyHostToDevice, st));
        BREAD_HIP(hipStreamSynchronize(st));
        c->n_layers_uploaded = n;
    }
    DecArgs a;
    memset(&a, 0, sizeof(a));
    fill_roles(c->shape, a);
    a.layers = (const DecLayer *)c->d_layers;
    a.L = n;
    a.x0 = nullptr;
    a.hidden = hidden;
    a.idx_out = idx;
    a.w_out = w;
    a.gsh_out = gsh;
    return launch(c, a, st);
}

size_t bread_decode_layer_record_bytes()
{
    return sizeof(DecLayer);
}

int bread_decode_grid(const bread_moe_shape_t &s)
{
    DecArgs a;
    memset(&a, 0, sizeof(a));
    fill_roles(s, a);
    return a.nR + a.nS + a.nG + a.nD;
}
