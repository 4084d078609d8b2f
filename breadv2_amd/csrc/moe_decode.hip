// moe_decode.hip — persistent MoE decode (one token, B = 1) for gfx950 at the
// Qwen3.5-35B-A3B shape (H 2048, I = I_sh = 512, E <= 256, K <= 8), over one
// layer or a stack of layers per launch.
//
// For each layer l of the launch:  x = RMSNorm(h) * w_l  (or the given x for
// a single pre-normalised layer),  h += MoE_l(x).
//
// Grid: one 1024-thread workgroup per CU (256), all resident at once.
// Workgroup g owns router row g, gate/up rows 2g and 2g+1 of every expert
// slot (slot 0 = shared expert, slot k = routed rank k-1) and output rows
// 8g..8g+7.  Its 16 waves have fixed jobs:
//   waves 0..7   poll the previous layer's output (four columns a thread),
//                normalise it and take the router-row and shared-gate dots
//                of their columns;
//   waves 0..3   poll the router logits (wave 0 then runs softmax/top-k and
//                the combine);
//   waves 1..8   the gate/up rows of routed slot k = wave;
//   waves 4..11  x in 16-bit block fixed point, during the logits exchange;
//   waves 9, 10  shared-expert gate/up rows (before routing is known);
//   waves 9..14  the down-projection bands of the routed slots (8 rows x
//                420 B each);
//   wave 15      certifies the ranks against the logit radii;
//   waves 12..15 the next layer's routing-independent weights (router row,
//                norm weights, shared-gate vector, shared gate/up rows and
//                shared down band), once this layer's h is in, and the first
//                layer's at kernel entry.
// Weights travel HBM -> LDS by gfx950 direct-to-LDS loads, so no wave holds
// weight registers while loads are in flight.  On gfx9, s_waitcnt vmcnt counts
// loads and stores together and in order, so a poll issued behind weight
// loads waits for them: the logit pollers never hold weight loads, and the
// next layer's weights are requested early enough (after this layer's h is
// in) to have landed before that layer's first poll returns.
//
// The gate/up dots multiply the Q4_K nibbles with x in 16-bit block fixed
// point (x ~= s (256 hi + lo), hi and lo int8) by v_dot4_i32_i8, with exact
// integer sums; the min term uses fp32 sums of x.  Everything else is fp32.
//
// Routing is published rank by rank: wave 0 writes expert k to LDS as soon as
// selection pass k ends, and the gate/up and down waves start that slot's
// loads at once, so the top-k passes overlap the expert streams.  The Q6_K
// down weights are unpacked into registers while h is in flight (exact fp16
// quants q - 32 and fp32 run scales d * sc); after it arrives only the dot
// products remain.
//
// Three exchanges per layer cross workgroups, each carried by the data
// itself (no counters, no atomics, no waits for store completion):
//   logits   each workgroup stores its router logit as a 64-bit word tagged
//            with the layer's epoch; every workgroup polls the words directly
//            and runs softmax/top-k itself;
//   h        SwiGLU outputs (K+1) x 512, triple-buffered by layer, and
//   hidden   the layer's output rows, double-buffered by layer parity: a slot
//            holds a signalling-NaN sentinel until its owner stores the value,
//            and readers poll until no sentinel is left.  Arithmetic never
//            produces a signalling NaN, so a stored value never looks unwritten.
//            At the start of layer l the owner re-arms its slots of the hidden
//            buffer layer l writes (last read during layer l-1) and of the h
//            buffer layer l+1 writes (last read during layer l-2): having seen
//            every workgroup's h of layer l-1, it knows all of them are past
//            those reads.  The same wave's next loads wait for the re-arm stores
//            (s_waitcnt counts both in order), and everything it publishes
//            later comes after, so no reader can see a stale value.
// The host passes the number of layers run so far on this context (the
// epoch); tags and parities derive from it.  Data that crosses workgroups is
// written and read with device-coherent (sc1) accesses, so no cache writeback
// or invalidate is needed.  Every wait is bounded and flags a sticky error
// instead of hanging.
//
// Replaces the reference's 45 launches per layer and its host routing round
// trip (one_layer.cu:1812-1983, route_layer :937-992), and the per-layer host
// loop over layers (main.cu:685).
#include <string.h>

#include "bread_internal.h"
#include "quant_dot.h"
#include "route_dev.h"

namespace {

constexpr int G = 256;                   // workgroups, one per CU
constexpr int NT = 1024;                 // threads per workgroup
constexpr int NWV = NT / WAVE;           // 16 waves
constexpr int DH = 2048;
constexpr int DI = 512;
constexpr int NBH = DH / QK;             // Q4_K superblocks per gate/up row
constexpr int GU_ROW = NBH * Q4K_BYTES;  // 1152 B
constexpr int DN_ROW = (DI / QK) * Q6K_BYTES;  // 420 B
constexpr int GR = DI / G;               // gate/up rows per workgroup and slot
constexpr int OR = DH / G;               // output rows per workgroup
constexpr int BAND = OR * DN_ROW;        // one slot's down rows of a workgroup: 3360 B
constexpr int BAND16 = BAND / 16;        // 210 16-byte chunks
constexpr int MAXK = 8;
constexpr int NSLOT = MAXK + 1;
constexpr int NPOLL = 4;                 // waves 0..3 poll the logits, one a lane
constexpr int W_GU = 1;                  // waves 1..8: routed gate/up, slot k = wave
constexpr int W_SH = 9;                  // waves 9, 10: shared gate/up
constexpr int W_DN = 9;                  // waves 9..15: the routed down waves (bands, then the wait for the final ranks)
constexpr int N_DN = NWV - W_DN;         // 7
constexpr int N_DNL = N_DN - 1;          // waves 9..14 load the bands (wave 15 certifies instead)
constexpr int DN_LOADS = (MAXK * BAND16 + N_DNL * WAVE - 1) / (N_DNL * WAVE);  // 5
constexpr int W_XQ = 4;                  // waves 4..11 convert x to fixed point (quant_x)
constexpr int N_XQ = 8;
constexpr int W_PF = 12;                 // waves 12..15 prefetch routing-independent weights, never poll
constexpr int N_XPOLL = 8;               // waves 0..7 poll the previous layer's output (4 columns a thread) and take the router partials
constexpr int N_HPOLL = W_PF;            // waves 0..11 poll the SwiGLU outputs
constexpr int W_RAD = 4;                 // wave 4 publishes the logit's radius
constexpr int W_CERT = NWV - 1;          // wave 15 certifies the routing (a down wave that loads no band)
constexpr uint32_t SPIN_DEFAULT = 1u << 18;  // sleeps a bounded wait allows after its first look
// The layer's RMSNorm here sums the squares as a tree, the reference
// (cpu_rms_norm_weighted, layer_ops.cu:203-212) sequentially, so the two
// inv_rms differ by a factor c: the sequential sum of 2048 non-negative terms
// is within (n-1)u of the exact one, the tree within 17u, so the sums differ
// by at most 1.24e-4 relative, inv_rms (square root, one division, the eps
// add) by at most 6.3e-5.  Every element of x then differs from c times the
// reference's by at most 4u relative.  A common factor keeps the order of the
// logits, so the certificate holds with each radius widened by 4u sum |w x|
// and its tau and spread taken with this bound on |c - 1|; the recomputations
// rebuild the reference's own x (ref_x).
constexpr float CERT_KAPPA = 1.220703125e-4f;  // 2^-13 >= |c - 1|
constexpr int AUX_COHERENT = 16;             // sc1: device-coherent access
constexpr uint32_t SENTINEL = 0x7FA5A5A5u;   // signalling NaN: "not written yet"
// Exchange layouts: every workgroup publishes into lines of its own, so a
// store never invalidates lines other workgroups write (measured on MI355X:
// an all-to-all round over shared lines costs up to 1.8x one over private
// lines).
constexpr int LG_STRIDE = 8;             // tagged logit words: one per 64 B
constexpr int XREC = 32;                 // floats per workgroup record (128 B): output rows, h values

static_assert(DH % G == 0 && DI % G == 0 && GR == 2 && OR == 8, "row ownership assumes 256 workgroups");
static_assert(NBH == 8 && DI / QK == 2, "lane layouts assume H = 2048 and I = 512");
static_assert(BAND % 16 == 0, "down bands are loaded in 16-byte chunks");
static_assert(NPOLL * WAVE == 256 && 4 * N_XPOLL * WAVE == DH, "pollers: one logit a lane; four columns a thread");
static_assert(W_GU + MAXK == W_SH && W_SH + 2 <= NWV, "wave roles");
static_assert(N_XQ * WAVE * 4 == DH && W_XQ >= NPOLL && W_XQ + N_XQ <= NWV,
              "fixed-point x: non-polling waves, four columns a thread");
static_assert(G * ((MAXK + 2) / 2) <= 2 * N_HPOLL * WAVE, "h poll: at most two chunks a thread");
static_assert(NSLOT * DI >= 2 * DH, "S.h holds h and its squares for the exact norm until the ranks are final");
static_assert(BREAD_RSTAT_PER_EXPERT == 1 && BREAD_RSTAT_PAIR == 2 && BREAD_RSTAT_EXACT == 3,
              "certify's return values index the routing counters");

// Trace points recorded per (workgroup, layer) when a trace buffer is given.
enum {
    TP_START = 0,   // layer entered
    TP_XREADY = 1,  // previous layer's output seen, x in LDS, router partials taken
    TP_LOGIT = 2,   // own logit published
    TP_POLLED = 3,  // every logit seen
    TP_RANK1 = 4,   // rank-1 expert known
    TP_ROUTED = 5,  // every rank known, weights in LDS
    TP_DDOT = 6,    // wave 0's down dots done
    TP_COMB = 7,    // down dots of every wave done (after the barrier)
    TP_HREADY = 8,  // every h seen
    TP_OUT = 9,     // output rows stored
    TP_HLAST = 10,  // the last routed slot's gate/up wave stored its h
    TP_DNIN = 11,   // every routed down band in LDS (seen by wave 0)
    TP_PASSES = 12, // last selection pass done
    TP_CERT = 13,   // ranks final (certified, or recomputed)
    TP_XDOT = 14,   // uncertified: own logit in the reference's order done
    TP_XPOLL = 15,  // uncertified: every such logit seen
    TP_PREP = 16,   // certificate wave: radii and maxima settled
    TP_READY = 17,  // certificate wave: every pass seen
    TP_N = 18
};

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
    uint32_t epoch0;         // layers run on this context before this launch
    int hphase0;             // epoch0 % 3 (kept separately: 2^32 is not a multiple of 3)
    const float *x0;         // non-NULL: layer 0 input given (already normalised)
    float *hidden;           // [H] caller's hidden: input of layer 0, output of every layer
    float eps;
    uint64_t *tlogits;       // [256][LG_STRIDE] tagged logits
    uint64_t *texact;        // [256][LG_STRIDE] tagged exact logits (uncertified layers)
    uint64_t *tradius;       // [256][LG_STRIDE] tagged radii of the logits
    float *xbuf;             // [2][G][XREC] layer outputs by parity: rows 8g..8g+7 of workgroup g
    float *hbuf;             // [3][G][XREC] SwiGLU outputs by layer mod 3: [slot][rows 2g, 2g+1]
    int32_t *idx_out;        // [L][rstride][K] or NULL (this token's record of each layer)
    float *w_out;            // [L][rstride][K] or NULL
    float *gsh_out;          // [L][rstride] or NULL
    int rstride;             // tokens per layer record of the routing outputs
    bread_decode_sync *sync;
    uint64_t *trace;         // [G][L][TP_N] or NULL
    int E, K;
    uint32_t spin;           // sleeps a bounded wait allows after its first look
};

struct Smem {
    float x[DH];                       // normalised input of the layer
    uint32_t xqh[DH / 4];              // x in 16-bit block fixed point: high bytes, 4 columns a word
    uint32_t xql[DH / 4];              // low bytes
    float xqs[DH / 32];                // block scales (32 columns)
    float xsum[DH / 16];               // fp32 sums of 16-column runs of x
    float nw[DH];                      // RMSNorm weights (prefetched)
    float h[NSLOT * DI];               // SwiGLU outputs of every slot
    uint32_t down[MAXK * BAND / 4];    // routed down bands, slot k at (k - 1) * BAND
    uint32_t sdown[2][BAND / 4];       // shared down band, by layer parity (prefetched a layer ahead)
    float wrow[DH];                    // router row g (prefetched)
    uint16_t shg[DH];                  // shared-expert gate vector (prefetched)
    uint4 shw[2][4][WAVE];             // shared gate/up rows: [row][hg, qg, hu, qu][lane] (prefetched)
    uint4 gu[MAXK][4 * GR][WAVE];      // routed gate/up rows: [slot-1][4 row + (hg, qg, hu, qu)][lane]
    __attribute__((aligned(16))) float lg[256];  // router logits of the layer (scratch of the exact softmax)
    float red[NWV];                    // sum-of-squares partials
    float rl[N_XPOLL], gl[N_XPOLL];    // router / shared-gate partials of the polling waves
    float rbw[N_XPOLL];                // their radius terms
    float lr[256];                     // radii of the logits: |logit - reference sum| <= lr
    float2 smax;                       // the max and sum of the selection softmax
    float own_lg;                      // this workgroup's logit, as published
    float dot[NSLOT][OR];              // down dots
    float hown[OR];                    // this workgroup's rows of h before the layer
    int idx[MAXK];                     // routed experts, rank order
    uint32_t key[MAXK];                // their probability keys
    float w[MAXK];                     // their weights
    float sgsh;                        // sigmoid of the shared-gate logit
    float gsh;                         // the shared-gate logit
    int nready;                        // ranks published in idx
    int wready;                        // key, w and smax of the ranks written (after the passes)
    int lgcnt;                         // polling waves done with the logits
    int rlcnt;                         // x-polling waves whose router partials are in S.rl
    int rbcnt;                         // x-polling waves whose radius terms are in S.rbw
    int dncnt;                         // down waves whose bands are in LDS
    int gucnt;                         // routed gate/up waves whose weights are in LDS
    int xqcnt;                         // waves done converting their part of x (quant_x)
    int gudone;                        // routed gate/up waves done computing
    int ddcnt;                         // waves done with their down dots (last layer of a launch)
    int cert;                          // 0: ranks may still change; 1: certified; 2: recomputed exactly
    int abort;                         // a wait failed: the workgroup leaves
    int expired;                       // a wait on another wave of the workgroup ran out
    uint32_t spin;                     // DecArgs::spin
};
// more than half of a CU's 160 KB, so the dispatcher puts one workgroup per CU
static_assert(sizeof(Smem) > 80 * 1024 && sizeof(Smem) <= 160 * 1024, "LDS footprint");

// ---------------------------------------------------------------- memory helpers

// An empty asm hides v's value from the optimiser, so per-lane address math
// that depends on it is recomputed where it is used instead of being hoisted
// out of the layer loop and kept live (spilled) across the whole kernel.
__device__ __forceinline__ int opaque(int v)
{
    asm volatile("" : "+v"(v));
    return v;
}

// Direct-to-LDS load (gfx950 global_load_lds_dwordx4): lane i of the wave
// writes its 16 bytes at lds_wave_base + 16 i; the wave base must be uniform.
// The data is in LDS once the issuing wave's vmcnt drains.
__device__ __forceinline__ void lds_load16(const void *src, void *lds_wave_base)
{
    __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, 0);
}

__device__ __forceinline__ void cstore(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void cstore2(float *p, float a, float b)
{
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p),
                       ((uint64_t)__builtin_bit_cast(uint32_t, b) << 32) | __builtin_bit_cast(uint32_t, a),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS flags shared by the waves of the workgroup.  LDS performs one wave's
// accesses in order, so data written before a flag is seen by a wave that
// has seen the flag; the signal fences keep the compiler from reordering.
__device__ __forceinline__ int lds_get(const int *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void lds_put(int *p, int v)
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void lds_add(int *p, int v)
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A wait on another wave of the workgroup ran out: the workgroup leaves at
// its next check, which flags BREAD_DEV_ERR_LOCAL.
__device__ __forceinline__ void lds_expire(Smem &S)
{
    lds_put(&S.expired, 1);
    lds_put(&S.abort, 1);
}

// Wave-level bounded wait for an LDS flag; false if the workgroup aborts or
// the wait runs out (lds_expire).  A look is one LDS read with no sleep
// after it, and the abort flag is read every 16th look: measured, the
// single-layer launch is 0.19 us shorter than with a 64-cycle sleep and the
// abort flag read at every look (longer sleeps cost 0.2-0.4 us).  slow:
// sleep between looks (for waits expected to last microseconds).
__device__ __forceinline__ bool lds_wait(Smem &S, const int *p, int target, bool slow = false)
{
    const uint32_t lim = S.spin;
    for (uint32_t it = 0;; it++) {
        if (lds_get(p) >= target) {
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            return true;
        }
        if ((it & 15) == 15 && lds_get(&S.abort)) return false;
        if (it >= lim) break;
        if (slow) __builtin_amdgcn_s_sleep(8);
        else __builtin_amdgcn_s_sleep(0);
    }
    lds_expire(S);
    return false;
}

// Called by one lane.
__device__ __forceinline__ void trace_here(const DecArgs &a, int l, int tp)
{
    if (a.trace) a.trace[((size_t)blockIdx.x * a.L + l) * TP_N + tp] = wall_clock64();
}

__device__ __forceinline__ void trace_point(const DecArgs &a, int l, int tp)
{
    if (threadIdx.x == 0) trace_here(a, l, tp);
}

// The same, from the calling wave's lane 0.
__device__ __forceinline__ void trace_point_lane0(const DecArgs &a, int l, int tp)
{
    if (lane_id() == 0) trace_here(a, l, tp);
}

// The layer record is the same for the whole grid: keep it in scalar registers.
__device__ __forceinline__ DecLayer load_layer(const DecArgs &a, int l)
{
    // the table is read through the constant address space: scalar loads,
    // counted apart from the wave's vector loads, so reading a record does
    // not wait for the weight loads in flight
    typedef const __attribute__((address_space(4))) uint64_t *ConstWords;
    static_assert(sizeof(DecLayer) % 8 == 0, "layer record in 64-bit words");
    DecLayer d = a.one;
    if (a.layers) {
        const ConstWords p = (ConstWords)uniform_ptr(a.layers + l);
        uint64_t w[sizeof(DecLayer) / 8];
#pragma unroll
        for (int i = 0; i < (int)(sizeof(DecLayer) / 8); i++) w[i] = p[i];
        __builtin_memcpy(&d, w, sizeof(d));
    }
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

__device__ __forceinline__ bool unwritten(float v)
{
    return __builtin_bit_cast(uint32_t, v) == SENTINEL;
}

// Per-thread bounded poll of 4 coherent floats at byte offset off of a
// buffer until none of the checked ones (all four, or the low two when hi is
// false) is the sentinel, sleeping at most lim times.  Returns false on
// time-out (flagging the error) or when another workgroup flagged one.
__device__ __forceinline__ bool poll4(bread_decode_sync *s, __amdgpu_buffer_rsrc_t r, uint32_t off, float4 &v,
                                      uint32_t lim, bool hi = true)
{
    for (uint32_t it = 0;; it++) {
        v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX_COHERENT));
        if (!unwritten(v.x) && !unwritten(v.y) && !(hi && (unwritten(v.z) || unwritten(v.w)))) return true;
        if (it >= lim) break;
        if ((it & 63) == 63 && has_error(s)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    flag_error(s, BREAD_DEV_ERR_HWAIT);
    return false;
}

// Exchange words of the routing: the 32-bit layer tag (bits 63-32, from the
// context's layer epoch) and an fp32 value (31-0), one word per workgroup in
// its own 64-byte line.  Three kinds: the fast logit, its radius (stored a
// little later, in a separate line, so that the logit's line is written
// once) and the logit in the reference's order (only in layers whose
// routing is not certified).  The logit and radius words are rewritten every
// layer; an exact-logit word can be many layers old, which 32-bit tags tell
// apart (the host clears the words before the count wraps).
__device__ __forceinline__ uint64_t tag_word(uint32_t tag, float v)
{
    return ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ void publish(uint64_t *p, uint32_t tag, float v)
{
    __hip_atomic_store(p, tag_word(tag, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-thread bounded poll of one tagged word of this layer.
__device__ __forceinline__ uint64_t load_word(const uint64_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-thread bounded poll of one tagged word of this layer, w its first
// read, sleeping at most lim times.
__device__ __forceinline__ bool poll_word_from(bread_decode_sync *s, const uint64_t *p, uint32_t tag, float &v,
                                               uint64_t w, uint32_t lim)
{
    for (uint32_t it = 0;; it++) {
        if ((uint32_t)(w >> 32) == tag) {
            v = __builtin_bit_cast(float, (uint32_t)w);
            return true;
        }
        if (it >= lim) break;
        if ((it & 63) == 63 && has_error(s)) return false;
        __builtin_amdgcn_s_sleep(1);
        w = load_word(p);
    }
    flag_error(s, BREAD_DEV_ERR_LWAIT);
    return false;
}

__device__ __forceinline__ bool poll_word(bread_decode_sync *s, const uint64_t *p, uint32_t tag, float &v,
                                          uint32_t lim)
{
    return poll_word_from(s, p, tag, v, load_word(p), lim);
}

// ---------------------------------------------------------------- routing

// Selection over E <= 256 probabilities, lane i holding entries i + 64 v.
// A probability key (bits + 2, or 1 for NaN, 0 for none; below 2^30) is
// packed with its register number as (key << 2) | (3 - v): within a lane the
// packed keys are distinct, and across the wave the unsigned maximum is the
// largest probability with, among equal ones, the lowest v; the lowest lane
// holding that maximum then has the lowest index i = lane + 64 v.  That is
// cpu_topk's strict '>' scan from i = 0 (layer_ops.cu:231-243).  Each lane
// keeps its four packed keys sorted, so a pass is one wave max, one ballot
// and a shift in the winning lane.  (A radix search for the K-th largest key
// finds the whole set without passes, but on gfx950 its ballot counts chain
// through VCC and took longer than the eight passes, and the passes publish
// rank 1 far sooner.)
struct Sel {
    uint32_t k0, k1, k2, k3;  // packed keys, descending
};

__device__ __forceinline__ void cswap(uint32_t &a, uint32_t &b)
{
    const uint32_t hi = umax32(a, b), lo = a ^ b ^ hi;
    a = hi;
    b = lo;
}

__device__ __forceinline__ Sel sel_init(const uint32_t (&key)[4])
{
    Sel s{(key[0] << 2) | 3u, (key[1] << 2) | 2u, (key[2] << 2) | 1u, key[3] << 2};
    cswap(s.k0, s.k1);
    cswap(s.k2, s.k3);
    cswap(s.k0, s.k2);
    cswap(s.k1, s.k3);
    cswap(s.k1, s.k2);
    return s;
}

// One pass: returns the winning index; M gets its probability key.
__device__ __forceinline__ int sel_pass(Sel &s, int lane, uint32_t &M)
{
    const uint32_t top = wave_max_u32(s.k0);
    const uint64_t b = __builtin_amdgcn_ballot_w64(s.k0 == top);
    const int wl = (int)__builtin_ctzll(b);
    const bool w = lane == wl;
    s.k0 = w ? s.k1 : s.k0;
    s.k1 = w ? s.k2 : s.k1;
    s.k2 = w ? s.k3 : s.k2;
    s.k3 = w ? 0u : s.k3;
    M = top >> 2;
    return wl + WAVE * (int)(3u - (top & 3u));
}

// ---------------------------------------------------------------- gate/up

// A gate/up lane owns qs chunk c = lane%8 of superblock sbl = lane/8 of a row:
// x columns base + [0,16) (low nibbles) and base + 32 + [0,16) (high nibbles),
// base = sbl*256 + 64*(c/2) + 16*(c%2).  The 64 lanes cover all H columns once.
__device__ __forceinline__ int gu_base(int lane)
{
    const int c = lane & 7;
    return (lane >> 3) * QK + 64 * (c >> 1) + 16 * (c & 1);
}

// Direct-to-LDS loads of gate/up rows r0 .. r0+N of one expert: w[4i + q]
// receives, for row r0+i, q = 0: the gate superblock head of the lane,
// 1: its gate qs chunk, 2/3: the same for up.
template <int N>
__device__ __forceinline__ void gu_issue(const uint8_t *gbase, const uint8_t *ubase, int r0, uint4 (*w)[WAVE])
{
    const int lane = opaque(lane_id());
    const uint32_t oh = (uint32_t)((lane >> 3) * Q4K_BYTES);
    const uint32_t oq = oh + 16u + 16u * (uint32_t)(lane & 7);
#pragma unroll
    for (int i = 0; i < N; i++) {
        const uint8_t *gr = gbase + (size_t)(r0 + i) * GU_ROW, *ur = ubase + (size_t)(r0 + i) * GU_ROW;
        lds_load16(gr + oh, &w[4 * i + 0][0]);
        lds_load16(gr + oq, &w[4 * i + 1][0]);
        lds_load16(ur + oh, &w[4 * i + 2][0]);
        lds_load16(ur + oq, &w[4 * i + 3][0]);
    }
}

// x of the layer in 16-bit block fixed point for the gate/up integer dots
// (q4k_chunk_dot_q16): per 32-column block b, s_b = max|x| / 32511 and
// x_i ~= s_b * q_i with q_i = rint(x_i / s_b) = 256 hi_i + lo_i, hi in
// [-127, 127], lo in [-128, 127]; the error is at most s_b / 2 (relative
// 1.5e-5 of the block maximum).  Also the fp32 sum of every 16-column run
// (the Q4_K min term).  Thread t (0..511) converts columns 4t..4t+3; eight
// threads share a block, four a run.
__device__ __forceinline__ void quant_x(Smem &S, int t)
{
    const float4 v = *reinterpret_cast<const float4 *>(&S.x[4 * t]);
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = fmaxf(m, dpp_f<0xB1>(m));   // quad_perm [1,0,3,2]
    m = fmaxf(m, dpp_f<0x4E>(m));   // quad_perm [2,3,0,1]
    m = fmaxf(m, dpp_f<0x141>(m));  // row_half_mirror: the 8-lane block
    const float inv = m > 0.f ? 32511.0f / m : 0.f;
    const float xv[4] = {v.x, v.y, v.z, v.w};
    uint32_t hw = 0, lw = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int q = __float2int_rn(xv[k] * inv);
        const int hi = (q + 128) >> 8;
        const int lo = q - 256 * hi;
        hw |= ((uint32_t)hi & 0xFFu) << (8 * k);
        lw |= ((uint32_t)lo & 0xFFu) << (8 * k);
    }
    S.xqh[t] = hw;
    S.xql[t] = lw;
    if ((t & 7) == 0) S.xqs[t >> 3] = m / 32511.0f;
    float r = (v.x + v.y) + (v.z + v.w);
    r += dpp_f<0xB1>(r);
    r += dpp_f<0x4E>(r);
    if ((t & 3) == 0) S.xsum[t >> 2] = r;
}

// Gate/up + SwiGLU of the N rows staged by gu_issue (the wave's own loads
// must have landed); every lane gets the results.  The dots run on the
// fixed-point x of quant_x with integer products (q4k_chunk_dot_q16).
template <int N>
__device__ __forceinline__ void gu_compute(const Smem &S, const uint4 (*w)[WAVE], float (&out)[N])
{
    const int lane = opaque(lane_id());
    const int base = gu_base(lane);
    const uint32_t j = (uint32_t)(lane & 7) >> 1;
    const uint4 lh = *reinterpret_cast<const uint4 *>(&S.xqh[base >> 2]);
    const uint4 ll = *reinterpret_cast<const uint4 *>(&S.xql[base >> 2]);
    const uint4 hh = *reinterpret_cast<const uint4 *>(&S.xqh[(base >> 2) + 8]);
    const uint4 hl = *reinterpret_cast<const uint4 *>(&S.xql[(base >> 2) + 8]);
    const float2 sc = *reinterpret_cast<const float2 *>(&S.xqs[base >> 5]);  // blocks 2j, 2j+1
    const float sxl = S.xsum[base >> 4], sxh = S.xsum[(base >> 4) + 2];
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float gt = wave_sum(
            q4k_chunk_dot_q16(w[4 * i][lane], w[4 * i + 1][lane], j, lh, ll, hh, hl, sc.x, sc.y, sxl, sxh));
        const float up = wave_sum(
            q4k_chunk_dot_q16(w[4 * i + 2][lane], w[4 * i + 3][lane], j, lh, ll, hh, hl, sc.x, sc.y, sxl, sxh));
        out[i] = silu_mul(gt, up);
    }
}

// ---------------------------------------------------------------- down

// Down unit u: slot u/2, rows 4*(u%2) .. +4 of the workgroup, 16 lanes a row;
// a lane owns superblock b = (lane/8)%2, half n = (lane/4)%2 and l in
// [8t, 8t+8), t = lane%4 (the Q6_K unit of quant_dot.h), i.e. the 32 weights
// at columns b*256 + 128n + 32s + 8t + k, s < 4, k < 8.
//
// Pre-decode: the lane's 32 quants q - 32 as fp16 pairs (exact: the byte
// placed under the fp16 exponent of 1024 gives 1024 + q, and subtracting
// 1056 leaves q - 32), q[2i] in the low half of word i, with the group
// scale d * sc (exact in fp32: 11 x 8 bits) of each run s of 8 weights.  The
// dot then takes sum_s (d sc_s) sum_k (q - 32) h with the fp16 operand
// widened inside the FMA (v_fma_mix_f32): the weight is the dequantised
// d * sc * (q - 32) of dequant_q4k_cpu.c:155-170 with the product rounded
// once per run instead of once per weight, and the pre-decode costs one
// permute and half a packed subtraction per weight instead of a conversion
// and an FMA.
typedef _Float16 dn_half2 __attribute__((ext_vector_type(2)));

struct DnWeights {
    uint32_t q[16];  // fp16 pairs (q - 32): word 4s + 2 half + j holds k = 4 half + 2j, +1 of run s
    float ds[4];     // d * sc of run s
};

__device__ __forceinline__ uint32_t q6_pair_f16(uint32_t q, uint32_t sel)
{
    const uint32_t p = __builtin_amdgcn_perm(0x64646464u, q, sel);
    const dn_half2 v = __builtin_bit_cast(dn_half2, p) - (dn_half2){(_Float16)1056.0f, (_Float16)1056.0f};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ void down_predecode(const Smem &S, int u, int sb, DnWeights &w)
{
    const int lane = opaque(lane_id());
    const int slot = u >> 1;
    const int row = 4 * (u & 1) + (lane >> 4);
    const int b = (lane >> 3) & 1, n = (lane >> 2) & 1, t = lane & 3;
    const uint32_t *band = slot == 0 ? S.sdown[sb] : S.down + (slot - 1) * (BAND / 4);
    // the superblock starts 2 b bytes past a word boundary (rows are 420
    // bytes, superblocks 210), as do all of its fields the lane reads:
    // words from one aligned base with constant offsets, then byte shifts
    const uint32_t ob = (uint32_t)(row * DN_ROW + b * Q6K_BYTES);
    const uint32_t sh = ob & 3u;
    const uint32_t *p = band + (ob >> 2);
    const uint32_t *pa = p + 16 * n + 2 * t, *pb = p + 8 * n + 2 * t, *pc = p + 2 * n;
    const uint2 ql0 = make_uint2(__builtin_amdgcn_alignbyte(pa[1], pa[0], sh), __builtin_amdgcn_alignbyte(pa[2], pa[1], sh));
    const uint2 ql1 = make_uint2(__builtin_amdgcn_alignbyte(pa[9], pa[8], sh), __builtin_amdgcn_alignbyte(pa[10], pa[9], sh));
    const uint2 qh = make_uint2(__builtin_amdgcn_alignbyte(pb[33], pb[32], sh), __builtin_amdgcn_alignbyte(pb[34], pb[33], sh));
    const uint2 scw = make_uint2(__builtin_amdgcn_alignbyte(pc[49], pc[48], sh), __builtin_amdgcn_alignbyte(pc[50], pc[49], sh));
    const float d = h2f((p[52] >> (8u * sh)) & 0xFFFFu);
    const uint32_t i2 = (uint32_t)t >> 1;
#pragma unroll
    for (int s = 0; s < 4; s++) w.ds[s] = d * q6k_scale(scw, i2 + 2 * s);
#pragma unroll
    for (int half = 0; half < 2; half++) {
        uint32_t q[4];
        q6k_unpack(half ? ql0.y : ql0.x, half ? ql1.y : ql1.x, half ? qh.y : qh.x, q);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            // bytes 0, 1 and 2, 3 of q[s] under the fp16 exponent byte 0x64
            w.q[4 * s + 2 * half] = q6_pair_f16(q[s], 0x04010400u);
            w.q[4 * s + 2 * half + 1] = q6_pair_f16(q[s], 0x04030402u);
        }
    }
}

// Down units beyond the 16 waves (u >= 16, only for K = 8) are pre-decoded by
// waves 1 and 2 into their own gate/up staging slot of LDS, free once their
// gate/up is done: the quant words of lane i at uint4 [0..3][i], the run
// scales at [4][i].
__device__ __forceinline__ void predecode_to_lds(const Smem &S, int u, int sb, uint4 (*dst)[WAVE])
{
    DnWeights w;
    down_predecode(S, u, sb, w);
    const int lane = opaque(lane_id());
#pragma unroll
    for (int q = 0; q < 4; q++) dst[q][lane] = make_uint4(w.q[4 * q], w.q[4 * q + 1], w.q[4 * q + 2], w.q[4 * q + 3]);
    dst[4][lane] = make_uint4(__builtin_bit_cast(uint32_t, w.ds[0]), __builtin_bit_cast(uint32_t, w.ds[1]),
                              __builtin_bit_cast(uint32_t, w.ds[2]), __builtin_bit_cast(uint32_t, w.ds[3]));
}

// Position of column c of a slot's SwiGLU row in LDS.  A down lane reads its
// 32 columns as 8 float4 chunks j = 2s + (k >= 4); the 16 lane positions
// (b, n, t) of one chunk are stored contiguously, so each 16-byte read of a
// wave covers 256 consecutive bytes (the four rows' lanes read the same
// addresses, which LDS broadcasts).  Measured on MI355X: 81 against 256
// cycles per read instruction with 16 waves reading, for the plain layout's
// stride.  Columns 2w, 2w+1 stay adjacent.
__device__ __forceinline__ int hpos(int c)
{
    const int b = c >> 8, n = (c >> 7) & 1, s = (c >> 5) & 3, t = (c >> 3) & 3, k = c & 7;
    return 64 * (2 * s + (k >> 2)) + 32 * b + 16 * n + 4 * t + (k & 3);
}

// fp16 weight pair times two fp32 values, accumulated in fp32 (v_fma_mix_f32)
__device__ __forceinline__ float dn_fma2(uint32_t wp, float x0, float x1, float a)
{
    const dn_half2 h = __builtin_bit_cast(dn_half2, wp);
    return fmaf((float)h.y, x1, fmaf((float)h.x, x0, a));
}

__device__ __forceinline__ float down_acc(const Smem &S, int u, const DnWeights &w)
{
    const int lane = opaque(lane_id());
    const int slot = u >> 1;
    const int b = (lane >> 3) & 1, n = (lane >> 2) & 1, t = lane & 3;
    const float *hs = S.h + slot * DI + 32 * b + 16 * n + 4 * t;
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const float4 v0 = *reinterpret_cast<const float4 *>(hs + 128 * s);
        const float4 v1 = *reinterpret_cast<const float4 *>(hs + 128 * s + 64);
        float r = dn_fma2(w.q[4 * s], v0.x, v0.y, 0.f);
        r = dn_fma2(w.q[4 * s + 1], v0.z, v0.w, r);
        r = dn_fma2(w.q[4 * s + 2], v1.x, v1.y, r);
        r = dn_fma2(w.q[4 * s + 3], v1.z, v1.w, r);
        acc = fmaf(w.ds[s], r, acc);
    }
    return sum16(acc);
}

__device__ __forceinline__ void down_dot(Smem &S, int u, const DnWeights &w)
{
    const int lane = opaque(lane_id());
    const float acc = down_acc(S, u, w);
    if ((lane & 15) == 0) S.dot[u >> 1][4 * (u & 1) + (lane >> 4)] = acc;
}

__device__ __forceinline__ void down_dot_lds(Smem &S, int u, const uint4 (*src)[WAVE])
{
    const int lane = opaque(lane_id());
    DnWeights w;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint4 v = src[q][lane];
        w.q[4 * q] = v.x; w.q[4 * q + 1] = v.y; w.q[4 * q + 2] = v.z; w.q[4 * q + 3] = v.w;
    }
    const uint4 v = src[4][lane];
    w.ds[0] = __builtin_bit_cast(float, v.x); w.ds[1] = __builtin_bit_cast(float, v.y);
    w.ds[2] = __builtin_bit_cast(float, v.z); w.ds[3] = __builtin_bit_cast(float, v.w);
    const float acc = down_acc(S, u, w);
    if ((lane & 15) == 0) S.dot[u >> 1][4 * (u & 1) + (lane >> 4)] = acc;
}

// ---------------------------------------------------------------- fixed weights

// Routing-independent weights of a layer into LDS, by waves 12..15 (256
// lanes, 8 direct-to-LDS loads each): router row g, norm weights, shared-gate
// vector, shared gate/up rows and the shared down band (into sdown[sb]).
// These waves never poll and never load a layer's input, so the loads delay
// no exchange: gfx9 completes a wave's loads in order, and the layer-record
// load at the top of each layer is followed by a wait for all of the wave's
// loads.
__device__ __forceinline__ void prefetch(Smem &S, const DecLayer &Ly, int g, int E, int wid, int sb)
{
    const int lane = opaque(lane_id());
    if (wid < W_PF) return;
    const int w4 = wid - W_PF;           // 0..3
    const int c = WAVE * w4 + lane;      // 0..255
#pragma unroll
    for (int i = 0; i < 2; i++) {        // 16-byte chunk c + 256 i of a 2048-float row
        if (g < E) lds_load16(Ly.router + (size_t)g * DH + 4 * (c + 256 * i), &S.wrow[4 * (WAVE * w4 + 256 * i)]);
        if (Ly.norm_w) lds_load16(Ly.norm_w + 4 * (c + 256 * i), &S.nw[4 * (WAVE * w4 + 256 * i)]);
    }
    if (Ly.shg) lds_load16(Ly.shg + 8 * c, &S.shg[8 * WAVE * w4]);
    // shared gate/up: wave w4 loads row w4/2, gate (w4 even) or up
    const int r = GR * g + (w4 >> 1);
    const uint8_t *base = ((w4 & 1) ? Ly.up_sh : Ly.gate_sh) + (size_t)r * GU_ROW;
    const uint32_t oh = (uint32_t)((lane >> 3) * Q4K_BYTES);
    const uint32_t oq = oh + 16u + 16u * (uint32_t)(lane & 7);
    lds_load16(base + oh, &S.shw[w4 >> 1][2 * (w4 & 1)][0]);
    lds_load16(base + oq, &S.shw[w4 >> 1][2 * (w4 & 1) + 1][0]);
    if (c < BAND16) lds_load16(Ly.down_sh + (size_t)g * BAND + 16 * c, &S.sdown[sb][4 * WAVE * w4]);
}

// ---------------------------------------------------------------- exact routing

// w[k] = w[k] * x[k] (rounded) for the DH columns, by one wave; its later LDS
// loads see the stores.
__device__ __forceinline__ void products_in_place(float *w, const float *x, int lane)
{
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < DH / (4 * WAVE); i++) {
        const int o = 4 * (WAVE * i + lane);
        const float4 xv = *reinterpret_cast<const float4 *>(&x[o]);
        const float4 wv = *reinterpret_cast<const float4 *>(&w[o]);
        *reinterpret_cast<float4 *>(&w[o]) = make_float4(wv.x * xv.x, wv.y * xv.y, wv.z * xv.z, wv.w * xv.w);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The uncertified case, run by wave W_CERT of every workgroup (all make the
// same decision from the same published data): the workgroup's own logit in the
// reference's order, ((0 + w_0 x_0) + w_1 x_1) + ... (one_layer.cu:969-971;
// every lane runs the same chain over the router row and x in LDS), exchanged
// through the exact-logit words; then the host's softmax arithmetic
// (softmax_keys_exact) and cpu_topk's passes on the exact logits: indices and
// weights as the reference computes them.  Returns false if a wait failed.
__device__ bool exact_routing(const DecArgs &a, const DecLayer &Ly, Smem &S, int g, int E, int K, uint32_t tag32,
                              int lane, int l, bool reload)
{
    float acc = 0.f;
    if (g < E) {
        if (reload) {
            // S.wrow held other rows (certify): this workgroup's again
#pragma unroll
            for (int i = 0; i < DH / (4 * WAVE); i++)
                lds_load16(Ly.router + (size_t)g * DH + 4 * (WAVE * i + lane), &S.wrow[4 * WAVE * i]);
            __builtin_amdgcn_s_waitcnt(0);
        }
        // the products w_k x_k in place, then their sequential sum
        products_in_place(S.wrow, S.x, lane);
        acc = seq_sum_lds(S.wrow, DH);
        if (lane == 0) publish(a.texact + LG_STRIDE * g, tag32, acc);
    }
    trace_point_lane0(a, l, TP_XDOT);
    float p[4];
    bool ok = true;
    const uint32_t lim = S.spin;
#pragma unroll
    for (int vv = 0; vv < 4; vv++) {
        const int e = lane + WAVE * vv;
        p[vv] = -__builtin_inff();
        if (e < E) {
            if (e == g) {
                p[vv] = acc;
            } else {
                float v = 0.f;
                ok = poll_word(a.sync, a.texact + LG_STRIDE * e, tag32, v, lim) && ok;
                p[vv] = v;
            }
        }
    }
    if (__builtin_amdgcn_ballot_w64(!ok)) return false;
    trace_point_lane0(a, l, TP_XPOLL);
    uint32_t key[4];
    softmax_keys_exact<4>(p, E, key, S.lg);
    for (int k = 0; k < K; k++) {
        uint32_t M;
        const int win = select_round<4>(key, M);
        if (lane == 0) {
            S.idx[k] = win < E ? win : 0;
            S.key[k] = M;
        }
    }
    return true;
}

// ---------------------------------------------------------------- certificate

// DPP move with `old` in the lanes that have no source.
template <int CTRL>
__device__ __forceinline__ float dpp_or(float old, float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_f(float v, int i)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), i));
}

// Wave W_CERT, once every logit is polled: every logit's radius read (four
// words a lane, in flight together) into S.lr, and the maxima over all
// experts: x = max radius, y = max |logit|, z = 1 if every logit and radius
// is finite and |logit| <= 64, w = 1 unless a wait failed.
__device__ float4 cert_prepare(const DecArgs &a, Smem &S, int E, uint32_t tag32, float (&lv)[4])
{
    const int lane = opaque(lane_id());
#pragma unroll
    for (int vv = 0; vv < 4; vv++) lv[vv] = -__builtin_inff();
    if (!lds_wait(S, &S.lgcnt, NPOLL)) return make_float4(0.f, 0.f, 0.f, 0.f);
    uint64_t w[4];
#pragma unroll
    for (int vv = 0; vv < 4; vv++) {
        const int e = lane + WAVE * vv;
        w[vv] = e < E ? load_word(a.tradius + LG_STRIDE * e) : tag_word(tag32, 0.f);
    }
    bool ok = false;
    const uint32_t lim = S.spin;
    for (uint32_t it = 0;; it++) {
        bool mine = true;
#pragma unroll
        for (int vv = 0; vv < 4; vv++) mine = mine && (uint32_t)(w[vv] >> 32) == tag32;
        if (__builtin_amdgcn_ballot_w64(!mine) == 0) {
            ok = true;
            break;
        }
        if (it >= lim) break;
        if ((it & 63) == 63 && has_error(a.sync)) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int vv = 0; vv < 4; vv++) {
            const int e = lane + WAVE * vv;
            if ((uint32_t)(w[vv] >> 32) != tag32) w[vv] = load_word(a.tradius + LG_STRIDE * e);
        }
    }
    if (!ok) {
        if (!has_error(a.sync)) flag_error(a.sync, BREAD_DEV_ERR_LWAIT);
        return make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float rm = 0.f, am = 0.f;
    bool fin = true;
#pragma unroll
    for (int vv = 0; vv < 4; vv++) {
        const int e = lane + WAVE * vv;
        if (e < E) {
            const float re = __builtin_bit_cast(float, (uint32_t)w[vv]);
            S.lr[e] = re;
            const float le = S.lg[e];
            lv[vv] = le;
            fin = fin && __builtin_isfinite(le) && __builtin_isfinite(re);
            rm = fmaxf(rm, re);
            am = fmaxf(am, fabsf(le));
        }
    }
    rm = wave_max(rm);
    am = wave_max(am);
    const bool sane = __builtin_amdgcn_ballot_w64(!fin) == 0 && am <= 64.f;
    return make_float4(rm, am, sane ? 1.f : 0.f, 1.f);
}

// The softmax rounding margin tau = 12 u (1 + max|l| + R) of the reference's
// logits (route_dev.h), taken from the fast logits' maximum magnitude am and
// largest radius rm with the norm's factor (CERT_KAPPA) on both sides.
__device__ __forceinline__ float cert_tau(float am, float rm)
{
    return 12.f * CERT_U * (1.f + CERT_KAPPA) * (1.f + (am + 2.f * rm) * (1.f + 2.f * CERT_KAPPA));
}

// The reference's spread limit (CERT_SPREAD) on the fast logits of ranks 0
// and K-1, radii and the norm's factor included.
__device__ __forceinline__ bool cert_spread_ok(float l0, float lk1, float rm)
{
    return l0 - lk1 + 2.f * rm <= CERT_SPREAD * (1.f - CERT_KAPPA);
}

// Wave W_CERT's one-radius certificate on wave 0's ranks as they arrive:
// each new rank's logit against the previous rank's (gap > T = 2 R_max +
// tau), and once rank K-1 is in, no expert outside the top K within T of it
// (counted, from the logits cert_prepare left in registers: exactly K
// logits >= l_{K-1} - T).  Strict gaps beyond every
// rounding mean the reference's order is the same.  Returns 1 (certified),
// 0 (not: the full certificate decides) or -1 (the workgroup aborts).
__device__ int cert_fast(Smem &S, int E, int K, float4 cm, const float (&lv)[4])
{
    const int lane = opaque(lane_id());
    const float T = 2.f * cm.x + cert_tau(cm.y, cm.x);
    bool good = cm.z != 0.f;
    int have = 0;
    float prev = 0.f, first = 0.f;
    const uint32_t lim = S.spin;
    for (uint32_t it = 0;; it++) {
        const int n = lds_get(&S.nready);
        if (n > have) {
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            for (int k = have; k < n; k++) {
                const float lk = S.lg[S.idx[k < MAXK ? k : 0]];
                if (k == 0) first = lk;
                if (k > 0 && !(prev - lk > T)) good = false;
                prev = lk;
            }
            have = n;
        }
        if (have >= K) break;
        if (lds_get(&S.abort)) return -1;
        if (it >= lim) {
            lds_expire(S);
            return -1;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    // the selected probabilities are normal floats (CERT_SPREAD)
    if (!good || !cert_spread_ok(first, prev, cm.x)) return 0;
    if (K >= E) return 1;
    const float lo = prev - T;
    int cnt = 0;
#pragma unroll
    for (int vv = 0; vv < 4; vv++) {
        const int e = lane + WAVE * vv;
        cnt += __builtin_popcountll(__builtin_amdgcn_ballot_w64(e < E && lv[vv] >= lo));
    }
    return cnt == K ? 1 : 0;
}

// Wave W_CERT's wait for the K ranks, gathering each rank's expert and
// logit into lane k as the ranks arrive (the LDS reads overlap the passes),
// then rank K: the largest logit not selected, the lowest such index (its
// probability key is the one the passes would give it: key_of).  False if
// the workgroup aborts.
__device__ bool cert_gather(Smem &S, int E, int K, int &wk, float &lk)
{
    const int lane = opaque(lane_id());
    int have = 0;
    wk = 0;
    lk = 0.f;
    bool ok = false;
    const uint32_t lim = S.spin;
    for (uint32_t it = 0;; it++) {
        const int n = lds_get(&S.nready);
        if (n > have) {
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (lane >= have && lane < n) {
                wk = S.idx[lane < MAXK ? lane : 0];
                lk = S.lg[wk];
            }
            have = n;
        }
        if (have >= K) {
            ok = true;
            break;
        }
        if (lds_get(&S.abort)) return false;
        if (it >= lim) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if (!ok) {
        lds_expire(S);
        return false;
    }
    if (K >= E) return true;
    int ws[MAXK];
#pragma unroll
    for (int i = 0; i < MAXK; i++) ws[i] = i < K ? __builtin_amdgcn_readlane(wk, i) : -1;
    float bm = -__builtin_inff();
    int bi = E;
#pragma unroll
    for (int vv = 0; vv < 4; vv++) {
        const int e = lane + WAVE * vv;
        bool sel = e >= E;
#pragma unroll
        for (int i = 0; i < MAXK; i++) sel = sel || ws[i] == e;
        const float le = S.lg[e < E ? e : 0];
        if (!sel && (le > bm || bi == E)) {
            bm = le;
            bi = e;
        }
    }
    // NaN logits are left to the certificate's finiteness check
    const float m = wave_max(bm);
    const uint64_t at = __builtin_amdgcn_ballot_w64(bi < E && bm == m);
    const int wl = at ? (int)__builtin_ctzll(at) : 0;
    const int eK = __builtin_amdgcn_readlane(bi, wl);
    if (lane == K) {
        wk = eK < E ? eK : 0;
        lk = m;
    }
    return true;
}

// The probability key the selection passes give a logit m (rank K's, when
// the certificate moves it into the top K).
__device__ __forceinline__ uint32_t key_of(const Smem &S, float m)
{
    const float2 ms = S.smax;
    return prob_key(expf(m - ms.x) / ms.y);
}

// The reference's normalised input (cpu_rms_norm_weighted, layer_ops.cu:
// 203-212) into S.x, by wave W_CERT before a recomputation in the reference's
// order: the sequential fp32 sum of the rounded squares, inv_rms =
// 1/sqrt(sum/H + eps), x = (h inv_rms) w.  P1 left the squares in S.h[0, DH)
// and h in S.h[DH, 2 DH); nothing else writes S.h before the ranks are final.
__device__ void ref_x(Smem &S, float eps, bool has_nw, int lane)
{
#pragma clang fp contract(off)
    const float ss = seq_sum_lds(S.h, DH);
    const float inv = 1.0f / sqrtf(ss / (float)DH + eps);
#pragma unroll
    for (int i = 0; i < DH / (4 * WAVE); i++) {
        const int o = 4 * (WAVE * i + lane);
        const float4 h = *reinterpret_cast<const float4 *>(&S.h[DH + o]);
        const float4 w = has_nw ? *reinterpret_cast<const float4 *>(&S.nw[o]) : make_float4(1.f, 1.f, 1.f, 1.f);
        *reinterpret_cast<float4 *>(&S.x[o]) =
            make_float4((h.x * inv) * w.x, (h.y * inv) * w.y, (h.z * inv) * w.z, (h.w * inv) * w.w);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Run by wave W_CERT once the K + 1 selection passes are published: the
// fast logits order the top K + 1 as the reference's sums would (route_dev.h
// gives each logit a radius around the reference's sequential sum).
//   1. One radius for all: every consecutive gap of the top K + 1 exceeds
//      2 R_max + tau (tau: the softmax rounding, so that strictly separated
//      sums give strictly ordered probabilities).
//   2. Each expert's own radius: with lo_k / hi_k = logit -/+ radius of rank
//      k and M_k the largest hi of every expert ranked below k, ranks 0..k
//      are certainly above the rest when min(lo_0..lo_k) > M_k + tau' (tau
//      plus the rounding of lo and hi); certified when that holds for
//      k = 0..K-1.
//   3. If the only doubt is the order of two adjacent ranks j, j+1 (j + 1 <=
//      K, separated from everything else), both logits are computed in the
//      reference's order here (their router rows staged in S.wrow and S.nw,
//      the products formed in place, then one lane's sequential sum each):
//      equal logits tie (the lower index first, as cpu_topk's strict '>'
//      takes it), logits more than tau apart order strictly.
//   4. Otherwise exact_routing (every logit in the reference's order).
// Steps 1-3 need rank K-1's logit within CERT_SPREAD of rank 0's (radii
// included); otherwise step 4.  Returns 1 (certified), 2 (a pair
// recomputed), 3 (every logit recomputed) or 0 (a wait failed).
__device__ int certify(const DecArgs &a, const DecLayer &Ly, Smem &S, int g, int E, int K, uint32_t tag32, int l,
                       float4 cm, int wk, float lk, bool normed)
{
#pragma clang fp contract(off)
    const int lane = opaque(lane_id());  // not hoisted out of the layer loop
    const int np = K < E ? K + 1 : K;
    const float rm = cm.x, am = cm.y;
    const float tau = cert_tau(am, rm);
    // steps 3 and 4 read (and step 4 rewrites) the ranks' keys, which wave 0
    // writes after its passes
    if (!lds_wait(S, &S.wready, 1)) return 0;
    // lane k < np holds rank k's expert and logit (cert_gather; rank K is
    // the first expert not selected)
    const bool sane = cm.z != 0.f && cert_spread_ok(lane_f(lk, 0), lane_f(lk, K - 1), rm);
    const bool rk = lane < np;
    // 1: consecutive gaps against one radius (lane k: ranks k-1, k)
    const float prev = dpp_or<0x111>(__builtin_inff(), lk);
    const bool gk = lane == 0 || !rk || prev - lk > 2.f * rm + tau;
    if (sane && __builtin_amdgcn_ballot_w64(!gk) == 0) return 1;
    const float rr = rk ? S.lr[wk] : 0.f;
    int j = -1;  // >= 0: only ranks j, j+1 are in doubt (step 3)
    if (sane && np > K) {
        // 2: per-expert radii.  um: the largest hi of the experts not selected
        int ws[MAXK + 1];
#pragma unroll
        for (int i = 0; i < MAXK + 1; i++) ws[i] = i < np ? __builtin_amdgcn_readlane(wk, i) : -1;
        float um = -__builtin_inff();
#pragma unroll
        for (int vv = 0; vv < 4; vv++) {
            const int e = lane + WAVE * vv;
            bool sel = e >= E;
#pragma unroll
            for (int i = 0; i < MAXK + 1; i++) sel = sel || ws[i] == e;
            if (!sel) um = fmaxf(um, S.lg[e] + S.lr[e]);
        }
        um = wave_max(um);
        const float tau2 = tau + 4.f * CERT_U * (rm + am);
        const float inf = __builtin_inff();
        // lane k: prefix min of lo over ranks 0..k, and the largest hi below
        // rank k (ranks k+1.. of the selected, then um); ranks sit in lanes
        // 0..np-1 of row 0, so row shifts suffice
        float pm = rk ? lk - rr : inf;
        pm = fminf(pm, dpp_or<0x111>(inf, pm));
        pm = fminf(pm, dpp_or<0x112>(inf, pm));
        pm = fminf(pm, dpp_or<0x114>(inf, pm));
        pm = fminf(pm, dpp_or<0x118>(inf, pm));
        float hx = dpp_or<0x101>(-inf, rk ? lk + rr : -inf);
        hx = fmaxf(hx, dpp_or<0x101>(-inf, hx));
        hx = fmaxf(hx, dpp_or<0x102>(-inf, hx));
        hx = fmaxf(hx, dpp_or<0x104>(-inf, hx));
        hx = fmaxf(hx, dpp_or<0x108>(-inf, hx));
        const bool sepk = rk && pm > fmaxf(hx, um) + tau2;
        const uint64_t sep = __builtin_amdgcn_ballot_w64(sepk);
        const uint64_t doubt = ~sep & ((1ull << K) - 1ull);
        if (doubt == 0) return 1;
        const int jd = (int)__builtin_ctzll(doubt);
        if ((doubt & (doubt - 1)) == 0 && ((sep >> (jd + 1)) & 1ull)) j = jd;
    }
    // steps 3 and 4 sum in the reference's order, on the reference's x
    // (built before step 3 reuses S.nw)
    if (normed) ref_x(S, a.eps, Ly.norm_w != nullptr, lane);
    bool clobbered = false;
    if (j >= 0) {
        // 3: the two logits of ranks j, j+1 in the reference's order
        const int ea = __builtin_amdgcn_readlane(wk, j);
        const int eb = __builtin_amdgcn_readlane(wk, j + 1);
        clobbered = true;
#pragma unroll
        for (int i = 0; i < DH / (4 * WAVE); i++) {
            lds_load16(Ly.router + (size_t)ea * DH + 4 * (WAVE * i + lane), &S.wrow[4 * WAVE * i]);
            lds_load16(Ly.router + (size_t)eb * DH + 4 * (WAVE * i + lane), &S.nw[4 * WAVE * i]);
        }
        __builtin_amdgcn_s_waitcnt(0);
        products_in_place(S.wrow, S.x, lane);
        products_in_place(S.nw, S.x, lane);
        const float acc = seq_sum_lds(lane == 1 ? S.nw : S.wrow, DH);
        const float la = lane_f(acc, 0), lb = lane_f(acc, 1);
        trace_point_lane0(a, l, TP_XDOT);
        if (__builtin_isfinite(la) && __builtin_isfinite(lb) && (la == lb || fabsf(la - lb) > tau)) {
            const bool swap = la == lb ? eb < ea : lb > la;
            const float lK = lane_f(lk, K);
            if (swap && lane == 0) {
                const uint32_t kb = j + 1 < K ? S.key[j + 1] : key_of(S, lK);
                if (j + 1 < K) {
                    S.idx[j + 1] = ea;
                    S.key[j + 1] = S.key[j];
                }
                S.idx[j] = eb;
                S.key[j] = kb;
            }
            return 2;
        }
    }
    // 4: every logit in the reference's order
    return exact_routing(a, Ly, S, g, E, K, tag32, lane, l, clobbered) ? 3 : 0;
}

// ---------------------------------------------------------------- logit radius

// The radius of a workgroup's fp32 logit around the reference's sequential
// sum s_n (route_dev.h: |s_n - s*_n| <= u (S + c_H A) + 2n 2^-150, S the
// sum of the |exact prefixes|).  Thread t of x-polling wave w holds columns
// 256 w + 4 t .. +3, which start at the prefix W_w + o_t (wave offset +
// in-wave exclusive prefix), so S <= sum_w 256 |W_w| + sum_t (4 |o_t| + 4 A_t)
// with A_t = sum |w_k x_k| of the thread.  The logit itself carries at most
// 17 u A of rounding (4 in a thread's fma chain, 6 in the wave tree, 7 across
// the waves), which the radius absorbs: per unit of A, 4 + c_H + 17 with 2 to
// spare for the fp32 rounding of the prefixes used here, and 4 more for the
// norm's per-element rounding against the reference's x (CERT_KAPPA).  wave_terms gives
// wave w's sum of the thread terms; the workgroup's radius adds
// u (sum_w 256 |W_w| + |logit|) to their sum, times (1 + 2^-9) for the fp32
// rounding of these sums, plus 1e-37 for underflow.
__device__ __forceinline__ float wave_terms(float r, float ra)
{
    const float incl = wave_scan_incl_f32(r);
    return wave_sum(4.f * fabsf(incl - r) + (27.f + cert_c_h(DH)) * ra);
}

// ---------------------------------------------------------------- kernel

__global__ __launch_bounds__(NT, 1) void k_decode(DecArgs a)
{
    __shared__ Smem S;
    const int g = (int)blockIdx.x;
    const int tid = (int)threadIdx.x;
    const int wid = wave_id();
    const int K = a.K, E = a.E;
    const int NU = 2 * (K + 1);   // down units
    bread_decode_sync *sy = a.sync;
    const float sent = __builtin_bit_cast(float, SENTINEL);
    // No barrier here: one would wait for the prefetch (a barrier waits for
    // the wave's direct-to-LDS loads), serialising it with layer 0's input
    // load.  P1's barrier publishes these three; layer 0 neither polls nor
    // waits before it, so no wave reads or sets them earlier.
    if (tid == 0) {
        S.abort = 0;
        S.expired = 0;
        S.spin = a.spin;
    }
    prefetch(S, load_layer(a, 0), g, E, wid, 0);

    for (int l = 0; l < a.L; l++) {
        // per-lane values recomputed each layer rather than kept live
        const int tid = opaque((int)threadIdx.x);
        const int lane = tid & (WAVE - 1);
        const DecLayer Ly = load_layer(a, l);
        const uint32_t tag32 = a.epoch0 + (uint32_t)l + 1u;
        const int par = (int)((a.epoch0 + (uint32_t)l) & 1u);
        float *xout = a.xbuf + par * (G * XREC);     // this layer's output rows
        const int hp = (a.hphase0 + l) % 3;
        float *hcur = a.hbuf + hp * (G * XREC);                    // this layer's h
        float *hnext = a.hbuf + (hp == 2 ? 0 : hp + 1) * (G * XREC);  // next layer's
        trace_point(a, l, TP_START);

        // ---- P1: h of the layer (caller's buffer for the first layer, else
        // the previous layer's output, polled) by waves 0..7, thread t:
        // columns 4t .. 4t+3
        if (wid == 0) {
            // re-arm this workgroup's rows of this layer's output buffer and
            // its record of the next layer's h buffer
            if (lane < OR) cstore(xout + XREC * g + lane, sent);
            if (lane <= K) cstore2(hnext + XREC * g + GR * lane, sent, sent);
            if (tid == 0) {
                S.nready = 0;
                S.wready = 0;
                S.xqcnt = 0;
                S.gudone = 0;
                S.lgcnt = 0;
                S.rlcnt = 0;
                S.rbcnt = 0;
                S.dncnt = 0;
                S.gucnt = 0;
                S.cert = 0;
                S.ddcnt = 0;
            }
        }
        float4 hv = make_float4(0.f, 0.f, 0.f, 0.f);
        float r, ra;  // x-polling waves: the thread's router partial and its sum of |products|
        if (wid < N_XPOLL) {
            bool ok = true;
            const bool own = (tid >> 1) == g;  // threads 2g, 2g+1 hold rows 8g..8g+7
            if (l == 0) {
                const float *src = a.x0 ? a.x0 : a.hidden;
                hv = *reinterpret_cast<const float4 *>(src + 4 * tid);
                if (own && a.x0)
                    *reinterpret_cast<float4 *>(&S.hown[4 * (tid & 1)]) =
                        *reinterpret_cast<const float4 *>(a.hidden + 4 * tid);
            } else {
                const auto r = rsrc(a.xbuf + (par ^ 1) * (G * XREC), G * XREC * 4);
                ok = poll4(sy, r, 4u * (uint32_t)(XREC * (tid >> 1) + 4 * (tid & 1)), hv, S.spin);
            }
            if (own && !(l == 0 && a.x0)) *reinterpret_cast<float4 *>(&S.hown[4 * (tid & 1)]) = hv;
            if (!(l == 0 && a.x0)) {
                // h and its rounded squares for the certificate's exact
                // norm (ref_x), in S.h: free until the ranks are final
                *reinterpret_cast<float4 *>(&S.h[4 * tid]) =
                    make_float4(__fmul_rn(hv.x, hv.x), __fmul_rn(hv.y, hv.y), __fmul_rn(hv.z, hv.z), __fmul_rn(hv.w, hv.w));
                *reinterpret_cast<float4 *>(&S.h[DH + 4 * tid]) = hv;
            }
            const float ss = wave_sum(fmaf(hv.x, hv.x, fmaf(hv.y, hv.y, fmaf(hv.z, hv.z, hv.w * hv.w))));
            if (lane == 0) S.red[wid] = ss;
            if (!ok) S.abort = 1;
        } else if (wid >= W_PF) {
            // the layer's prefetched weights have landed (the barrier below
            // is a workgroup fence: it waits for them anyway)
            __builtin_amdgcn_s_waitcnt(0);
        }
        __syncthreads();
        if (S.abort) {
            if (tid == 0 && S.expired) flag_error(sy, BREAD_DEV_ERR_LOCAL);
            break;
        }
        if (wid < N_XPOLL) {
            if (!(l == 0 && a.x0)) {
                float ss = 0.f;
#pragma unroll
                for (int w = 0; w < N_XPOLL; w++) ss += S.red[w];
                const float inv = 1.0f / sqrtf(ss / (float)DH + a.eps);  // layer_ops.cu:209
                if (Ly.norm_w) {
                    const float4 nw = *reinterpret_cast<const float4 *>(&S.nw[4 * tid]);
                    hv = make_float4(hv.x * inv * nw.x, hv.y * inv * nw.y, hv.z * inv * nw.z, hv.w * inv * nw.w);
                } else {
                    hv = make_float4(hv.x * inv, hv.y * inv, hv.z * inv, hv.w * inv);
                }
            }
            *reinterpret_cast<float4 *>(&S.x[4 * tid]) = hv;
            // P2: router / shared-gate partials of the wave's 256 columns,
            // from the registers that already hold them.  Wave 0 publishes
            // the logit as soon as the partials are in, without waiting for
            // the other waves at the barrier below; its radius (from the
            // wave terms of r and ra, wave_terms) follows in P3.
            float q = 0.f;
            r = 0.f;
            ra = 0.f;
            if (g < E) {
                const float4 wr = *reinterpret_cast<const float4 *>(&S.wrow[4 * tid]);
                r = fmaf(wr.x, hv.x, fmaf(wr.y, hv.y, fmaf(wr.z, hv.z, wr.w * hv.w)));
                ra = (fabsf(wr.x * hv.x) + fabsf(wr.y * hv.y)) + (fabsf(wr.z * hv.z) + fabsf(wr.w * hv.w));
            }
            if (Ly.shg) {
                const uint2 hh = *reinterpret_cast<const uint2 *>(&S.shg[4 * tid]);
                q = fmaf(h2f(hh.x), hv.x, fmaf(h2f(hh.x >> 16), hv.y, fmaf(h2f(hh.y), hv.z, h2f(hh.y >> 16) * hv.w)));
            }
            const float rt = wave_sum(r);
            q = wave_sum(q);
            if (lane == 0) {
                S.rl[wid] = rt;
                S.gl[wid] = q;
                lds_add(&S.rlcnt, 1);
            }
            if (wid == 0 && lds_wait(S, &S.rlcnt, N_XPOLL)) {
                float logit = 0.f;
#pragma unroll
                for (int w = 0; w < N_XPOLL; w++) logit += S.rl[w];
                if (lane == 0) {
                    S.own_lg = logit;
                    if (g < E) publish(a.tlogits + LG_STRIDE * g, tag32, logit);
                }
                trace_point(a, l, TP_LOGIT);
            }
        }
        __syncthreads();
        trace_point(a, l, TP_XREADY);

        // ---- P3: logits, routing, expert streams
        if (wid < N_XPOLL) {
            // the radius terms of the router partials; waves 0..3 while
            // their first logit reads are in flight.  Wave W_RAD then
            // publishes the radius.
            const bool other = wid < NPOLL && tid < E && tid != g;
            const uint64_t w0 = other ? load_word(a.tlogits + LG_STRIDE * tid) : 0;
            const float rb = wave_terms(r, ra);
            if (lane == 0) {
                S.rbw[wid] = rb;
                lds_add(&S.rbcnt, 1);
            }
            if (wid == W_RAD && lds_wait(S, &S.rbcnt, N_XPOLL)) {
                float pre = 0.f, scross = 0.f, bsum = 0.f;
#pragma unroll
                for (int w = 0; w < N_XPOLL; w++) {
                    scross += 256.f * fabsf(pre);
                    pre += S.rl[w];
                    bsum += S.rbw[w];
                }
                const float radius = (1.0f + 1.0f / 512) * CERT_U * (scross + bsum + fabsf(S.own_lg)) + 1e-37f;
                if (lane == 0 && g < E) publish(a.tradius + LG_STRIDE * g, tag32, radius);
            }
            if (wid < NPOLL) {
                // poll one logit a lane
                float v = -__builtin_inff();
                bool ok = true;
                if (tid == g) v = S.own_lg;
                else if (other) ok = poll_word_from(sy, a.tlogits + LG_STRIDE * tid, tag32, v, w0, S.spin);
                S.lg[tid] = v;
                if (!ok) lds_put(&S.abort, 1);
                if (lane == 0) lds_add(&S.lgcnt, 1);
                if (wid == 0) {
                    // the selection passes gate every expert stream: let this wave
                    // issue ahead of the other waves on its SIMD
                    __builtin_amdgcn_s_setprio(3);
                    if (lds_wait(S, &S.lgcnt, NPOLL)) {
                        trace_point(a, l, TP_POLLED);
                        float p[4];
#pragma unroll
                        for (int vv = 0; vv < 4; vv++) p[vv] = S.lg[lane + WAVE * vv];
                        uint32_t key[4];
#pragma unroll
                        for (int vv = 0; vv < 4; vv++) key[vv] = lane + WAVE * vv < E ? logit_key(p[vv]) : 0u;
                        Sel sel = sel_init(key);
                        int wsel = 0;  // lane k: rank k's expert
#pragma unroll
                        for (int k = 0; k < MAXK; k++) {
                            if (k >= K) break;
                            uint32_t M;
                            const int win = sel_pass(sel, lane, M);
                            if (lane == 0) {
                                S.idx[k] = win < E ? win : 0;
                                lds_put(&S.nready, k + 1);
                            }
                            if (lane == k) wsel = win < E ? win : 0;
                            if (k == 0) trace_point(a, l, TP_RANK1);
                        }
                        trace_point(a, l, TP_PASSES);
                        // the softmax, off the ranks' path: the ranks'
                        // probability keys and weights (P7 redoes them if the
                        // certificate settled the ranks anew)
                        uint32_t pk[4];
                        const float2 ms = softmax_keys<4>(p, E, pk);
                        uint32_t mk = 0u;
#pragma unroll
                        for (int vv = 0; vv < 4; vv++) {
                            const uint32_t q = (uint32_t)__shfl((int)pk[vv], wsel & (WAVE - 1));
                            if ((wsel >> 6) == vv) mk = q;
                        }
                        if (lane >= K) mk = 0u;
                        const float wk = renorm_weight(mk, K);
                        float gsh = 0.f;
#pragma unroll
                        for (int w = 0; w < N_XPOLL; w++) gsh += S.gl[w];
                        if (lane < K) {
                            S.key[lane] = mk;
                            S.w[lane] = wk;
                        }
                        if (lane == 0) {
                            S.smax = ms;  // for the certificate's key of rank K
                            S.sgsh = sigmoidf_ref(gsh);
                            S.gsh = gsh;
                            lds_put(&S.wready, 1);
                        }
                        trace_point(a, l, TP_ROUTED);
                    } else if (lane == 0) {
                        lds_put(&S.abort, 1);
                    }
                    __builtin_amdgcn_s_setprio(0);
                }
            }
        }
        if (wid >= W_XQ && wid < W_XQ + N_XQ) {
            // x in fixed point for the gate/up dots, by waves that do not
            // poll the logits: it runs during the logits exchange
            quant_x(S, WAVE * (wid - W_XQ) + lane);
            if (lane == 0) lds_add(&S.xqcnt, 1);
        }
        if (wid >= W_GU && wid < W_GU + K) {
            // routed gate/up of slot k = wave, as soon as rank k is known; the
            // result is published once the ranks are final (certified, or
            // recomputed exactly, which may change this rank: then redone)
            const int slot = wid - W_GU + 1;
            if (lds_wait(S, &S.nready, slot)) {
                int e = S.idx[slot - 1];
                float hv[GR];
                bool done = false;
                for (int round = 0; round < 2 && !done; round++) {
                    gu_issue<GR>(Ly.gate_exps + (uint64_t)e * Ly.gate_eb, Ly.up_exps + (uint64_t)e * Ly.up_eb, GR * g,
                                 S.gu[slot - 1]);
                    __builtin_amdgcn_s_waitcnt(0);
                    if (round == 0 && lane == 0) lds_add(&S.gucnt, 1);
                    if (!lds_wait(S, &S.xqcnt, N_XQ)) break;
                    gu_compute<GR>(S, S.gu[slot - 1], hv);
                    if (!lds_wait(S, &S.cert, 1)) break;
                    const int ef = S.idx[slot - 1];
                    done = ef == e;
                    e = ef;
                }
                if (done && lane == 0) {
                    cstore2(hcur + XREC * g + GR * slot, hv[0], hv[1]);
                    if (slot == K) trace_here(a, l, TP_HLAST);
                    lds_add(&S.gudone, 1);
                }
            }
        }
        if (wid == W_SH || wid == W_SH + 1) {
            // shared gate/up (weights prefetched), while routing runs
            float hsh[1];
            if (lds_wait(S, &S.xqcnt, N_XQ)) {
                gu_compute<1>(S, S.shw[wid - W_SH], hsh);
                if (lane == 0) cstore(hcur + XREC * g + (wid - W_SH), hsh[0]);
            }
        }
        if (wid >= W_DN) {
            // routed down bands; chunk ch (16 B) of slot ch / 210 + 1 lands
            // at byte 16 ch of S.down
            const int nchunk = K * BAND16;
            const int c0 = WAVE * (wid - W_DN);
            const int ln = opaque(lane);
            // the down bands are not needed before the h exchange: their
            // loads go out once every rank is known, behind the gate/up
            // loads, and again if the exact recomputation replaced the ranks
            // (wave W_CERT certifies the ranks and loads none: measured, the
            // stack's layers are 0.24 us shorter than with a share of the
            // bands issued after the certificate)
            int kind = -1;  // the certificate's outcome (BREAD_RSTAT_*), wave W_CERT
            if (wid == W_CERT) {
                // as urgent as wave 0's passes (another SIMD)
                __builtin_amdgcn_s_setprio(3);
                float lv[4];
                const float4 cm = cert_prepare(a, S, E, tag32, lv);
                trace_point_lane0(a, l, TP_PREP);
                int st = cm.w != 0.f ? cert_fast(S, E, K, cm, lv) : -1;
                trace_point_lane0(a, l, TP_READY);
                kind = BREAD_RSTAT_RADIUS;
                if (st == 0) {
                    int wk;
                    float lk;
                    st = cert_gather(S, E, K, wk, lk)
                             ? certify(a, Ly, S, g, E, K, tag32, l, cm, wk, lk, !(l == 0 && a.x0))
                             : 0;
                    kind = st;  // BREAD_RSTAT_PER_EXPERT, _PAIR or _EXACT
                }
                if (st <= 0) kind = -1;
                if (lane == 0) lds_put(st > 0 ? &S.cert : &S.abort, st > 1 ? 2 : 1);  // cert 2: ranks settled anew
                __builtin_amdgcn_s_setprio(0);
                trace_point_lane0(a, l, TP_CERT);
            }
            // (sleeping between looks: the bands are needed microseconds later,
            // and a spinning wave takes issue slots from the selection passes)
            bool ok = lds_wait(S, &S.nready, K, true);
            for (int round = 0; round < 2 && ok; round++) {
#pragma unroll
                for (int i = 0; i < DN_LOADS; i++) {
                    if (wid == W_CERT) break;
                    const int cw = c0 + N_DNL * WAVE * i;  // first chunk of this wave's load
                    if (cw >= nchunk) break;
                    const int ch = cw + ln;
                    if (ch < nchunk) {
                        const int sl = ch / BAND16;  // slot - 1
                        const uint8_t *base = Ly.down_exps + (uint64_t)S.idx[sl] * Ly.down_eb;
                        lds_load16(base + (size_t)g * BAND + 16 * (ch - sl * BAND16), &S.down[4 * cw]);
                    }
                }
                __builtin_amdgcn_s_waitcnt(0);
                ok = lds_wait(S, &S.cert, 1) && lds_get(&S.cert) == 2 && round == 0;
            }
            if (lane == 0) lds_add(&S.dncnt, 1);
            // workgroup 0 counts the layer's routing outcome: after the wave's
            // last wait of the layer, so that no wait covers the atomic
            if (g == 0 && kind >= 0 && lane == 0)
                __hip_atomic_fetch_add(&sy->rstat.v[kind], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // the next layer's routing-independent weights, now that this
            // layer's are consumed (the shared gate/up was used before waves
            // 9 and 10 loaded their bands)
            if (wid >= W_PF && l + 1 < a.L && lds_wait(S, &S.dncnt, N_DN, true))
                prefetch(S, load_layer(a, l + 1), g, E, wid, (l + 1) & 1);
        }

        // ---- P4 + P5: pre-decode this wave's down unit once every band is
        // in (units 16, 17 by waves 1, 2 into LDS), and every slot's h into
        // LDS, polled: chunk c = (workgroup w, q): float4 q of w's record
        // holds slots 2q and 2q+1 (rows 2w, 2w+1).  A polling wave issues its
        // first poll before the pre-decode, so the round trip overlaps it.
        DnWeights w0;
        const bool extra = wid >= W_GU && wid < W_GU + 2 && wid - W_GU + NWV < NU;
        uint4 (*xw)[WAVE] = &S.gu[wid >= W_GU && wid < W_GU + 2 ? wid - W_GU : 0][0];
        // (after every routed gate/up is computed: the pre-decode would
        // otherwise take VALU time from the gate/up dots)
        const bool pre = wid < NU && lds_wait(S, &S.dncnt, N_DN) && lds_wait(S, &S.gudone, K);
        const bool hpoll = wid < N_HPOLL && !lds_get(&S.abort);
        const int NQ = (K + 2) >> 1;  // float4 chunks in use per record
        const auto hr = rsrc(hcur, G * XREC * 4);
        // up to two chunks a thread, polled together
        const int c0 = tid, c1 = tid + N_HPOLL * WAVE;
        const bool two = c1 < G * NQ;
        const int wa = c0 / NQ, q0 = c0 - wa * NQ, wb = c1 / NQ, q1 = c1 - wb * NQ;
        const bool hi0 = 2 * q0 + 1 <= K, hi1 = 2 * q1 + 1 <= K;
        float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
        bool r0 = !(c0 < G * NQ), r1 = !two;
        if (hpoll) {
            if (!r0)
                v0 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    hr, (int)(4 * (XREC * wa + 4 * q0)), 0, AUX_COHERENT));
            if (!r1)
                v1 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    hr, (int)(4 * (XREC * wb + 4 * q1)), 0, AUX_COHERENT));
        }
        if (pre) {
            if (tid == 0) trace_here(a, l, TP_DNIN);
            down_predecode(S, wid, l & 1, w0);
            if (extra) predecode_to_lds(S, wid - W_GU + NWV, l & 1, xw);
        }
        if (hpoll) {
            bool ok = true;
            const uint32_t lim = S.spin;
            for (uint32_t it = 0;; it++) {
                if (!r0) r0 = !unwritten(v0.x) && !unwritten(v0.y) && !(hi0 && (unwritten(v0.z) || unwritten(v0.w)));
                if (!r1) r1 = !unwritten(v1.x) && !unwritten(v1.y) && !(hi1 && (unwritten(v1.z) || unwritten(v1.w)));
                if (r0 && r1) break;
                if (it >= lim) break;
                if ((it & 63) == 63 && has_error(sy)) break;
                __builtin_amdgcn_s_sleep(1);
                if (!r0)
                    v0 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        hr, (int)(4 * (XREC * wa + 4 * q0)), 0, AUX_COHERENT));
                if (!r1)
                    v1 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        hr, (int)(4 * (XREC * wb + 4 * q1)), 0, AUX_COHERENT));
            }
            if (!(r0 && r1)) {
                if (!has_error(sy)) flag_error(sy, BREAD_DEV_ERR_HWAIT);
                ok = false;
            }
            // S.h holds the exact norm's operands until the ranks are final
            // (the shared slot's values can arrive before then); a wave
            // past the pre-decode gate has seen every routed gate/up done,
            // which follows the final ranks
            if (!pre && !lds_wait(S, &S.cert, 1)) ok = false;
            // columns 2w, 2w+1 stay adjacent in the hpos layout
            if (c0 < G * NQ) {
                const int o = hpos(GR * wa);
                *reinterpret_cast<float2 *>(&S.h[2 * q0 * DI + o]) = make_float2(v0.x, v0.y);
                if (hi0) *reinterpret_cast<float2 *>(&S.h[(2 * q0 + 1) * DI + o]) = make_float2(v0.z, v0.w);
            }
            if (two) {
                const int o = hpos(GR * wb);
                *reinterpret_cast<float2 *>(&S.h[2 * q1 * DI + o]) = make_float2(v1.x, v1.y);
                if (hi1) *reinterpret_cast<float2 *>(&S.h[(2 * q1 + 1) * DI + o]) = make_float2(v1.z, v1.w);
            }
            if (!ok) S.abort = 1;
        }
        __syncthreads();
        if (S.abort) {
            if (tid == 0 && S.expired) flag_error(sy, BREAD_DEV_ERR_LOCAL);
            break;
        }
        trace_point(a, l, TP_HREADY);

        // ---- P6: down dots
        if (wid < NU) {
            down_dot(S, wid, w0);
            if (extra) down_dot_lds(S, wid - W_GU + NWV, xw);
        }
        trace_point(a, l, TP_DDOT);
        // the launch's last layer: the other waves leave, wave 0 waits for
        // their dots on an LDS count (0.08 us shorter than the barrier; with
        // a next layer, waves that skip the barrier start polling its input
        // early and the stack's layers were 0.45 us longer)
        const bool last = l + 1 == a.L;
        if (!last) __syncthreads();
        else if (lane == 0) lds_add(&S.ddcnt, 1);

        // ---- P7: next layer's fixed weights (every buffer they land in has
        // been consumed) by waves 12..15; combine in the reference order
        // (one_layer.cu:1443-1471) and publish the rows to the next layer and
        // the caller by wave 0

        if (wid == 0) {
            // the final ranks' weights, and the routing record
            const bool anew = lds_get(&S.cert) == 2;
            float wk = lane < K ? S.w[lane] : 0.f;
            if (anew) {
                wk = renorm_weight(lane < K ? S.key[lane] : 0u, K);
                if (lane < K) S.w[lane] = wk;
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
            }
            if (g == 0) {
                const int rl = l * a.rstride;
                if (a.idx_out && lane < K) a.idx_out[rl * K + lane] = S.idx[lane];
                if (a.w_out && lane < K) a.w_out[rl * K + lane] = wk;
                if (a.gsh_out && lane == 0) a.gsh_out[rl] = S.gsh;
            }
        }
        const bool dots = wid == 0 && (!last || lds_wait(S, &S.ddcnt, NWV));
        if (wid == 0) trace_point(a, l, TP_COMB);
        if (dots && lane < OR) {
            float d[NSLOT], wt[MAXK];
#pragma unroll
            for (int k = 0; k < NSLOT; k++) d[k] = S.dot[k][lane];
#pragma unroll
            for (int k = 0; k < MAXK; k++) wt[k] = S.w[k];
            float v = S.hown[lane];
            v += S.sgsh * d[0];
#pragma unroll
            for (int k = 0; k < MAXK; k++)
                if (k < K) v += wt[k] * d[k + 1];
            if (l + 1 < a.L) cstore(xout + XREC * g + lane, v);
            a.hidden[OR * g + lane] = v;
            if (lane == 0) trace_here(a, l, TP_OUT);
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
           s.n_experts >= s.top_k && s.top_k >= 1 && s.top_k <= MAXK;
}

__global__ void k_clear_words(uint64_t *p, int n)
{
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) p[i] = 0;
}

bool layer_ok(const bread_moe_layer_t &L)
{
    if (!bread_standard_qtypes(&L)) return false;
    // buffer loads and 16-byte band loads assume these alignments
    const uintptr_t m = (uintptr_t)L.gate_exps | (uintptr_t)L.up_exps | (uintptr_t)L.down_exps |
                        (uintptr_t)L.gate_shexp | (uintptr_t)L.up_shexp | (uintptr_t)L.down_shexp |
                        (uintptr_t)L.router | (uintptr_t)L.post_norm_w;
    return (m & 15u) == 0 && (L.gate_expert_bytes & 15u) == 0 && (L.up_expert_bytes & 15u) == 0 &&
           (L.down_expert_bytes & 15u) == 0 && ((uintptr_t)L.shexp_gate & 7u) == 0;
}

int launch(bread_moe_ctx_t *c, DecArgs &a, hipStream_t st)
{
    // Every workgroup waits on every other one, so all G must be resident at
    // once.  G equals the CU count and the LDS footprint allows one workgroup
    // per CU, so an otherwise idle device runs the whole grid at once.  A
    // cooperative launch would guarantee it but costs ~20 us per launch on
    // MI355X (a normal one ~2.4 us); without it, a device shared with other
    // long-running work can delay some workgroups, and the bounded waits then
    // flag an error rather than hang.
    if (c->decode_max_blocks < G) return BREAD_ERR_SHAPE;
    a.E = c->shape.n_experts;
    a.K = c->shape.top_k;
    a.tlogits = c->tlogits;
    a.texact = c->tlogits + 256 * LG_STRIDE;
    a.tradius = c->tlogits + 2 * 256 * LG_STRIDE;
    a.xbuf = c->xbuf;
    a.hbuf = c->hbuf;
    a.sync = c->dsync;
    a.trace = (c->trace && (size_t)G * a.L * TP_N <= c->trace_words) ? c->trace : nullptr;
    a.eps = c->shape.rms_eps;
    a.spin = c->spin_limit >= 0 ? (uint32_t)c->spin_limit : SPIN_DEFAULT;
    bread_clear_stale_error();
    if (c->epoch > UINT32_MAX - 1u - (uint32_t)a.L) {
        // the layer tags would wrap past 2^32 in this launch: every tagged
        // word back to tag 0 and the count restarted, so no word written
        // before can carry a tag of a later layer (a fill kernel, not a
        // memset, so that the launch can be captured in a graph)
        const int n = (int)bread_decode_tlogit_words();
        hipLaunchKernelGGL(k_clear_words, dim3((n + 255) / 256), dim3(256), 0, st, c->tlogits, n);
        BREAD_HIP(hipGetLastError());
        c->epoch = 0;
    }
    a.epoch0 = c->epoch;
    a.hphase0 = c->hphase;
    hipLaunchKernelGGL(k_decode, dim3(G), dim3(NT), 0, st, a);
    BREAD_HIP(hipGetLastError());
    c->epoch += (uint32_t)a.L;
    c->hphase = (c->hphase + a.L) % 3;
    return BREAD_OK;
}

} // namespace

int bread_decode_max_blocks(int *out)
{
    int dev = 0, cus = 0, per_cu = 0;
    BREAD_HIP(hipGetDevice(&dev));
    BREAD_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    BREAD_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_decode, NT, 0));
    *out = cus * per_cu;
    return BREAD_OK;
}

bool bread_decode_accepts(const bread_moe_ctx_t *c, const bread_moe_layer_t *L)
{
    return c->decode_max_blocks >= G && decode_shape_ok(c->shape) && layer_ok(*L);
}

int bread_launch_moe_decode(bread_moe_ctx_t *c, const bread_moe_layer_t *L, const float *x, float *hidden,
                            hipStream_t st, int tok)
{
    if (!decode_shape_ok(c->shape) || !layer_ok(*L)) return BREAD_ERR_SHAPE;
    DecArgs a;
    memset(&a, 0, sizeof(a));
    a.layers = nullptr;
    a.one = to_dec(*L);
    a.L = 1;
    a.x0 = x;
    a.hidden = hidden;
    const int K = c->shape.top_k;
    a.idx_out = c->idx + (size_t)tok * K;
    a.w_out = c->w + (size_t)tok * K;
    a.gsh_out = c->gsh + tok;
    a.rstride = 1;
    return launch(c, a, st);
}

int bread_launch_decode_layers(bread_moe_ctx_t *c, const bread_moe_layer_t *layers, int n, float *hidden,
                               int32_t *idx, float *w, float *gsh, hipStream_t st, int rstride)
{
    if (!decode_shape_ok(c->shape)) return BREAD_ERR_SHAPE;
    BREAD_REQUIRE(n <= c->max_layers, BREAD_ERR_CAPACITY, "more layers than the context holds");
    for (int l = 0; l < n; l++)
        if (!layer_ok(layers[l])) return BREAD_ERR_SHAPE;
    DecArgs a;
    memset(&a, 0, sizeof(a));
    if (n == 1) {
        // one layer travels in the kernel arguments: no table upload
        a.layers = nullptr;
        a.one = to_dec(layers[0]);
    } else {
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
        a.layers = (const DecLayer *)c->d_layers;
    }
    a.L = n;
    a.x0 = nullptr;
    a.hidden = hidden;
    a.idx_out = idx;
    a.w_out = w;
    a.gsh_out = gsh;
    a.rstride = rstride;
    return launch(c, a, st);
}

// Exchange buffers start out "unwritten" (sentinel everywhere).
int bread_decode_reset(bread_moe_ctx_t *c)
{
    BREAD_HIP(hipMemsetD32((hipDeviceptr_t)c->xbuf, (int)SENTINEL, bread_decode_xbuf_floats()));
    BREAD_HIP(hipMemsetD32((hipDeviceptr_t)c->hbuf, (int)SENTINEL, bread_decode_hbuf_floats()));
    BREAD_HIP(hipMemset(c->tlogits, 0, bread_decode_tlogit_words() * sizeof(uint64_t)));
    BREAD_HIP(hipMemset(c->dsync, 0, sizeof(bread_decode_sync)));
    c->epoch = 0;
    c->hphase = 0;
    return BREAD_OK;
}

size_t bread_decode_xbuf_floats()
{
    return 2 * G * XREC;
}

size_t bread_decode_tlogit_words()
{
    return 3 * 256 * LG_STRIDE;  // logits, exact logits, radii
}

size_t bread_decode_hbuf_floats()
{
    return 3 * G * XREC;
}

size_t bread_decode_layer_record_bytes()
{
    return sizeof(DecLayer);
}

int bread_decode_grid(const bread_moe_shape_t &)
{
    return G;
}

int bread_decode_trace_points()
{
    return TP_N;
}
