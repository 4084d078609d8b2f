// route_cert.h — certified routing of a multi-token batch from fast router
// sums (route.hip's k_route_fast: every logit summed in parallel, with a
// rigorous radius R >= |fast - the reference's sequential sum|).
//
// cert_select_wave vouches for one token's experts from its fast logits
// alone (about 97 % of tokens at the BASELINE router scales).  For the rest,
// route_token_exact sums in the reference's order (one_layer.cu:969-971)
// only the candidate rows, those whose interval could reach the top K, and
// selects among them exactly; when even the exact sums leave two
// probabilities that could round equal, or the logits are not finite or
// spread too far, it sums every row and selects with the host's arithmetic
// (topk_wave_exact).  Indices are bit-identical to the reference's on every
// outcome; weights come from the fast logits (within the layer tolerance)
// except on the last, where they are bit-identical too.
#pragma once

#include "route_dev.h"

constexpr int RX_CH = 16;             // rows summed in the reference's order together
constexpr int RX_SEG = 2048;          // columns a pass
constexpr int RX_ROW = RX_SEG + 4;    // LDS row: lanes' 16-byte reads 4 banks apart
constexpr int RX_MAX_E = 1024;
constexpr int RX_CAND = 64;           // candidate rows a token may list (more: every row)

struct RxSmem {
    float prod[RX_CH][RX_ROW];  // products of the rows being summed (also softmax scratch)
    float ex[RX_MAX_E];         // reference-order sums, by position in cand
    int cand[RX_MAX_E];         // rows to sum, increasing
    int n;                      // their number
};

// Certified selection of one token from fast logits lg[e] with radii rd[e]
// (one wave; entry e = lane + 64 v).  The certificate: every logit and
// radius finite, |l| <= 64, the top K by fast logit (larger first, the lower
// index among equal keys) spread at most CERT_SPREAD (widened by 2 max R),
// every consecutive pair of the top K and the last of them and the largest
// l + r below it more than their radii plus tau apart (tau = 12 u (1 +
// max|l| + 2 max R)).  When it holds, the reference's selection on its own
// sums picks the same experts in the same order: lane k < K returns rank k's
// expert and its weight (expf(l_k - l_0) renormalised over the K, which is
// the reference's softmax and renormalisation, layer_ops.cu:222-249, up to
// rounding) and the result is 1.  Otherwise the candidates, every expert e
// with l_e + r_e >= l_(K) - max R - tau (the K fast-top experts have
// reference sums at least l_(K) - max R, so no other expert can reach the
// top K or tie with it), go to cand[0 .. n_cand) in increasing order and
// the result is 0; -1 (cand not written) when the logits are not finite,
// exceed |64| or more than RX_CAND experts are candidates.  scr: the wave's
// LDS scratch of 2 RX_MAX_E floats.  E >= K.
template <int MAXV>
__device__ __forceinline__ int cert_select_wave(const float *lg, const float *rd, int E, int K, int &idx_k,
                                                float &w_k, int *cand, int &n_cand, float *scr)
{
    const int lane = lane_id();
    float l[MAXV], rr[MAXV];
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int e = lane + WAVE * v, ec = e < E ? e : E - 1;
        l[v] = lg[ec];
        rr[v] = rd[ec];
    }
    bool fin = true;
    float am = 0.f, rm = 0.f;
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        fin = fin && __builtin_isfinite(l[v]) && __builtin_isfinite(rr[v]);
        am = fmaxf(am, fabsf(l[v]));
        rm = fmaxf(rm, rr[v]);
        if (lane + WAVE * v < E) {
            scr[lane + WAVE * v] = l[v];
            scr[RX_MAX_E + lane + WAVE * v] = rr[v];
        }
    }
    am = wave_max(am);
    rm = wave_max(rm);
    if (__builtin_amdgcn_ballot_w64(!fin) != 0 || !(am <= 64.f)) return -1;
    const float tau = 12.f * CERT_U * (1.f + am + 2.f * rm);
    // selection: lane k < K records rank k's expert; the passes do nothing
    // else, so each waits only on the previous one's maximum
    int my_idx = 0;
    uint32_t taken = 0u;  // bit v: entry lane + 64 v selected
    if constexpr (MAXV == 4) {
        // Each lane sorts its four entries once (key << 2 | 3 - v, larger
        // first: equal keys put the lower index first); a pass then takes
        // the largest head in the wave (the lowest lane among equals, also
        // the lower index) and that lane moves to its next entry.  Any order
        // among equal keys would do here: such experts are within 4 ulps,
        // and the certificate then fails.
        uint32_t h[4];
#pragma unroll
        for (int v = 0; v < 4; v++) h[v] = lane + WAVE * v < E ? (logit_key(l[v]) << 2) | (uint32_t)(3 - v) : 0u;
#define RC_CX(a, b)                                   \
    {                                                 \
        const uint32_t hi_ = umax32(h[a], h[b]);      \
        h[b] = h[a] < h[b] ? h[a] : h[b];             \
        h[a] = hi_;                                   \
    }
        RC_CX(0, 1) RC_CX(2, 3) RC_CX(0, 2) RC_CX(1, 3) RC_CX(1, 2)
#undef RC_CX
        for (int k = 0; k < K; k++) {
            const uint32_t M = wave_max_u32(h[0]);
            const int wlane = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(h[0] == M));
            const int v = 3 - (int)(M & 3u);
            if (lane == wlane) {
                h[0] = h[1];
                h[1] = h[2];
                h[2] = h[3];
                h[3] = 0u;
                taken |= 1u << v;
            }
            if (lane == k) my_idx = wlane + WAVE * v;
        }
    } else {
        uint32_t key[MAXV];
#pragma unroll
        for (int v = 0; v < MAXV; v++) key[v] = lane + WAVE * v < E ? logit_key(l[v]) : 0u;
        for (int k = 0; k < K; k++) {
            uint32_t M;
            const int win = select_round<MAXV>(key, M);  // wave-uniform; its key is now 0
            if (lane == win % WAVE) taken |= 1u << (win / WAVE);
            if (lane == k) my_idx = win;
        }
    }
    // the selected logits and radii (this wave's own LDS writes, in order),
    // each rank against the next (DPP row_shl 1: K <= 16 lies in row 0)
    __builtin_amdgcn_wave_barrier();
    const float my_l = lane < K ? scr[my_idx] : 0.f, my_r = lane < K ? scr[RX_MAX_E + my_idx] : 0.f;
    const float nx_l = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, my_l), 0x101,
                                                                             0xF, 0xF, true));
    const float nx_r = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, my_r), 0x101,
                                                                             0xF, 0xF, true));
    const bool gap_ok = lane >= K - 1 || my_l - nx_l > my_r + nx_r + tau;
    const float top = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_l), 0));
    const float prev_l = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_l), K - 1));
    const float prev_r = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_r), K - 1));
    // the largest l + r among the experts not selected
    float rest = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < MAXV; v++)
        if (lane + WAVE * v < E && !((taken >> v) & 1u)) rest = fmaxf(rest, l[v] + rr[v]);
    rest = wave_max(rest);
    const bool ok = __builtin_amdgcn_ballot_w64(!gap_ok) == 0 && top - prev_l + 2.f * rm <= CERT_SPREAD &&
                    prev_l - rest > prev_r + tau;
    if (ok) {
        const float e = lane < K ? __expf(my_l - top) : 0.f;
        float s = 0.f;
        for (int k = 0; k < K; k++)
            s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), k));
        idx_k = my_idx;
        w_k = e / s;
        return 1;
    }
    const float thr = prev_l - rm - tau;
    int n = 0;
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int e = lane + WAVE * v;
        const bool c = e < E && l[v] + rr[v] >= thr;
        const uint64_t b = __builtin_amdgcn_ballot_w64(c);
        const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        if (c && n + below < RX_CAND) cand[n + below] = e;
        n += __builtin_popcountll(b);
    }
    n_cand = n;
    return n <= RX_CAND ? 0 : -1;
}

// The reference's sequential fp32 sum ((acc + p_0) + p_1) + ... of n values
// in LDS (n % 32 == 0; each lane may read its own array), with three blocks
// of 8 in flight ahead of the dependent adds (seq_sum_lds keeps one or two:
// here the adds run alone on the SIMD and would wait on LDS latency).
__device__ __forceinline__ void rx_add8(float &acc, const float (&v)[8])
{
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 8; j++) {
        acc = acc + v[j];
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ __forceinline__ float seq_sum_lds_deep(const float *p, int n, float acc)
{
    const int nb = n / 8;
    float v0[8], v1[8], v2[8], v3[8];
    lds_read8(p, 0, v0);
    lds_read8(p, 8, v1);
    lds_read8(p, 16, v2);
    for (int b = 0; b < nb; b += 4) {
        lds_read8(p, 8 * min(b + 3, nb - 1), v3);
        __builtin_amdgcn_sched_barrier(0);
        rx_add8(acc, v0);
        lds_read8(p, 8 * min(b + 4, nb - 1), v0);
        __builtin_amdgcn_sched_barrier(0);
        rx_add8(acc, v1);
        lds_read8(p, 8 * min(b + 5, nb - 1), v1);
        __builtin_amdgcn_sched_barrier(0);
        rx_add8(acc, v2);
        lds_read8(p, 8 * min(b + 6, nb - 1), v2);
        __builtin_amdgcn_sched_barrier(0);
        rx_add8(acc, v3);
    }
    return acc;
}

// The reference-order sums s = ((0 + q_0) + q_1) + ... + q_{H-1}, q_k =
// fl(W[r][k] x[k]) (one_layer.cu:969-971), of the rows r = S.cand[0 .. n)
// into S.ex[0 .. n), by a workgroup of NT threads (every thread calls it):
// the products of 16 rows are staged in LDS, RX_SEG columns at a time, then
// lanes 0..15 of wave 0 each add one row's in order.  H % 1024 == 0.
template <int NT>
__device__ void rows_exact_wg(RxSmem &S, const float *__restrict__ W, const float *__restrict__ x, int H, int n)
{
    constexpr int PER = RX_CH * RX_SEG / 4 / NT;  // float4 products a thread stages per pass
    static_assert(PER * NT * 4 == RX_CH * RX_SEG, "threads");
    const int tid = (int)threadIdx.x;
    for (int b0 = 0; b0 < n; b0 += RX_CH) {
        const int nb = n - b0 < RX_CH ? n - b0 : RX_CH;
        float s = 0.f;  // lane c < nb of wave 0: row S.cand[b0 + c]
        for (int k0 = 0; k0 < H; k0 += RX_SEG) {
            const int seg = H - k0 < RX_SEG ? H - k0 : RX_SEG;
            const int g4 = seg / 4;
            // float4 group g = tid + NT m: row g / g4 of the batch, columns
            // k0 + 4 (g % g4); rows past the batch read its last row again
            float4 q[PER];
#pragma unroll
            for (int m = 0; m < PER; m++) {
                const int g = tid + NT * m, r = g / g4, j = g - r * g4;
                const int rc = r < nb ? r : nb - 1;
                const float4 w4 = *reinterpret_cast<const float4 *>(W + (size_t)S.cand[b0 + rc] * H + k0 + 4 * j);
                const float4 x4 = *reinterpret_cast<const float4 *>(x + k0 + 4 * j);
                q[m] = make_float4(w4.x * x4.x, w4.y * x4.y, w4.z * x4.z, w4.w * x4.w);
            }
#pragma unroll
            for (int m = 0; m < PER; m++) {
                const int g = tid + NT * m, r = g / g4, j = g - r * g4;
                if (r < nb) *reinterpret_cast<float4 *>(&S.prod[r][4 * j]) = q[m];
            }
            __syncthreads();
            if (tid < nb) s = seq_sum_lds_deep(&S.prod[tid][0], seg, s);
            __syncthreads();
        }
        if (tid < nb) S.ex[b0 + tid] = s;
    }
    __syncthreads();
}

// Exact selection among the candidates S.cand[0 .. n) by their
// reference-order sums S.ex (one wave; candidates lane + 64 v).  Every
// expert outside the candidates lies more than tau below the K-th, so the
// reference's top K are candidates; among them its probabilities
// fl(expf(l - max) / s) order as e = expf(l - max) does (the host's expf,
// libm_expf_t with the table copy tab) when two e are equal (then the lower
// index first, as select_round takes it) or at least 4 representable values
// apart (then the quotients by the same s round apart).  Returns false when
// a consecutive pair of the top K, or the K-th and the best other
// candidate, is closer than that, or the K-th lies more than CERT_SPREAD
// below the top; true with lane k < K holding rank k's expert and weight
// (e renormalised over the K) otherwise.
template <int MAXV>
__device__ bool exact_select_candidates(const RxSmem &S, int n, int K, const uint64_t *tab, int &idx_k,
                                        float &w_k)
{
    const int lane = lane_id();
    float ex[MAXV];
    float mx = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        const int i = lane + WAVE * v;
        ex[v] = i < n ? S.ex[i] : -__builtin_inff();
        mx = fmaxf(mx, ex[v]);
    }
    mx = wave_max(mx);
    uint32_t key[MAXV];
    float ev[MAXV];
#pragma unroll
    for (int v = 0; v < MAXV; v++) {
        ev[v] = lane + WAVE * v < n ? libm_expf_t(ex[v] - mx, tab) : 0.f;
        key[v] = lane + WAVE * v < n ? prob_key(ev[v]) : 0u;
    }
    bool ok = true;
    uint32_t prev = 0u;
    float lk = mx, my_e = 0.f;
    int my_idx = 0;
    for (int k = 0; k < K; k++) {
        uint32_t M;
        const int win = select_round<MAXV>(key, M);
        if (k > 0) ok = ok && (M == prev || prev - M >= 4u);
        prev = M;
        float we = ev[0], wl = ex[0];
#pragma unroll
        for (int v = 1; v < MAXV; v++)
            if (win / WAVE == v) {
                we = ev[v];
                wl = ex[v];
            }
        we = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, we), win % WAVE));
        lk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), win % WAVE));
        if (lane == k) {
            my_idx = S.cand[win];
            my_e = we;
        }
    }
    // the best candidate left (0 when there is none)
    uint32_t lm = 0u;
#pragma unroll
    for (int v = 0; v < MAXV; v++) lm = umax32(lm, key[v]);
    const uint32_t rest = wave_max_u32(lm);
    ok = ok && (rest == 0u || rest == prev || prev - rest >= 4u) && mx - lk <= CERT_SPREAD;
    if (!ok) return false;
    float s = 0.f;
    for (int k = 0; k < K; k++)
        s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_e), k));
    idx_k = my_idx;
    w_k = my_e / s;
    return true;
}

// Routes one token after its certificate failed, by a workgroup of NT
// threads (every thread calls it; lane k < K of wave 0 returns rank k's
// expert and weight): the reference-order sums of the candidate rows
// cand[0 .. n_cand) (n_cand < 0: every row) of W with the token's x, then
// the exact selection among them.  Returns 1 when that decided the ranks;
// otherwise, or with n_cand < 0, every row is summed and the host's
// arithmetic selects (topk_wave_exact: weights bit-identical too) and it
// returns 2.  tab: libm_expf_tab's entries (LDS).
template <int MAXV, int NT>
__device__ int route_token_exact(RxSmem &S, const float *__restrict__ W, const float *__restrict__ x,
                                 const int *cand, int n_cand, int H, int E, int K, const uint64_t *tab, int &idx_k,
                                 float &w_k)
{
    const int tid = (int)threadIdx.x, lane = lane_id();
    if (n_cand >= 0) {
        for (int i = tid; i < n_cand; i += NT) S.cand[i] = cand[i];
        __syncthreads();
        rows_exact_wg<NT>(S, W, x, H, n_cand);
        if (tid < WAVE) {
            const bool ok = exact_select_candidates<MAXV>(S, n_cand, K, tab, idx_k, w_k);
            if (lane == 0) S.n = ok ? 1 : 0;
        }
        __syncthreads();
        const bool decided = S.n != 0;
        __syncthreads();  // every thread has read S.n before anything writes S again
        if (decided) return 1;
    }
    for (int e = tid; e < E; e += NT) S.cand[e] = e;
    __syncthreads();
    rows_exact_wg<NT>(S, W, x, H, E);
    if (tid < WAVE) topk_wave_exact<MAXV>(S.ex, E, K, &S.prod[0][0], idx_k, w_k);
    __syncthreads();
    return 2;
}
