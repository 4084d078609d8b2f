// bread_device.h — device helpers shared by the gfx950 kernels of the MoE
// feed-forward path: fp16 decode, K-quant field unpacking, alignment-tolerant
// loads and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define QK 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210
#define Q80_BYTES 34
#define Q80_ELEMS 32
#define WAVE 64

// ---------------------------------------------------------------------------
// fp16 decode
// ---------------------------------------------------------------------------

// Bitwise restatement of bread_h2f (bread_utils.h:27-47): subnormals become
// mantissa * 2^-24, Inf/NaN keep their payload bits.  Used where results must
// match the reference bit for bit (the dequant export).
__device__ __forceinline__ float h2f_exact(uint32_t h)
{
    h &= 0xFFFFu;
    const uint32_t sign = (h >> 15) << 31;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    const uint32_t mantissa = h & 0x3FFu;
    if (exponent == 0) {
        const float val = (float)mantissa * (1.0f / 16777216.0f);
        return (h >> 15) ? -val : val;
    }
    const uint32_t bits = exponent == 31 ? (sign | 0x7F800000u | (mantissa << 13))
                                         : (sign | ((exponent + 112u) << 23) | (mantissa << 13));
    return __builtin_bit_cast(float, bits);
}

// Hardware conversion (v_cvt_f32_f16): identical to h2f_exact for every
// finite value including subnormals; only quiets signalling NaNs.  Used in
// the matvec paths, whose contract is a tolerance.
__device__ __forceinline__ float h2f(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

__device__ __forceinline__ uint16_t f2h(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---------------------------------------------------------------------------
// K-quant fields
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t byte_of(uint32_t w, uint32_t k)
{
    return (w >> (8u * k)) & 0xFFu;
}

// Byte k (0..11) of the Q4_K packed scales held as three dwords.
__device__ __forceinline__ uint32_t scale_byte(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t k)
{
    const uint32_t w = k < 4 ? s0 : (k < 8 ? s1 : s2);
    return byte_of(w, k & 3u);
}

// 6-bit (scale, min) pair j (0..7) of a Q4_K superblock, the unpacking of
// get_scale_min_k4 (dequant_q4k_cpu.c:70-79).
__device__ __forceinline__ void scale_min_k4(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t &sc, uint32_t &m)
{
    if (j < 4) {
        sc = scale_byte(s0, s1, s2, j) & 63u;
        m = scale_byte(s0, s1, s2, j + 4) & 63u;
    } else {
        sc = (scale_byte(s0, s1, s2, j + 4) & 0x0Fu) | ((scale_byte(s0, s1, s2, j - 4) >> 6) << 4);
        m = (scale_byte(s0, s1, s2, j + 4) >> 4) | ((scale_byte(s0, s1, s2, j) >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------
// Loads
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint4 ld_b128(const uint8_t *p)
{
    return *reinterpret_cast<const uint4 *>(p);
}

__device__ __forceinline__ uint32_t ld_b32(const uint8_t *p)
{
    return *reinterpret_cast<const uint32_t *>(p);
}

// 8 bytes starting at a 2-byte aligned address, from aligned dword loads.
// Every dword loaded holds at least one wanted byte (for p = 4m the third
// load repeats the second), so nothing outside the object's aligned dwords
// is read.  Q6_K and Q8_0 blocks (210 and 34 bytes) are only 2-byte aligned.
__device__ __forceinline__ uint2 ld8_a2(const uint8_t *p)
{
    // aligned down by pointer arithmetic, which keeps the global address
    // space (a pointer rebuilt from an integer gets flat loads)
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint8_t *b = p - sh;
    const uint32_t w0 = ld_b32(b);
    const uint32_t w1 = ld_b32(b + 4);
    const uint32_t w2 = ld_b32(b + (sh ? 8 : 4));
    uint2 r;
    r.x = __builtin_amdgcn_alignbyte(w1, w0, sh);
    r.y = __builtin_amdgcn_alignbyte(w2, w1, sh);
    return r;
}

// 16-bit value at a 2-byte aligned address.
__device__ __forceinline__ uint32_t ld16_a2(const uint8_t *p)
{
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t w = ld_b32(p - sh);
    return (w >> (8u * sh)) & 0xFFFFu;
}

// 8 bytes at a 2-byte aligned byte offset of a dword array (LDS), from
// aligned dwords.
__device__ __forceinline__ uint2 lds8_a2(const uint32_t *base, uint32_t off)
{
    const uint32_t a = off >> 2, sh = off & 3u;
    const uint32_t w0 = base[a], w1 = base[a + 1], w2 = base[(off + 7) >> 2];
    uint2 o;
    o.x = __builtin_amdgcn_alignbyte(w1, w0, sh);
    o.y = __builtin_amdgcn_alignbyte(w2, w1, sh);
    return o;
}

// 16-bit value at a 2-byte aligned byte offset of a dword array (LDS).
__device__ __forceinline__ uint32_t lds16_a2(const uint32_t *base, uint32_t off)
{
    return (base[off >> 2] >> (8u * (off & 3u))) & 0xFFFFu;
}

// ---------------------------------------------------------------------------
// wave64 reductions (DPP inside 16-lane rows, cross-row by permute)
// ---------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, true));
}

// Inclusive prefix sum over the wave in lane order, all on DPP: row_shr 1,
// 2, 4, 8 inside the 16-lane rows (lanes without a source add 0), then each
// row's total into the rows after it (row_bcast 15 into rows 1 and 3,
// row_bcast 31 into rows 2 and 3).
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, true);
}

__device__ __forceinline__ int wave_scan_incl(int v)
{
    v += dpp_i<0x111, 0xF>(v);
    v += dpp_i<0x112, 0xF>(v);
    v += dpp_i<0x114, 0xF>(v);
    v += dpp_i<0x118, 0xF>(v);
    v += dpp_i<0x142, 0xA>(v);
    v += dpp_i<0x143, 0xC>(v);
    return v;
}

// Sum over aligned groups of 8 lanes; the result is in every lane of the group.
__device__ __forceinline__ float sum8(float v)
{
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    return v;
}

__device__ __forceinline__ float sum16(float v)
{
    v = sum8(v);
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
}

// Cross-row exchange of gfx950's v_permlane16_swap / v_permlane32_swap with
// both operands the same register: .a holds, in every lane, the value of the
// lane 16 (or 32) below it in its 32 (64) lane group, .b the one above, so
// combining .a and .b merges two rows (halves) in every lane without LDS.
struct lane_pair {
    uint32_t a, b;
};

__device__ __forceinline__ lane_pair swap16(uint32_t v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return {r[0], r[1]};
}

__device__ __forceinline__ lane_pair swap32(uint32_t v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return {r[0], r[1]};
}

__device__ __forceinline__ float sum32(float v)
{
    v = sum16(v);
    const lane_pair p = swap16(__builtin_bit_cast(uint32_t, v));
    return __builtin_bit_cast(float, p.a) + __builtin_bit_cast(float, p.b);
}

// Sum over the wave; the result is in every lane.
__device__ __forceinline__ float wave_sum(float v)
{
    v = sum32(v);
    const lane_pair p = swap32(__builtin_bit_cast(uint32_t, v));
    return __builtin_bit_cast(float, p.a) + __builtin_bit_cast(float, p.b);
}

// Max over the wave (NaN-ignoring fmaxf); the result is in every lane.
__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    lane_pair p = swap16(__builtin_bit_cast(uint32_t, v));
    v = fmaxf(__builtin_bit_cast(float, p.a), __builtin_bit_cast(float, p.b));
    p = swap32(__builtin_bit_cast(uint32_t, v));
    return fmaxf(__builtin_bit_cast(float, p.a), __builtin_bit_cast(float, p.b));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, true);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t u64_max(uint64_t a, uint64_t b)
{
    return b > a ? b : a;
}

// Unsigned 64-bit max over the wave; the result is in every lane.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v)
{
    v = u64_max(v, dpp_u64<0xB1>(v));
    v = u64_max(v, dpp_u64<0x4E>(v));
    v = u64_max(v, dpp_u64<0x141>(v));
    v = u64_max(v, dpp_u64<0x140>(v));
    lane_pair lo = swap16((uint32_t)v), hi = swap16((uint32_t)(v >> 32));
    v = u64_max(((uint64_t)hi.a << 32) | lo.a, ((uint64_t)hi.b << 32) | lo.b);
    lo = swap32((uint32_t)v);
    hi = swap32((uint32_t)(v >> 32));
    return u64_max(((uint64_t)hi.a << 32) | lo.a, ((uint64_t)hi.b << 32) | lo.b);
}

__device__ __forceinline__ int lane_id()
{
    return (int)(threadIdx.x & (WAVE - 1));
}

// Wave index inside the workgroup, marked wave-uniform (scalar register), so
// addresses and buffer descriptors built from it stay scalar.
__device__ __forceinline__ int wave_id()
{
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE));
}

__device__ __forceinline__ int uniform(int v)
{
    return __builtin_amdgcn_readfirstlane(v);
}

__device__ __forceinline__ uint64_t uniform64(uint64_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p)
{
    return reinterpret_cast<T *>(uniform64(reinterpret_cast<uint64_t>(p)));
}

constexpr uint32_t BUF_WORD3 = 0x00020000u;  // raw buffer descriptor word 3 (gfx9)

// Raw buffer descriptor over [base, base + bytes): loads beyond the range
// return zeros.  The base is made wave-uniform explicitly: a descriptor the
// compiler keeps in vector registers costs a waterfall loop around every load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(const_cast<void *>(base)), (short)0,
                                             uniform((int)bytes), (int)BUF_WORD3);
}
