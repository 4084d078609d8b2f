// synth.hip — HBM-resident expert arena and the seeded synthetic weight
// generator (bench and test inputs).
//
// Generator: word(seed, i) = fmix64(seed * 0x632BE59BD9B4E019 + (i + 1) *
// 0x9E3779B97F4A7C15) (the SplitMix64 output function over a counter), so
// every byte depends only on (seed, byte position).  breadv2_amd/synth.py is
// the host twin of the quantized generators, bit for bit.
#include <stdlib.h>
#include <string.h>

#include "bread_internal.h"
#include "bread_device.h"

namespace {

__host__ __device__ __forceinline__ uint64_t fmix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t rng_word(uint64_t seed, uint64_t i)
{
    return fmix64(seed * 0x632BE59BD9B4E019ull + (i + 1) * 0x9E3779B97F4A7C15ull);
}

// fp16 bits of U(1e-3, 1e-2) from a 16-bit uniform; fp32 multiply then add
// (no contraction), round to nearest even.
__device__ __forceinline__ uint32_t scale_f16(uint32_t u16)
{
#pragma clang fp contract(off)
    const float u = (float)u16 * (1.0f / 65536.0f);
    const float v = 1e-3f + 9e-3f * u;
    return f2h(v);
}

__device__ __forceinline__ uint32_t q4k_byte(uint64_t seed, uint64_t sb, uint32_t off)
{
    const uint64_t w = rng_word(seed, sb * 18 + off / 8);
    if (off < 4) {
        const uint32_t lo = (uint32_t)w;
        const uint32_t hdr = scale_f16(lo & 0xFFFFu) | (scale_f16(lo >> 16) << 16);
        return (hdr >> (8 * off)) & 0xFFu;
    }
    return (uint32_t)(w >> (8 * (off % 8))) & 0xFFu;
}

__device__ __forceinline__ uint32_t q6k_byte(uint64_t seed, uint64_t sb, uint32_t off)
{
    const uint64_t w = rng_word(seed, sb * 27 + off / 8);
    if (off >= 208) {
        const uint32_t d = scale_f16((uint32_t)w & 0xFFFFu);
        return (d >> (8 * (off - 208))) & 0xFFu;
    }
    const uint32_t raw = (uint32_t)(w >> (8 * (off % 8))) & 0xFFu;
    if (off >= 192) return (uint32_t)(uint8_t)(int8_t)((int)(raw & 63u) - 32);
    return raw;
}

template <int QT>
__global__ __launch_bounds__(256) void k_synth_quant(uint8_t *__restrict__ dst, uint64_t n_bytes, uint64_t seed)
{
    const uint32_t BB = QT == BREAD_QTYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    const uint64_t n_dw = (n_bytes + 3) / 4;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n_dw;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t b0 = i * 4;
        uint32_t v = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint64_t b = b0 + k;
            if (b < n_bytes) {
                const uint64_t sb = b / BB;
                const uint32_t off = (uint32_t)(b % BB);
                const uint32_t byte = QT == BREAD_QTYPE_Q4_K ? q4k_byte(seed, sb, off) : q6k_byte(seed, sb, off);
                v |= byte << (8 * k);
            }
        }
        if (b0 + 4 <= n_bytes) {
            *reinterpret_cast<uint32_t *>(dst + b0) = v;
        } else {
            for (int k = 0; b0 + k < n_bytes; k++) dst[b0 + k] = (uint8_t)(v >> (8 * k));
        }
    }
}

__device__ __forceinline__ void normal_pair(uint64_t seed, uint64_t i, float &z0, float &z1)
{
    const uint64_t w = rng_word(seed, i);
    const float u1 = (float)((w >> 40) + 1) * (1.0f / 16777216.0f);          // (0, 1]
    const float u2 = (float)((w >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);  // [0, 1)
    const float r = sqrtf(-2.0f * logf(u1));
    float s, c;
    sincosf(6.283185307179586f * u2, &s, &c);
    z0 = r * c;
    z1 = r * s;
}

template <typename T>
__global__ __launch_bounds__(256) void k_synth_normal(T *__restrict__ dst, uint64_t n, uint64_t seed, float mean,
                                                      float std)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; 2 * i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float z0, z1;
        normal_pair(seed, i, z0, z1);
        const float v0 = mean + std * z0, v1 = mean + std * z1;
        if constexpr (sizeof(T) == 4) {
            dst[2 * i] = v0;
            if (2 * i + 1 < n) dst[2 * i + 1] = v1;
        } else {
            dst[2 * i] = f2h(v0);
            if (2 * i + 1 < n) dst[2 * i + 1] = f2h(v1);
        }
    }
}

dim3 grid_for(uint64_t items)
{
    const uint64_t g = (items + 255) / 256;
    return dim3((unsigned)(g < 262144 ? (g ? g : 1) : 262144));
}

uint64_t align256(uint64_t v)
{
    return (v + 255) & ~(uint64_t)255;
}

} // namespace

extern "C" int bread_synth_q4k(void *dst, uint64_t n_blocks, uint64_t seed, bread_stream_t stream)
{
    BREAD_REQUIRE(dst, BREAD_ERR_ARG, "NULL destination");
    BREAD_REQUIRE(((uintptr_t)dst & 3) == 0, BREAD_ERR_ALIGN, "destination must be 4-byte aligned");
    if (!n_blocks) return BREAD_OK;
    const uint64_t nb = n_blocks * Q4K_BYTES;
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_synth_quant<BREAD_QTYPE_Q4_K>, grid_for((nb + 3) / 4), dim3(256), 0, to_hip(stream),
                       (uint8_t *)dst, nb, seed);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

extern "C" int bread_synth_q6k(void *dst, uint64_t n_blocks, uint64_t seed, bread_stream_t stream)
{
    BREAD_REQUIRE(dst, BREAD_ERR_ARG, "NULL destination");
    BREAD_REQUIRE(((uintptr_t)dst & 3) == 0, BREAD_ERR_ALIGN, "destination must be 4-byte aligned");
    if (!n_blocks) return BREAD_OK;
    const uint64_t nb = n_blocks * Q6K_BYTES;
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_synth_quant<BREAD_QTYPE_Q6_K>, grid_for((nb + 3) / 4), dim3(256), 0, to_hip(stream),
                       (uint8_t *)dst, nb, seed);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

extern "C" int bread_synth_normal_f32(float *dst, uint64_t n, uint64_t seed, float mean, float std,
                                      bread_stream_t stream)
{
    BREAD_REQUIRE(dst, BREAD_ERR_ARG, "NULL destination");
    if (!n) return BREAD_OK;
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_synth_normal<float>, grid_for((n + 1) / 2), dim3(256), 0, to_hip(stream), dst, n, seed,
                       mean, std);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

extern "C" int bread_synth_normal_f16(uint16_t *dst, uint64_t n, uint64_t seed, float mean, float std,
                                      bread_stream_t stream)
{
    BREAD_REQUIRE(dst, BREAD_ERR_ARG, "NULL destination");
    if (!n) return BREAD_OK;
    bread_clear_stale_error();
    hipLaunchKernelGGL(k_synth_normal<uint16_t>, grid_for((n + 1) / 2), dim3(256), 0, to_hip(stream), dst, n,
                       seed, mean, std);
    BREAD_HIP(hipGetLastError());
    return BREAD_OK;
}

// ---------------------------------------------------------------------------
// Arena
// ---------------------------------------------------------------------------

bread_arena_layout bread_arena_plan(const bread_moe_shape_t &s, const int types[6])
{
    bread_arena_layout p{};
    for (int i = 0; i < 6; i++) p.types[i] = types[i];
    const uint64_t H = s.hidden, I = s.expert_inter, Ish = s.shared_inter, E = s.n_experts;
    p.gate_expert_bytes = I * bread_expert_row_bytes(types[0], (int)H);
    p.up_expert_bytes = I * bread_expert_row_bytes(types[1], (int)H);
    p.down_expert_bytes = H * bread_expert_row_bytes(types[2], (int)I);
    uint64_t o = 0;
    p.off_gate = o; o = align256(o + E * p.gate_expert_bytes);
    p.off_up = o; o = align256(o + E * p.up_expert_bytes);
    p.off_down = o; o = align256(o + E * p.down_expert_bytes);
    p.off_gate_sh = o; o = align256(o + Ish * bread_expert_row_bytes(types[3], (int)H));
    p.off_up_sh = o; o = align256(o + Ish * bread_expert_row_bytes(types[4], (int)H));
    p.off_down_sh = o; o = align256(o + H * bread_expert_row_bytes(types[5], (int)Ish));
    p.off_router = o; o = align256(o + E * H * 4);
    p.off_shgate = o; o = align256(o + H * 2);
    p.off_norm = o; o = align256(o + H * 4);
    p.layer_bytes = o;
    return p;
}

namespace {
// the reference GPU path's mix (one_layer.cu:1966-1977)
constexpr int STANDARD_TYPES[6] = {BREAD_QTYPE_Q4_K, BREAD_QTYPE_Q4_K, BREAD_QTYPE_Q6_K,
                                   BREAD_QTYPE_Q4_K, BREAD_QTYPE_Q4_K, BREAD_QTYPE_Q6_K};
}  // namespace

extern "C" int bread_arena_create(const bread_moe_shape_t *s, int n_layers, bread_arena_t **out)
{
    BREAD_REQUIRE(s && out && n_layers > 0, BREAD_ERR_ARG, "NULL shape/out or n_layers <= 0");
    BREAD_REQUIRE(s->hidden > 0 && s->hidden % QK == 0 && s->expert_inter > 0 && s->expert_inter % QK == 0 &&
                      s->shared_inter > 0 && s->shared_inter % QK == 0 && s->n_experts > 0,
                  BREAD_ERR_SHAPE, "hidden and intermediate sizes must be positive multiples of 256");
    *out = nullptr;
    bread_arena_t *a = (bread_arena_t *)calloc(1, sizeof(bread_arena_t));
    BREAD_REQUIRE(a, BREAD_ERR_NOMEM, "host allocation");
    a->shape = *s;
    a->n_layers = n_layers;
    a->lay = (bread_arena_layout *)calloc((size_t)n_layers, sizeof(bread_arena_layout));
    a->layers = (uint8_t **)calloc((size_t)n_layers, sizeof(uint8_t *));
    a->flags = (int *)calloc((size_t)n_layers, sizeof(int));
    hipError_t e = hipGetDevice(&a->device);
    if (!a->lay || !a->layers || !a->flags) e = hipErrorOutOfMemory;
    const bread_arena_layout std_lay = bread_arena_plan(*s, STANDARD_TYPES);
    for (int l = 0; l < n_layers && e == hipSuccess; l++) {
        a->lay[l] = std_lay;
        a->flags[l] = BREAD_ARENA_HAS_SHGATE;
        e = hipMalloc((void **)&a->layers[l], std_lay.layer_bytes);
    }
    if (e != hipSuccess) {
        bread_arena_destroy(a);
        return bread_fail(e == hipErrorOutOfMemory ? BREAD_ERR_NOMEM : BREAD_ERR_HIP, "bread_arena_create",
                          hipGetErrorString(e));
    }
    *out = a;
    return BREAD_OK;
}

extern "C" int bread_arena_destroy(bread_arena_t *a)
{
    if (!a) return BREAD_OK;
    if (a->layers)
        for (int l = 0; l < a->n_layers; l++) (void)hipFree(a->layers[l]);
    free(a->layers);
    free(a->flags);
    free(a->lay);
    free(a);
    return BREAD_OK;
}

int bread_arena_relayout(bread_arena_t *a, int l, const int types[6])
{
    bool same = true;
    for (int i = 0; i < 6; i++) same = same && a->lay[l].types[i] == types[i];
    if (same) return BREAD_OK;
    const bread_arena_layout p = bread_arena_plan(a->shape, types);
    if (p.layer_bytes != a->lay[l].layer_bytes) {
        uint8_t *nb = nullptr;
        const hipError_t e = hipMalloc((void **)&nb, p.layer_bytes);
        if (e != hipSuccess)
            return bread_fail(e == hipErrorOutOfMemory ? BREAD_ERR_NOMEM : BREAD_ERR_HIP, "bread_arena_relayout",
                              hipGetErrorString(e));
        BREAD_HIP(hipDeviceSynchronize());  // no launch may still read the old block
        BREAD_HIP(hipFree(a->layers[l]));
        a->layers[l] = nb;
    }
    a->lay[l] = p;
    return BREAD_OK;
}

extern "C" int bread_arena_set_layer_types(bread_arena_t *a, int layer, int gate_type, int up_type, int down_type,
                                           int gate_shexp_type, int up_shexp_type, int down_shexp_type)
{
    BREAD_REQUIRE(a, BREAD_ERR_ARG, "NULL arena");
    BREAD_REQUIRE(layer >= 0 && layer < a->n_layers, BREAD_ERR_ARG, "layer out of range");
    const int types[6] = {gate_type, up_type, down_type, gate_shexp_type, up_shexp_type, down_shexp_type};
    for (int i = 0; i < 6; i++)
        BREAD_REQUIRE(bread_expert_qtype(types[i]), BREAD_ERR_QTYPE, "expert tensors must be Q4_K or Q6_K");
    return bread_arena_relayout(a, layer, types);
}

extern "C" uint64_t bread_arena_layer_bytes(const bread_arena_t *a)
{
    if (!a) return 0;
    uint64_t m = 0;
    for (int l = 0; l < a->n_layers; l++) m = a->lay[l].layer_bytes > m ? a->lay[l].layer_bytes : m;
    return m;
}

extern "C" int bread_arena_layer(const bread_arena_t *a, int layer, bread_moe_layer_t *L)
{
    BREAD_REQUIRE(a && L, BREAD_ERR_ARG, "NULL arena or descriptor");
    BREAD_REQUIRE(layer >= 0 && layer < a->n_layers, BREAD_ERR_ARG, "layer out of range");
    uint8_t *b = a->layers[layer];
    const bread_arena_layout &p = a->lay[layer];
    L->gate_exps = b + p.off_gate;
    L->up_exps = b + p.off_up;
    L->down_exps = b + p.off_down;
    L->gate_expert_bytes = p.gate_expert_bytes;
    L->up_expert_bytes = p.up_expert_bytes;
    L->down_expert_bytes = p.down_expert_bytes;
    L->gate_type = p.types[0];
    L->up_type = p.types[1];
    L->down_type = p.types[2];
    L->gate_shexp = b + p.off_gate_sh;
    L->up_shexp = b + p.off_up_sh;
    L->down_shexp = b + p.off_down_sh;
    L->gate_shexp_type = p.types[3];
    L->up_shexp_type = p.types[4];
    L->down_shexp_type = p.types[5];
    L->router = (const float *)(b + p.off_router);
    L->shexp_gate = (a->flags[layer] & BREAD_ARENA_HAS_SHGATE) ? (const uint16_t *)(b + p.off_shgate) : nullptr;
    L->post_norm_w = (a->flags[layer] & BREAD_ARENA_HAS_NORM) ? (const float *)(b + p.off_norm) : nullptr;
    return BREAD_OK;
}
