// abi_caller.cpp — a C++ translation unit that calls libbread_moe the way the
// reference's own translation units would after the swap:
//   - bread_matvec through the reference's own prototype (one_layer.cu:46-47,
//     main.cu:65-66, expert_bench.cu:15-16), with CUDA's `half` and
//     `cudaStream_t` spelled as HIP's __half and hipStream_t, called with the
//     arguments of one_layer.cu:1840-1843 (shared gate/up) and :1966-1977
//     (routed gate/up, then down);
//   - the MoE block of one_layer_forward as one bread_moe_forward_f16 call on
//     the fp16 d_hidden / d_normed2 buffers (one_layer.cu:1800-1986).
// Built and linked by tests/test_abi.py; run on a GPU by
// tests/test_gpu_abi_caller.py, which writes the inputs and checks the
// outputs against the CPU oracle.
//
//   abi_caller matvec DIR  DIR/meta.txt: "rows cols qtype"; DIR/w.bin (weights),
//                          DIR/x.bin (fp16 [cols]) -> DIR/y.bin (fp16 [rows])
//   abi_caller moe DIR     DIR/meta.txt: "H I Ish E K eps"; DIR/{gate,up,down}_exps.bin,
//                          DIR/{gate,up,down}_sh.bin (Q4_K gate/up, Q6_K down),
//                          DIR/router.bin (fp32 [E][H]), DIR/shgate.bin (fp16 [H]),
//                          DIR/norm_w.bin (fp32 [H]), DIR/hidden.bin (fp16 [H])
//                          -> DIR/hidden_out.bin, DIR/normed.bin (fp16 [H]),
//                             DIR/idx.bin (int32 [K]), DIR/w.bin (fp32 [K])
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include <string>
#include <vector>

#include "bread_moe.h"

// The reference's declaration, unchanged but for the HIP spelling of its types.
typedef __half half;
typedef hipStream_t cudaStream_t;
extern void bread_matvec(void *w, half *x, half *y, int rows, int cols, int qtype, cudaStream_t stream);

#define CHECK_HIP(e)                                                                  \
    do {                                                                              \
        hipError_t rc_ = (e);                                                         \
        if (rc_ != hipSuccess) {                                                      \
            fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(rc_), __FILE__, __LINE__); \
            exit(2);                                                                  \
        }                                                                             \
    } while (0)

#define CHECK_BREAD(e)                                                                \
    do {                                                                              \
        int rc_ = (e);                                                                \
        if (rc_ != BREAD_OK) {                                                        \
            fprintf(stderr, "%s failed: %s (%s)\n", #e, bread_status_str(rc_), bread_last_error()); \
            exit(3);                                                                  \
        }                                                                             \
    } while (0)

static std::vector<char> read_file(const std::string &path)
{
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path.c_str());
        exit(4);
    }
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    std::vector<char> v((size_t)n);
    if (n > 0 && fread(v.data(), 1, (size_t)n, f) != (size_t)n) exit(4);
    fclose(f);
    return v;
}

static void write_file(const std::string &path, const void *p, size_t n)
{
    FILE *f = fopen(path.c_str(), "wb");
    if (!f || fwrite(p, 1, n, f) != n) {
        fprintf(stderr, "cannot write %s\n", path.c_str());
        exit(4);
    }
    fclose(f);
}

static void *upload(const std::string &path, size_t *bytes = nullptr)
{
    const std::vector<char> h = read_file(path);
    void *d = nullptr;
    CHECK_HIP(hipMalloc(&d, h.size() + 16));
    CHECK_HIP(hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice));
    if (bytes) *bytes = h.size();
    return d;
}

static int run_matvec(const std::string &dir)
{
    int rows = 0, cols = 0, qtype = 0;
    FILE *m = fopen((dir + "/meta.txt").c_str(), "r");
    if (!m || fscanf(m, "%d %d %d", &rows, &cols, &qtype) != 3) return 4;
    fclose(m);
    void *d_w = upload(dir + "/w.bin");
    half *d_x = static_cast<half *>(upload(dir + "/x.bin"));
    half *d_y = nullptr;
    CHECK_HIP(hipMalloc(&d_y, (size_t)rows * sizeof(half)));
    cudaStream_t stream_a;
    CHECK_HIP(hipStreamCreate(&stream_a));
    // one_layer.cu:1966-1967 / 1976-1977: bread_matvec(d_w, d_in, d_out, rows, cols, type, stream_a)
    bread_matvec(d_w, d_x, d_y, rows, cols, qtype, stream_a);
    CHECK_HIP(hipStreamSynchronize(stream_a));
    std::vector<half> y((size_t)rows);
    CHECK_HIP(hipMemcpy(y.data(), d_y, y.size() * sizeof(half), hipMemcpyDeviceToHost));
    write_file(dir + "/y.bin", y.data(), y.size() * sizeof(half));
    CHECK_HIP(hipStreamDestroy(stream_a));
    CHECK_HIP(hipFree(d_w));
    CHECK_HIP(hipFree(d_x));
    CHECK_HIP(hipFree(d_y));
    return 0;
}

static int run_moe(const std::string &dir)
{
    bread_moe_shape_t s;
    bread_moe_shape_default(&s);
    FILE *m = fopen((dir + "/meta.txt").c_str(), "r");
    if (!m || fscanf(m, "%d %d %d %d %d %f", &s.hidden, &s.expert_inter, &s.shared_inter, &s.n_experts, &s.top_k,
                     &s.rms_eps) != 6)
        return 4;
    fclose(m);
    const int H = s.hidden, K = s.top_k, E = s.n_experts;
    // the layer descriptor, as the reference's loader tables fill it
    bread_moe_layer_t lay = {};
    size_t nb = 0;
    lay.gate_exps = upload(dir + "/gate_exps.bin", &nb);
    lay.gate_expert_bytes = nb / (size_t)E;
    lay.up_exps = upload(dir + "/up_exps.bin", &nb);
    lay.up_expert_bytes = nb / (size_t)E;
    lay.down_exps = upload(dir + "/down_exps.bin", &nb);
    lay.down_expert_bytes = nb / (size_t)E;
    lay.gate_type = lay.up_type = BREAD_QTYPE_Q4_K;
    lay.down_type = BREAD_QTYPE_Q6_K;
    lay.gate_shexp = upload(dir + "/gate_sh.bin");
    lay.up_shexp = upload(dir + "/up_sh.bin");
    lay.down_shexp = upload(dir + "/down_sh.bin");
    lay.gate_shexp_type = lay.up_shexp_type = BREAD_QTYPE_Q4_K;
    lay.down_shexp_type = BREAD_QTYPE_Q6_K;
    lay.router = static_cast<const float *>(upload(dir + "/router.bin"));
    lay.shexp_gate = static_cast<const uint16_t *>(upload(dir + "/shgate.bin"));
    const float *norm_w = static_cast<const float *>(upload(dir + "/norm_w.bin"));
    uint16_t *d_hidden = static_cast<uint16_t *>(upload(dir + "/hidden.bin"));
    uint16_t *d_normed2 = nullptr;
    int32_t *d_idx = nullptr;
    float *d_wt = nullptr;
    CHECK_HIP(hipMalloc(&d_normed2, (size_t)H * sizeof(uint16_t)));
    CHECK_HIP(hipMalloc(&d_idx, (size_t)K * sizeof(int32_t)));
    CHECK_HIP(hipMalloc(&d_wt, (size_t)K * sizeof(float)));
    cudaStream_t stream_a;
    CHECK_HIP(hipStreamCreate(&stream_a));
    bread_moe_ctx_t *g_moe = nullptr;
    CHECK_BREAD(bread_moe_ctx_create(&s, 1, &g_moe));
    // one_layer.cu:1800-1986 as one call on the fp16 d_hidden / d_normed2 buffers
    CHECK_BREAD(bread_moe_forward_f16(g_moe, &lay, norm_w, d_hidden, d_normed2, 1, d_idx, d_wt, nullptr,
                                      (bread_stream_t)stream_a));
    int dev_err = 0;
    CHECK_BREAD(bread_moe_ctx_check(g_moe, &dev_err));
    std::vector<uint16_t> hid((size_t)H), nrm((size_t)H);
    std::vector<int32_t> idx((size_t)K);
    std::vector<float> wt((size_t)K);
    CHECK_HIP(hipMemcpy(hid.data(), d_hidden, hid.size() * 2, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(nrm.data(), d_normed2, nrm.size() * 2, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(idx.data(), d_idx, idx.size() * 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(wt.data(), d_wt, wt.size() * 4, hipMemcpyDeviceToHost));
    write_file(dir + "/hidden_out.bin", hid.data(), hid.size() * 2);
    write_file(dir + "/normed.bin", nrm.data(), nrm.size() * 2);
    write_file(dir + "/idx.bin", idx.data(), idx.size() * 4);
    write_file(dir + "/w.bin", wt.data(), wt.size() * 4);
    CHECK_BREAD(bread_moe_ctx_destroy(g_moe));
    CHECK_HIP(hipStreamDestroy(stream_a));
    return 0;
}

int main(int argc, char **argv)
{
    if (argc != 3) {
        fprintf(stderr, "usage: %s matvec|moe DIR\n", argv[0]);
        return 1;
    }
    const std::string mode = argv[1], dir = argv[2];
    if (mode == "matvec") return run_matvec(dir);
    if (mode == "moe") return run_moe(dir);
    fprintf(stderr, "unknown mode %s\n", mode.c_str());
    return 1;
}
