// gguf_load.hip — GGUF v2/v3 model files: header, metadata and tensor index
// parsing over a read-only mapping of the file, and the copy of a layer's
// MoE tensors into the HBM arena.
//
// Replaces the parser of gguf.c:306-384 (header, skipped metadata, tensor
// records, data section at the next alignment boundary) and the MoE parts of
// the reference's loader: the expert tensor scan of loader.c:160-206 (expert
// count from the outermost dimension, expert stride tensor.size / n_experts),
// the shared-expert uploads of loader.c:551-569 and the router / shared-gate
// / norm lookups of one_layer.cu:964-980 and :1413-1415.  Differences: a
// malformed file returns BREAD_ERR_FORMAT instead of exiting, every tensor's
// data range is checked against the file size, and scalar metadata can be
// queried.
//
// File layout (little-endian): "GGUF", u32 version, u64 n_tensors, u64 n_kv;
// n_kv x (string key, u32 value type, value); n_tensors x (string name, u32
// n_dims, u64 dims[n_dims] (dims[0] innermost), u32 ggml type, u64 offset
// from the data section); padding to general.alignment (default 32); data.
// A string is u64 length + bytes; an array is u32 element type + u64 count +
// elements.
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <string>
#include <vector>

#include "bread_internal.h"

namespace {

enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STRING = 8, KV_ARRAY = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12,
};

struct TypeSize {
    uint32_t type, block, bytes;
};

// ggml tensor types: elements per block and bytes per block (the GGUF
// format's block layouts).
constexpr TypeSize kTypes[] = {
    {0, 1, 4},      {1, 1, 2},      {30, 1, 2},     {28, 1, 8},     {24, 1, 1},     {25, 1, 2},
    {26, 1, 4},     {27, 1, 8},     {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
    {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
    {14, 256, 210}, {15, 256, 292}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
    {20, 32, 18},   {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {29, 256, 56},
};

const TypeSize *type_size(uint32_t t)
{
    for (const TypeSize &s : kTypes)
        if (s.type == t) return &s;
    return nullptr;
}

struct Kv {
    std::string key;
    uint32_t type;
    uint64_t u;  // integer / bool value (two's complement for signed)
    double f;    // float value
    std::string s;
};

struct Tensor {
    std::string name;
    uint32_t type, n_dims;
    uint64_t dims[4], offset, size, n_elems;
};

// Bounds-checked little-endian reader over the mapped file.
struct Reader {
    const uint8_t *p;
    uint64_t n, pos = 0;
    bool ok = true;
    bool need(uint64_t k)
    {
        if (!ok || k > n - pos) ok = false;
        return ok;
    }
    template <typename T>
    T get()
    {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str()
    {
        const uint64_t len = get<uint64_t>();
        if (!need(len)) return std::string();
        std::string s(reinterpret_cast<const char *>(p + pos), (size_t)len);
        pos += len;
        return s;
    }
    void skip(uint64_t k)
    {
        if (need(k)) pos += k;
    }
};

uint64_t scalar_bytes(uint32_t t)
{
    switch (t) {
    case KV_U8: case KV_I8: case KV_BOOL: return 1;
    case KV_U16: case KV_I16: return 2;
    case KV_U32: case KV_I32: case KV_F32: return 4;
    case KV_U64: case KV_I64: case KV_F64: return 8;
    }
    return 0;
}

bool read_value(Reader &r, uint32_t t, Kv *kv, int depth)
{
    if (depth > 4) return false;
    if (t == KV_STRING) {
        if (kv) kv->s = r.str();
        else r.skip(r.get<uint64_t>());
        return r.ok;
    }
    if (t == KV_ARRAY) {
        const uint32_t et = r.get<uint32_t>();
        const uint64_t count = r.get<uint64_t>();
        const uint64_t eb = scalar_bytes(et);
        if (eb) {
            if (count > (r.n - r.pos) / eb) return r.ok = false;
            r.skip(count * eb);
        } else {
            if (et != KV_STRING && et != KV_ARRAY) return r.ok = false;
            for (uint64_t i = 0; i < count && r.ok; i++) read_value(r, et, nullptr, depth + 1);
        }
        return r.ok;
    }
    const uint64_t b = scalar_bytes(t);
    if (!b) return r.ok = false;
    uint64_t u = 0;
    if (r.need(b)) {
        memcpy(&u, r.p + r.pos, b);
        r.pos += b;
    }
    if (kv) {
        // sign-extend signed integers; keep float values as double
        switch (t) {
        case KV_I8: u = (uint64_t)(int64_t)(int8_t)u; break;
        case KV_I16: u = (uint64_t)(int64_t)(int16_t)u; break;
        case KV_I32: u = (uint64_t)(int64_t)(int32_t)u; break;
        case KV_F32: { float f; memcpy(&f, &u, 4); kv->f = f; break; }
        case KV_F64: { double f; memcpy(&f, &u, 8); kv->f = f; break; }
        }
        kv->u = u;
    }
    return r.ok;
}

}  // namespace

struct bread_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t file_bytes = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t data_off = 0;
    std::vector<Kv> kvs;
    std::vector<Tensor> tensors;
};

static void gguf_release(bread_gguf_t *g)
{
    if (!g) return;
    if (g->map) munmap(const_cast<uint8_t *>(g->map), g->file_bytes);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

static int gguf_parse(bread_gguf_t *g)
{
    Reader r{g->map, g->file_bytes};
    const uint32_t magic = r.get<uint32_t>();
    BREAD_REQUIRE(r.ok && magic == 0x46554747u, BREAD_ERR_FORMAT, "not a GGUF file (magic)");
    g->version = r.get<uint32_t>();
    BREAD_REQUIRE(g->version == 2 || g->version == 3, BREAD_ERR_FORMAT, "unsupported GGUF version (2 and 3 are)");
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    // a KV pair takes at least 13 bytes of the file and a tensor record 24;
    // records are appended as they parse, so memory grows with the bytes read
    BREAD_REQUIRE(r.ok && n_kv <= g->file_bytes / 13 && n_tensors <= g->file_bytes / 24, BREAD_ERR_FORMAT,
                  "header counts exceed the file");
    for (uint64_t i = 0; i < n_kv; i++) {
        g->kvs.emplace_back();
        Kv &kv = g->kvs.back();
        kv.key = r.str();
        kv.type = r.get<uint32_t>();
        kv.u = 0;
        kv.f = 0.0;
        BREAD_REQUIRE(r.ok && read_value(r, kv.type, &kv, 0), BREAD_ERR_FORMAT, "metadata");
        if (kv.key == "general.alignment" && kv.type == KV_U32) g->alignment = (uint32_t)kv.u;
    }
    BREAD_REQUIRE(g->alignment > 0, BREAD_ERR_FORMAT, "general.alignment is 0");
    for (uint64_t i = 0; i < n_tensors; i++) {
        g->tensors.emplace_back();
        Tensor &t = g->tensors.back();
        t.name = r.str();
        t.n_dims = r.get<uint32_t>();
        BREAD_REQUIRE(r.ok && t.n_dims <= 4, BREAD_ERR_FORMAT, "tensor with more than 4 dimensions");
        t.n_elems = 1;
        for (uint32_t d = 0; d < 4; d++) {
            t.dims[d] = d < t.n_dims ? r.get<uint64_t>() : 0;
            if (d < t.n_dims) {
                BREAD_REQUIRE(t.dims[d] == 0 || t.n_elems <= UINT64_MAX / t.dims[d], BREAD_ERR_FORMAT,
                              "tensor element count overflows");
                t.n_elems *= t.dims[d];
            }
        }
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        BREAD_REQUIRE(r.ok, BREAD_ERR_FORMAT, "tensor records");
        const TypeSize *ts = type_size(t.type);
        t.size = (ts && t.n_elems % ts->block == 0) ? t.n_elems / ts->block * ts->bytes : 0;
    }
    g->data_off = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (const Tensor &t : g->tensors) {
        const bool fits = g->data_off <= g->file_bytes && t.offset <= g->file_bytes - g->data_off &&
                          t.size <= g->file_bytes - g->data_off - t.offset;
        BREAD_REQUIRE(fits, BREAD_ERR_FORMAT, "tensor data beyond the end of the file");
    }
    return BREAD_OK;
}

static const Tensor *find(const bread_gguf_t *g, const char *name)
{
    for (const Tensor &t : g->tensors)
        if (t.name == name) return &t;
    return nullptr;
}

static const Kv *find_kv(const bread_gguf_t *g, const char *key)
{
    for (const Kv &kv : g->kvs)
        if (kv.key == key) return &kv;
    return nullptr;
}

static void fill(const bread_gguf_t *g, const Tensor &t, bread_gguf_tensor_t *o)
{
    o->name = t.name.c_str();
    o->type = t.type;
    o->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) o->dims[d] = t.dims[d];
    o->offset = t.offset;
    o->size = t.size;
    o->n_elems = t.n_elems;
    o->data = g->map + g->data_off + t.offset;
}

extern "C" int bread_gguf_open(const char *path, bread_gguf_t **out)
{
    BREAD_REQUIRE(path && out, BREAD_ERR_ARG, "NULL path or out");
    *out = nullptr;
    bread_gguf_t *g = new (std::nothrow) bread_gguf_t();
    BREAD_REQUIRE(g, BREAD_ERR_NOMEM, "host allocation");
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) {
        gguf_release(g);
        return bread_fail(BREAD_ERR_ARG, "bread_gguf_open", "cannot open the file");
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        gguf_release(g);
        return bread_fail(BREAD_ERR_FORMAT, "bread_gguf_open", "empty or unreadable file");
    }
    g->file_bytes = (uint64_t)st.st_size;
    void *m = mmap(nullptr, g->file_bytes, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        gguf_release(g);
        return bread_fail(BREAD_ERR_NOMEM, "bread_gguf_open", "mmap failed");
    }
    g->map = static_cast<const uint8_t *>(m);
    int rc;
    try {
        rc = gguf_parse(g);
    } catch (const std::bad_alloc &) {
        rc = bread_fail(BREAD_ERR_NOMEM, "bread_gguf_open", "host allocation while parsing");
    }
    if (rc != BREAD_OK) {
        gguf_release(g);
        return rc;
    }
    *out = g;
    return BREAD_OK;
}

extern "C" int bread_gguf_close(bread_gguf_t *g)
{
    gguf_release(g);
    return BREAD_OK;
}

extern "C" int bread_gguf_info(const bread_gguf_t *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv,
                               uint64_t *data_offset, uint32_t *alignment)
{
    BREAD_REQUIRE(g, BREAD_ERR_ARG, "NULL file");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kvs.size();
    if (data_offset) *data_offset = g->data_off;
    if (alignment) *alignment = g->alignment;
    return BREAD_OK;
}

extern "C" int bread_gguf_tensor(const bread_gguf_t *g, uint64_t idx, bread_gguf_tensor_t *out)
{
    BREAD_REQUIRE(g && out, BREAD_ERR_ARG, "NULL file or out");
    BREAD_REQUIRE(idx < g->tensors.size(), BREAD_ERR_ARG, "tensor index out of range");
    fill(g, g->tensors[idx], out);
    return BREAD_OK;
}

extern "C" int bread_gguf_find(const bread_gguf_t *g, const char *name, bread_gguf_tensor_t *out)
{
    BREAD_REQUIRE(g && name && out, BREAD_ERR_ARG, "NULL argument");
    const Tensor *t = find(g, name);
    if (!t) return BREAD_ERR_ARG;  // absence is an answer, not an error to record
    fill(g, *t, out);
    return BREAD_OK;
}

extern "C" int bread_gguf_kv_int(const bread_gguf_t *g, const char *key, int64_t *value)
{
    BREAD_REQUIRE(g && key && value, BREAD_ERR_ARG, "NULL argument");
    const Kv *kv = find_kv(g, key);
    if (!kv || kv->type == KV_STRING || kv->type == KV_ARRAY || kv->type == KV_F32 || kv->type == KV_F64)
        return BREAD_ERR_ARG;
    *value = (int64_t)kv->u;
    return BREAD_OK;
}

extern "C" int bread_gguf_kv_float(const bread_gguf_t *g, const char *key, double *value)
{
    BREAD_REQUIRE(g && key && value, BREAD_ERR_ARG, "NULL argument");
    const Kv *kv = find_kv(g, key);
    if (!kv || (kv->type != KV_F32 && kv->type != KV_F64)) return BREAD_ERR_ARG;
    *value = kv->f;
    return BREAD_OK;
}

extern "C" int bread_gguf_kv_str(const bread_gguf_t *g, const char *key, char *buf, size_t buf_len)
{
    BREAD_REQUIRE(g && key && buf && buf_len > 0, BREAD_ERR_ARG, "NULL argument");
    const Kv *kv = find_kv(g, key);
    if (!kv || kv->type != KV_STRING) return BREAD_ERR_ARG;
    const size_t n = kv->s.size() < buf_len - 1 ? kv->s.size() : buf_len - 1;
    memcpy(buf, kv->s.data(), n);
    buf[n] = '\0';
    return BREAD_OK;
}

extern "C" uint64_t bread_ggml_type_size(uint32_t type, uint64_t n_elems)
{
    const TypeSize *ts = type_size(type);
    return (ts && n_elems % ts->block == 0) ? n_elems / ts->block * ts->bytes : 0;
}

static std::string layer_name(int layer, const char *suffix)
{
    char b[128];
    snprintf(b, sizeof(b), "blk.%d.%s", layer, suffix);
    return b;
}

extern "C" int bread_gguf_moe_shape(const bread_gguf_t *g, int layer, bread_moe_shape_t *shape)
{
    BREAD_REQUIRE(g && shape, BREAD_ERR_ARG, "NULL argument");
    const Tensor *gate = find(g, layer_name(layer, "ffn_gate_exps.weight").c_str());
    const Tensor *gsh = find(g, layer_name(layer, "ffn_gate_shexp.weight").c_str());
    BREAD_REQUIRE(gate && gate->n_dims == 3, BREAD_ERR_SHAPE, "layer has no 3-d ffn_gate_exps tensor");
    BREAD_REQUIRE(gsh && gsh->n_dims == 2, BREAD_ERR_SHAPE, "layer has no ffn_gate_shexp tensor");
    bread_moe_shape_default(shape);
    shape->hidden = (int)gate->dims[0];
    shape->expert_inter = (int)gate->dims[1];
    shape->n_experts = (int)gate->dims[2];
    shape->shared_inter = (int)gsh->dims[1];
    // top-k and epsilon from the architecture's metadata when present
    char arch[64];
    if (bread_gguf_kv_str(g, "general.architecture", arch, sizeof(arch)) == BREAD_OK) {
        int64_t k;
        double eps;
        const std::string a(arch);
        if (bread_gguf_kv_int(g, (a + ".expert_used_count").c_str(), &k) == BREAD_OK) shape->top_k = (int)k;
        if (bread_gguf_kv_float(g, (a + ".attention.layer_norm_rms_epsilon").c_str(), &eps) == BREAD_OK)
            shape->rms_eps = (float)eps;
    }
    return BREAD_OK;
}

// One layer's MoE tensors into layer `arena_layer` of the arena: routed and
// shared gate/up/down (each Q4_K or Q6_K, as the file gives them; the arena
// layer is re-laid out for those types), the fp32 router, the optional fp16
// shared gate and the optional fp32 post-attention norm weight.
extern "C" int bread_arena_load_gguf(bread_arena_t *a, int arena_layer, const bread_gguf_t *g, int gguf_layer)
{
    BREAD_REQUIRE(a && g, BREAD_ERR_ARG, "NULL arena or file");
    BREAD_REQUIRE(arena_layer >= 0 && arena_layer < a->n_layers, BREAD_ERR_ARG, "arena layer out of range");
    const bread_moe_shape_t &s = a->shape;
    const uint64_t H = (uint64_t)s.hidden, I = (uint64_t)s.expert_inter, Ish = (uint64_t)s.shared_inter;
    const uint64_t E = (uint64_t)s.n_experts;
    constexpr uint32_t EXPERT = 0xFFFFFFFFu;  // Q4_K or Q6_K
    struct Want {
        const char *suffix;
        uint32_t type;
        uint64_t d0, d1, d2;  // expected dims (d2 = 0: 2-d, d1 = 0: 1-d)
        bool optional;
    };
    const Want want[] = {
        {"ffn_gate_exps.weight", EXPERT, H, I, E, false},
        {"ffn_up_exps.weight", EXPERT, H, I, E, false},
        {"ffn_down_exps.weight", EXPERT, I, H, E, false},
        {"ffn_gate_shexp.weight", EXPERT, H, Ish, 0, false},
        {"ffn_up_shexp.weight", EXPERT, H, Ish, 0, false},
        {"ffn_down_shexp.weight", EXPERT, Ish, H, 0, false},
        {"ffn_gate_inp.weight", 0 /* F32 */, H, E, 0, false},
        {"ffn_gate_inp_shexp.weight", 1 /* F16 */, H, 0, 0, true},
        {"post_attention_norm.weight", 0 /* F32 */, H, 0, 0, true},
    };
    const Tensor *found[9];
    int types[6];
    for (int i = 0; i < 9; i++) {
        const Want &w = want[i];
        const Tensor *t = find(g, layer_name(gguf_layer, w.suffix).c_str());
        found[i] = t;
        if (!t) {
            BREAD_REQUIRE(w.optional, BREAD_ERR_SHAPE, "a MoE tensor of the layer is missing");
            continue;
        }
        if (w.type == EXPERT) {
            BREAD_REQUIRE(bread_expert_qtype((int)t->type), BREAD_ERR_QTYPE, "expert tensors must be Q4_K or Q6_K");
            types[i] = (int)t->type;
        } else {
            BREAD_REQUIRE(t->type == w.type, BREAD_ERR_QTYPE, "router, shared gate and norm must be F32, F16, F32");
        }
        const uint32_t nd = w.d2 ? 3 : (w.d1 ? 2 : 1);
        // vectors may carry trailing unit dimensions ([H] or [H, 1])
        bool dims_ok = (nd == 1 ? t->n_elems == w.d0 : t->n_dims == nd) && t->dims[0] == w.d0;
        if (nd >= 2) dims_ok = dims_ok && t->dims[1] == w.d1;
        if (nd == 3) dims_ok = dims_ok && t->dims[2] == w.d2;
        BREAD_REQUIRE(dims_ok && t->size > 0, BREAD_ERR_SHAPE, "tensor dimensions differ from the arena's shape");
    }
    const int rc = bread_arena_relayout(a, arena_layer, types);
    if (rc) return rc;
    const bread_arena_layout &p = a->lay[arena_layer];
    const uint64_t off[9] = {p.off_gate,    p.off_up,     p.off_down,   p.off_gate_sh, p.off_up_sh,
                             p.off_down_sh, p.off_router, p.off_shgate, p.off_norm};
    uint8_t *base = a->layers[arena_layer];
    for (int i = 0; i < 9; i++) {
        if (!found[i]) continue;
        BREAD_HIP(hipMemcpy(base + off[i], g->map + g->data_off + found[i]->offset, found[i]->size,
                            hipMemcpyHostToDevice));
    }
    a->flags[arena_layer] = (found[7] ? BREAD_ARENA_HAS_SHGATE : 0) | (found[8] ? BREAD_ARENA_HAS_NORM : 0);
    return BREAD_OK;
}
