// GGUF model files on the host: the file is mapped read-only, its header,
// metadata and tensor table are parsed with every read bounds-checked, and one
// layer's MoE tensors are bound into a jx_moe_layer_desc whose pointers point
// into the mapping -- the expert path's share of ModelFile::parse_gguf
// (src/gguf.cpp:810-889) and MoETransformerEngine::bind_tensors
// (src/transformer.cpp:1954-1972, 2116-2186).  jx_moe_layer_create then
// copies the bytes to HBM once.  No device code.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/jxmoe.h"

namespace {

thread_local std::string g_gguf_err;

int gfail(int code, const std::string& msg) {
    g_gguf_err = msg;
    return code;
}

// GGUF metadata value types (the GGUF specification; GGUFValueType, include/gguf.h:10-24)
enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

// Block geometry of the GGML types a GGUF file may hold (include/common.h:119-189):
// (elements per block, bytes per block).  Unknown codes count as 4-byte elements,
// as tensor_byte_size does (include/common.h:191-195).
struct Geom {
    uint32_t blk, bytes;
};
Geom geom(uint32_t t) {
    switch (t) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 36};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
        case 16: return {256, 66};  // IQ2_XXS
        case 17: return {256, 74};  // IQ2_XS
        case 18: return {256, 98};  // IQ3_XXS
        case 19: return {256, 50};  // IQ1_S
        case 20: return {32, 18};   // IQ4_NL
        case 21: return {256, 110}; // IQ3_S
        case 22: return {256, 82};  // IQ2_S
        case 23: return {256, 136}; // IQ4_XS
        case 24: return {1, 1};     // I8
        case 25: return {1, 2};     // I16
        case 26: return {1, 4};     // I32
        case 27: return {1, 8};     // I64
        case 28: return {1, 8};     // F64
        case 29: return {256, 56};  // IQ1_M
        case 30: return {1, 2};     // BF16
        case 31: return {1, 1};     // FP8_E4M3
        case 36: return {256, 86};  // IQ2_M
        default: return {1, 4};
    }
}

struct Value {
    uint32_t type = V_U32;
    uint64_t u = 0;     // unsigned integers, bool; signed integers as their two's complement
    double f = 0.0;     // floats
    std::string s;      // strings
    uint64_t count = 0; // arrays: element count
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t rel = 0;     // offset inside the data section
    uint64_t off = 0;     // offset from the start of the file
    uint64_t bytes = 0;   // whole-tensor bytes: ceil(elements / block) * block bytes
};

// Bounds-checked little-endian reader over the mapping.
struct Cursor {
    const uint8_t* p;
    uint64_t size, pos;
    template <typename T>
    bool get(T& v) {
        if (pos > size || size - pos < sizeof(T)) return false;
        std::memcpy(&v, p + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool str(std::string& s) {
        uint64_t n = 0;
        if (!get(n) || pos > size || size - pos < n) return false;
        s.assign(reinterpret_cast<const char*>(p + pos), (size_t)n);
        pos += n;
        return true;
    }
    bool skip(uint64_t n) {
        if (pos > size || size - pos < n) return false;
        pos += n;
        return true;
    }
};

bool read_value(Cursor& c, uint32_t type, Value& v, int depth = 0) {
    v.type = type;
    switch (type) {
        case V_U8: case V_I8: case V_BOOL: {
            uint8_t x;
            if (!c.get(x)) return false;
            v.u = type == V_I8 ? (uint64_t)(int64_t)(int8_t)x : (type == V_BOOL ? (x != 0) : x);
            return true;
        }
        case V_U16: case V_I16: {
            uint16_t x;
            if (!c.get(x)) return false;
            v.u = type == V_I16 ? (uint64_t)(int64_t)(int16_t)x : x;
            return true;
        }
        case V_U32: case V_I32: {
            uint32_t x;
            if (!c.get(x)) return false;
            v.u = type == V_I32 ? (uint64_t)(int64_t)(int32_t)x : x;
            return true;
        }
        case V_U64: case V_I64: return c.get(v.u);
        case V_F32: {
            float x;
            if (!c.get(x)) return false;
            v.f = x;
            return true;
        }
        case V_F64: return c.get(v.f);
        case V_STR: return c.str(v.s);
        case V_ARR: {  // at most 10M entries, as the reference reader accepts (src/gguf.cpp:771)
            uint32_t et = 0;
            if (depth > 8 || !c.get(et) || !c.get(v.count) || v.count > 10000000ull) return false;
            const uint64_t fixed = et == V_U8 || et == V_I8 || et == V_BOOL ? 1 : et == V_U16 || et == V_I16 ? 2
                                 : et == V_U32 || et == V_I32 || et == V_F32 ? 4
                                 : et == V_U64 || et == V_I64 || et == V_F64 ? 8 : 0;
            if (fixed) return v.count <= (c.size - c.pos) / fixed && c.skip(v.count * fixed);
            for (uint64_t i = 0; i < v.count; ++i) {  // strings, nested arrays
                Value e;
                if (!read_value(c, et, e, depth + 1)) return false;
            }
            return true;
        }
        default: return false;
    }
}

}  // namespace

struct jx_gguf {
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_offset = 0;
    std::unordered_map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> index;
    std::vector<std::vector<float>> owned;  // zero routers bound for dense FFN layers
    ~jx_gguf() {
        if (base) munmap(const_cast<uint8_t*>(base), size);
        if (fd >= 0) close(fd);
    }
};

namespace {

int parse(jx_gguf* g) {
    Cursor c{g->base, g->size, 0};
    uint32_t magic = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!c.get(magic) || magic != 0x46554747u) return gfail(JX_ERR_INVALID, "not a GGUF file (magic)");
    if (!c.get(g->version) || (g->version != 2 && g->version != 3))
        return gfail(JX_ERR_UNSUPPORTED, "GGUF version " + std::to_string(g->version) + " (2 and 3 are read)");
    if (!c.get(n_tensors) || !c.get(n_kv)) return gfail(JX_ERR_INVALID, "truncated GGUF header");
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t type = 0;
        Value v;
        if (!c.str(key) || !c.get(type) || !read_value(c, type, v))
            return gfail(JX_ERR_INVALID, "truncated or malformed metadata entry " + std::to_string(i));
        if (key == "general.alignment" && type != V_F32 && type != V_F64 && type != V_STR && type != V_ARR && v.u > 0)
            g->alignment = (uint32_t)v.u;
        g->meta[key] = std::move(v);
    }
    if (n_tensors > (g->size - c.pos) / 24) return gfail(JX_ERR_INVALID, "tensor count exceeds the file");
    g->tensors.resize((size_t)n_tensors);
    for (auto& t : g->tensors) {
        uint64_t ne = 1;
        if (!c.str(t.name) || !c.get(t.n_dims) || t.n_dims > 4)
            return gfail(JX_ERR_INVALID, "malformed tensor descriptor");
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            if (!c.get(t.dims[d])) return gfail(JX_ERR_INVALID, "truncated tensor dims: " + t.name);
            if (t.dims[d] != 0 && ne > UINT64_MAX / t.dims[d]) return gfail(JX_ERR_INVALID, "tensor too large: " + t.name);
            ne *= t.dims[d];
        }
        if (!c.get(t.type) || !c.get(t.rel)) return gfail(JX_ERR_INVALID, "truncated tensor descriptor: " + t.name);
        const Geom gm = geom(t.type);
        t.bytes = (ne + gm.blk - 1) / gm.blk * gm.bytes;
    }
    // the data section starts at the next multiple of general.alignment
    const uint64_t a = g->alignment;
    g->data_offset = (c.pos + a - 1) / a * a;
    for (size_t i = 0; i < g->tensors.size(); ++i) {
        Tensor& t = g->tensors[i];
        t.off = g->data_offset + t.rel;
        if (t.off < t.rel || t.off > g->size || g->size - t.off < t.bytes)
            return gfail(JX_ERR_INVALID, "tensor exceeds the file: " + t.name);
        g->index[t.name] = i;
    }
    return JX_OK;
}

const Tensor* find(const jx_gguf* g, const std::string& name) {
    auto it = g->index.find(name);
    return it == g->index.end() ? nullptr : &g->tensors[it->second];
}

uint32_t meta_u32(const jx_gguf* g, const std::string& key, uint32_t def) {
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return def;
    return it->second.type == V_F32 || it->second.type == V_F64 ? 0u : (uint32_t)it->second.u;
}

float meta_f32(const jx_gguf* g, const std::string& key, float def) {
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return def;
    return it->second.type == V_F32 || it->second.type == V_F64 ? (float)it->second.f : 0.0f;
}

uint64_t row_bytes(uint32_t type, uint64_t cols) {
    const Geom gm = geom(type);
    return (cols + gm.blk - 1) / gm.blk * gm.bytes;
}

}  // namespace

extern "C" {

const char* jx_gguf_last_error(void) { return g_gguf_err.c_str(); }

int jx_gguf_open(const char* path, jx_gguf** out) {
    if (!path || !out) return gfail(JX_ERR_INVALID, "null argument");
    *out = nullptr;
    auto* g = new jx_gguf();
    g->fd = open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0) {
        delete g;
        return gfail(JX_ERR_INVALID, std::string("cannot open ") + path);
    }
    g->size = (uint64_t)st.st_size;
    if (g->size < 24) {
        delete g;
        return gfail(JX_ERR_INVALID, "file too small for a GGUF header");
    }
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        delete g;
        return gfail(JX_ERR_INVALID, std::string("cannot map ") + path);
    }
    g->base = static_cast<const uint8_t*>(m);
    const int r = parse(g);
    if (r != JX_OK) {
        delete g;
        return r;
    }
    *out = g;
    return JX_OK;
}

void jx_gguf_close(jx_gguf* g) { delete g; }

int64_t jx_gguf_tensor_count(const jx_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int64_t jx_gguf_find_tensor(const jx_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->index.find(name);
    return it == g->index.end() ? -1 : (int64_t)it->second;
}

int jx_gguf_tensor_info(const jx_gguf* g, int64_t i, const char** name, int32_t* type, int32_t* n_dims, uint64_t* dims,
                        uint64_t* file_offset, uint64_t* nbytes, const void** data) {
    if (!g || i < 0 || (uint64_t)i >= g->tensors.size()) return gfail(JX_ERR_INVALID, "tensor index out of range");
    const Tensor& t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (type) *type = (int32_t)t.type;
    if (n_dims) *n_dims = (int32_t)t.n_dims;
    if (dims)
        for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (file_offset) *file_offset = t.off;
    if (nbytes) *nbytes = t.bytes;
    if (data) *data = g->base + t.off;
    return JX_OK;
}

int jx_gguf_get_u32(const jx_gguf* g, const char* key, uint32_t def, uint32_t* out) {
    if (!g || !key || !out) return gfail(JX_ERR_INVALID, "null argument");
    *out = meta_u32(g, key, def);
    return JX_OK;
}

int jx_gguf_get_f32(const jx_gguf* g, const char* key, float def, float* out) {
    if (!g || !key || !out) return gfail(JX_ERR_INVALID, "null argument");
    *out = meta_f32(g, key, def);
    return JX_OK;
}

int jx_gguf_get_str(const jx_gguf* g, const char* key, const char** out) {
    if (!g || !key || !out) return gfail(JX_ERR_INVALID, "null argument");
    auto it = g->meta.find(key);
    *out = (it != g->meta.end() && it->second.type == V_STR) ? it->second.s.c_str() : nullptr;
    return JX_OK;
}

int jx_gguf_moe_layer_desc(jx_gguf* g, int32_t layer, jx_moe_layer_desc* d) {
    if (!g || !d) return gfail(JX_ERR_INVALID, "null argument");
    std::memset(d, 0, sizeof(*d));
    auto it = g->meta.find("general.architecture");
    const std::string arch = it != g->meta.end() && it->second.type == V_STR ? it->second.s : "qwen2moe";
    const std::string bp = "blk." + std::to_string(layer) + ".";
    const Tensor* ge = find(g, bp + "ffn_gate_exps.weight");
    const Tensor* ue = find(g, bp + "ffn_up_exps.weight");
    const Tensor* de = find(g, bp + "ffn_down_exps.weight");
    const Tensor* router = find(g, bp + "ffn_gate_inp.weight");
    if (ge && ue && de) {  // packed experts [d_model, d_ff, E] / [d_ff, d_model, E]
        if (ge->n_dims < 2) return gfail(JX_ERR_INVALID, bp + "ffn_gate_exps.weight has fewer than 2 dims");
        d->d_model = (int32_t)ge->dims[0];
        d->d_ff = (int32_t)ge->dims[1];
        d->n_experts = ge->n_dims >= 3 ? (int32_t)ge->dims[2]
                                       : (int32_t)meta_u32(g, arch + ".expert_count", 8);
        d->top_k = (int32_t)meta_u32(g, arch + ".expert_used_count", 2);
        if (!router) return gfail(JX_ERR_UNSUPPORTED, bp + "ffn_gate_inp.weight missing (no router)");
    } else {  // a dense FFN is the MoE block with one expert at top-1 (transformer.cpp:2187-2199)
        ge = find(g, bp + "ffn_gate.weight");
        ue = find(g, bp + "ffn_up.weight");
        de = find(g, bp + "ffn_down.weight");
        if (!ge || !ue || !de) return gfail(JX_ERR_INVALID, "layer " + std::to_string(layer) + " has no FFN tensors");
        d->d_model = (int32_t)ge->dims[0];
        d->d_ff = ge->n_dims >= 2 ? (int32_t)ge->dims[1] : (int32_t)meta_u32(g, arch + ".feed_forward_length", 256);
        d->n_experts = 1;
        d->top_k = 1;
        router = nullptr;
    }
    const uint64_t E = (uint64_t)d->n_experts, D = (uint64_t)d->d_model, Fd = (uint64_t)d->d_ff;
    if (E == 0 || D == 0 || Fd == 0) return gfail(JX_ERR_INVALID, "zero-sized expert tensor");
    // the packed expert slices must hold whole rows (expert e at e * bytes / E, transformer.cpp:2166-2185)
    if (ge->bytes != E * Fd * row_bytes(ge->type, D) || ue->bytes != E * Fd * row_bytes(ue->type, D) ||
        de->bytes != E * D * row_bytes(de->type, Fd))
        return gfail(JX_ERR_UNSUPPORTED, bp + " expert tensors are not whole rows per expert");
    d->gate_type = (int32_t)ge->type;
    d->up_type = (int32_t)ue->type;
    d->down_type = (int32_t)de->type;
    d->gate_exps = g->base + ge->off;
    d->up_exps = g->base + ue->off;
    d->down_exps = g->base + de->off;
    if (router) {
        if (router->dims[0] != D || (router->n_dims >= 2 ? router->dims[1] : 1) != E)
            return gfail(JX_ERR_INVALID, bp + "ffn_gate_inp.weight is not [d_model, n_experts]");
        d->router = reinterpret_cast<const float*>(g->base + router->off);
        d->router_type = (int32_t)router->type;
    } else {  // one expert: the selection is that expert with weight 1 whatever the logit
        g->owned.emplace_back((size_t)D, 0.0f);
        d->router = g->owned.back().data();
        d->router_type = JX_TYPE_F32;
    }
    const Tensor* sg = find(g, bp + "ffn_gate_shexp.weight");
    const Tensor* su = find(g, bp + "ffn_up_shexp.weight");
    const Tensor* sd = find(g, bp + "ffn_down_shexp.weight");
    if (sg && su && sd) {  // shared expert (transformer.cpp:2142-2146)
        const uint64_t Fs = sg->n_dims >= 2 ? sg->dims[1] : 0;
        if (Fs == 0 || sg->dims[0] != D || sg->bytes != Fs * row_bytes(sg->type, D) ||
            su->bytes != Fs * row_bytes(su->type, D) || sd->bytes != D * row_bytes(sd->type, Fs))
            return gfail(JX_ERR_UNSUPPORTED, bp + " shared expert tensors do not match d_model");
        d->d_ff_shared = (int32_t)Fs;
        d->sh_gate_type = (int32_t)sg->type;
        d->sh_up_type = (int32_t)su->type;
        d->sh_down_type = (int32_t)sd->type;
        d->sh_gate = g->base + sg->off;
        d->sh_up = g->base + su->off;
        d->sh_down = g->base + sd->off;
        if (const Tensor* si = find(g, bp + "ffn_gate_inp_shexp.weight")) {
            if (si->type != JX_TYPE_F32 || si->bytes != D * 4)
                return gfail(JX_ERR_UNSUPPORTED, bp + "ffn_gate_inp_shexp.weight must be F32 [d_model]");
            d->sh_gate_inp = reinterpret_cast<const float*>(g->base + si->off);
        }
    }
    // the steps either side of the block: ffn_norm and post_ffw_norm are used when F32
    // (transformer.cpp:2585-2587, 2758-2760), eps from <arch>.attention.layer_norm_rms_epsilon (1972)
    const Tensor* fn = find(g, bp + "ffn_norm.weight");
    const Tensor* pn = find(g, bp + "post_ffw_norm.weight");
    if (fn && fn->type == JX_TYPE_F32 && fn->bytes == D * 4) d->ffn_norm = reinterpret_cast<const float*>(g->base + fn->off);
    if (pn && pn->type == JX_TYPE_F32 && pn->bytes == D * 4)
        d->post_ffw_norm = reinterpret_cast<const float*>(g->base + pn->off);
    d->rms_norm_eps = meta_f32(g, arch + ".attention.layer_norm_rms_epsilon", 1e-5f);
    // the gemma family gates with GELU-tanh (hp_.use_gelu, transformer.cpp:1994-1995)
    const bool gemma = arch == "gemma" || arch == "gemma2" || arch == "gemma3" || arch == "gemma4";
    d->activation = gemma ? JX_ACT_GELU_TANH : JX_ACT_SILU;
    return JX_OK;
}

}  // extern "C"
