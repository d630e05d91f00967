// gguf.cpp -- read-only GGUF (v2 / v3) access for the Q8_0 path: the tensor
// directory, the key/value metadata and the tensor bytes, all in place in a
// private read-only mapping of the file.
//
// Replaces, for the tensors this library consumes, what the reference gets
// from ggml's gguf_init_from_file (src/model_loader.c:101-120): the name
// lookup of vcpm_model_get_tensor(_f32), the F32 copies vcpm_model_ensure_f32
// makes of norms, biases and special tokens (src/model_loader.c:254-352), the
// per-block weight names of fill_minicpm4_weights (src/gen_init.c:34-67,
// src/model_loader.c:609-613) and the LM config keys, defaults and
// sanitisation of vcpm_model_load (src/model_loader.c:52-97,139-219).
//
// The format (ggml's published GGUF layout): "GGUF", u32 version, u64
// tensor count, u64 key/value count; key/value pairs (string key, u32 type,
// value); tensor infos (string name, u32 n_dims, u64 ne[n_dims], u32 ggml
// type, u64 offset); padding to general.alignment (default 32); tensor data,
// each tensor at data_start + offset.  Strings are u64 length + bytes.  All
// little-endian.  Every read is bounds-checked against the file size.
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/vxm_q8.h"

namespace {

enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STR = 8, KV_ARR = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12,
};

struct Kv {
    uint32_t type = 0;
    const uint8_t *val = nullptr;   // scalar bytes / string length field / array header
    std::string str;                // KV_STR value
};

struct Tensor {
    std::string name;
    vxm_gguf_tensor_info info{};
};

// (block elements, block bytes) of the ggml types whose size this reader knows
bool type_size(int32_t t, int64_t *blk, int64_t *bytes) {
    switch (t) {
    case VXM_GGML_F32: *blk = 1; *bytes = 4; return true;
    case VXM_GGML_F16: *blk = 1; *bytes = 2; return true;
    case 2: *blk = 32; *bytes = 18; return true;    // Q4_0
    case 3: *blk = 32; *bytes = 20; return true;    // Q4_1
    case 6: *blk = 32; *bytes = 22; return true;    // Q5_0
    case 7: *blk = 32; *bytes = 24; return true;    // Q5_1
    case VXM_GGML_Q8_0: *blk = 32; *bytes = 34; return true;
    case 9: *blk = 32; *bytes = 36; return true;    // Q8_1
    case 24: *blk = 1; *bytes = 1; return true;     // I8
    case 25: *blk = 1; *bytes = 2; return true;     // I16
    case 26: *blk = 1; *bytes = 4; return true;     // I32
    case 27: *blk = 1; *bytes = 8; return true;     // I64
    case 28: *blk = 1; *bytes = 8; return true;     // F64
    case VXM_GGML_BF16: *blk = 1; *bytes = 2; return true;
    default: return false;
    }
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else {   // subnormal: normalise
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 0x400u)) { mm <<= 1; sh++; }
            u = sign | ((uint32_t)(113 - sh) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

}  // namespace

struct vxm_gguf {
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_start = 0;
    std::unordered_map<std::string, Kv> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> by_name;
    std::string err;
};

namespace {

struct Reader {
    const uint8_t *p;
    size_t size, pos = 0;
    bool ok = true;
    bool need(size_t n) {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <class T> T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    bool str(std::string *out) {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return false;
        if (out) out->assign((const char *)p + pos, n);
        pos += n;
        return true;
    }
};

size_t scalar_bytes(uint32_t t) {
    switch (t) {
    case KV_U8: case KV_I8: case KV_BOOL: return 1;
    case KV_U16: case KV_I16: return 2;
    case KV_U32: case KV_I32: case KV_F32: return 4;
    case KV_U64: case KV_I64: case KV_F64: return 8;
    default: return 0;
    }
}

bool skip_value(Reader &r, uint32_t t, int depth) {
    if (const size_t b = scalar_bytes(t)) {
        if (r.need(b)) r.pos += b;
        return r.ok;
    }
    if (t == KV_STR) return r.str(nullptr);
    if (t == KV_ARR && depth < 4) {
        const uint32_t et = r.get<uint32_t>();
        const uint64_t n = r.get<uint64_t>();
        if (const size_t b = scalar_bytes(et)) {
            if (n > (r.size - r.pos) / b) return r.ok = false;
            r.pos += n * b;
            return r.ok;
        }
        for (uint64_t i = 0; i < n && r.ok; i++) skip_value(r, et, depth + 1);
        return r.ok;
    }
    return r.ok = false;
}

int fail(vxm_gguf *g, char *err, size_t err_size, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (g) g->err = buf;
    if (err && err_size) snprintf(err, err_size, "%s", buf);
    return code;
}

const Kv *find_kv(const vxm_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    return it == g->kv.end() ? nullptr : &it->second;
}

// integer value of a scalar key of any integer / bool type
bool kv_int(const Kv *k, int64_t *out) {
    if (!k) return false;
    const uint8_t *v = k->val;
    switch (k->type) {
    case KV_U8: case KV_BOOL: *out = v[0]; return true;
    case KV_I8: *out = (int8_t)v[0]; return true;
    case KV_U16: { uint16_t x; memcpy(&x, v, 2); *out = x; return true; }
    case KV_I16: { int16_t x; memcpy(&x, v, 2); *out = x; return true; }
    case KV_U32: { uint32_t x; memcpy(&x, v, 4); *out = x; return true; }
    case KV_I32: { int32_t x; memcpy(&x, v, 4); *out = x; return true; }
    case KV_U64: { uint64_t x; memcpy(&x, v, 8); *out = (int64_t)x; return true; }
    case KV_I64: { int64_t x; memcpy(&x, v, 8); *out = x; return true; }
    default: return false;
    }
}

}  // namespace

extern "C" int vxm_gguf_close(vxm_gguf *g) {
    if (!g) return VXM_ERR_INVALID_ARG;
    if (g->map) munmap((void *)g->map, g->size);
    delete g;
    return VXM_OK;
}

extern "C" int vxm_gguf_open(const char *path, vxm_gguf **out, char *err, size_t err_size) {
    if (!out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    if (!path || !path[0]) return fail(nullptr, err, err_size, VXM_ERR_INVALID_ARG, "gguf: empty path");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(nullptr, err, err_size, VXM_ERR_IO, "gguf: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail(nullptr, err, err_size, VXM_ERR_MODEL_FORMAT, "gguf: %s is not a GGUF file (too short)", path);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return fail(nullptr, err, err_size, VXM_ERR_IO, "gguf: cannot map %s", path);
    vxm_gguf *g = new vxm_gguf();
    g->map = (const uint8_t *)m;
    g->size = (size_t)st.st_size;
    auto bad = [&](int code, const char *what) {
        const int rc = fail(g, err, err_size, code, "gguf: %s: %s", path, what);
        vxm_gguf_close(g);
        return rc;
    };
    Reader r{g->map, g->size};
    if (memcmp(g->map, "GGUF", 4) != 0) return bad(VXM_ERR_MODEL_FORMAT, "bad magic");
    r.pos = 4;
    g->version = r.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return bad(VXM_ERR_MODEL_FORMAT, "unsupported GGUF version");
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    if (n_tensors > g->size / 24 || n_kv > g->size / 13) return bad(VXM_ERR_MODEL_FORMAT, "counts exceed the file");
    for (uint64_t i = 0; i < n_kv && r.ok; i++) {
        std::string key;
        if (!r.str(&key)) break;
        Kv k;
        k.type = r.get<uint32_t>();
        k.val = g->map + r.pos;
        if (k.type == KV_STR) {
            if (!r.str(&k.str)) break;
        } else if (!skip_value(r, k.type, 0)) {
            break;
        }
        g->kv[key] = std::move(k);
    }
    if (!r.ok) return bad(VXM_ERR_MODEL_FORMAT, "truncated or malformed key/value section");
    int64_t a = 32;
    if (kv_int(find_kv(g, "general.alignment"), &a) && (a <= 0 || (a & (a - 1)) || a > (1 << 20)))
        return bad(VXM_ERR_MODEL_FORMAT, "general.alignment is not a power of two");
    g->alignment = (uint32_t)a;
    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors && r.ok; i++) {
        Tensor &t = g->tensors[i];
        if (!r.str(&t.name)) break;
        const uint32_t nd = r.get<uint32_t>();
        if (nd < 1 || nd > 4) return bad(VXM_ERR_MODEL_FORMAT, "tensor with more than 4 dimensions");
        vxm_gguf_tensor_info &ti = t.info;
        ti.n_dims = (int32_t)nd;
        int64_t n = 1;
        for (int d = 0; d < 4; d++) {
            ti.ne[d] = 1;
            if ((uint32_t)d < nd) {
                const uint64_t e = r.get<uint64_t>();
                if (e > ((uint64_t)1 << 40) || (e && (uint64_t)n > ((uint64_t)1 << 62) / e))
                    return bad(VXM_ERR_MODEL_FORMAT, "tensor dimension out of range");
                ti.ne[d] = (int64_t)e;
            }
            n *= ti.ne[d];
        }
        ti.type = (int32_t)r.get<uint32_t>();
        ti.offset = r.get<uint64_t>();
        int64_t blk, bytes;
        if (type_size(ti.type, &blk, &bytes)) {
            if (ti.ne[0] % blk) return bad(VXM_ERR_MODEL_FORMAT, "row length not a multiple of the type's block");
            ti.nbytes = (uint64_t)(n / blk * bytes);
        }
        ti.n_elements = n;
    }
    if (!r.ok) return bad(VXM_ERR_MODEL_FORMAT, "truncated or malformed tensor directory");
    g->data_start = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (uint64_t i = 0; i < n_tensors; i++) {
        vxm_gguf_tensor_info &ti = g->tensors[i].info;
        if (ti.offset % g->alignment) return bad(VXM_ERR_MODEL_FORMAT, "tensor data not aligned");
        if (g->data_start > g->size || ti.offset > g->size - g->data_start ||
            ti.nbytes > g->size - g->data_start - ti.offset)
            return bad(VXM_ERR_MODEL_FORMAT, "tensor data beyond the end of the file");
        ti.data = g->map + g->data_start + ti.offset;
        ti.name = g->tensors[i].name.c_str();
        g->by_name[g->tensors[i].name] = (int64_t)i;
    }
    *out = g;
    return VXM_OK;
}

extern "C" const char *vxm_gguf_last_error(const vxm_gguf *g) { return g ? g->err.c_str() : ""; }
extern "C" int32_t vxm_gguf_version(const vxm_gguf *g) { return g ? (int32_t)g->version : -1; }
extern "C" int64_t vxm_gguf_n_tensors(const vxm_gguf *g) { return g ? (int64_t)g->tensors.size() : -1; }

extern "C" int64_t vxm_gguf_find_tensor(const vxm_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : it->second;
}

extern "C" int vxm_gguf_tensor(const vxm_gguf *g, int64_t idx, vxm_gguf_tensor_info *out) {
    if (!g || !out || idx < 0 || idx >= (int64_t)g->tensors.size()) return VXM_ERR_INVALID_ARG;
    *out = g->tensors[idx].info;
    return VXM_OK;
}

extern "C" int32_t vxm_gguf_get_i32(const vxm_gguf *g, const char *key, int32_t def) {
    int64_t v;
    return kv_int(find_kv(g, key), &v) ? (int32_t)v : def;
}

extern "C" float vxm_gguf_get_f32(const vxm_gguf *g, const char *key, float def) {
    const Kv *k = find_kv(g, key);
    if (!k) return def;
    if (k->type == KV_F32) {
        float f;
        memcpy(&f, k->val, 4);
        return f;
    }
    if (k->type == KV_F64) {
        double d;
        memcpy(&d, k->val, 8);
        return (float)d;
    }
    int64_t v;
    return kv_int(k, &v) ? (float)v : def;
}

extern "C" const char *vxm_gguf_get_str(const vxm_gguf *g, const char *key, const char *def) {
    const Kv *k = find_kv(g, key);
    return (k && k->type == KV_STR) ? k->str.c_str() : def;
}

extern "C" int vxm_gguf_tensor_f32(const vxm_gguf *g, int64_t idx, float *out, int64_t n) {
    if (!g || !out || idx < 0 || idx >= (int64_t)g->tensors.size()) return VXM_ERR_INVALID_ARG;
    const vxm_gguf_tensor_info &t = g->tensors[idx].info;
    if (n != t.n_elements) return VXM_ERR_INVALID_ARG;
    const uint8_t *s = (const uint8_t *)t.data;
    switch (t.type) {
    case VXM_GGML_F32:
        memcpy(out, s, (size_t)n * 4);
        return VXM_OK;
    case VXM_GGML_F16:
        for (int64_t i = 0; i < n; i++) {
            uint16_t h;
            memcpy(&h, s + 2 * i, 2);
            out[i] = half_to_float(h);
        }
        return VXM_OK;
    case VXM_GGML_BF16:
        for (int64_t i = 0; i < n; i++) {
            uint16_t h;
            memcpy(&h, s + 2 * i, 2);
            const uint32_t u = (uint32_t)h << 16;
            memcpy(out + i, &u, 4);
        }
        return VXM_OK;
    case VXM_GGML_Q8_0:   // value = (float)qs * fp32(d), block by block
        for (int64_t b = 0; b < n / 32; b++) {
            uint16_t h;
            memcpy(&h, s + 34 * b, 2);
            const float d = half_to_float(h);
            const int8_t *q = (const int8_t *)(s + 34 * b + 2);
            for (int j = 0; j < 32; j++) out[32 * b + j] = (float)q[j] * d;
        }
        return VXM_OK;
    default:
        return VXM_ERR_NOT_IMPLEMENTED;
    }
}

extern "C" int vxm_gguf_layer_q8_0(vxm_gguf *g, const char *prefix, int32_t layer, int64_t hidden, int64_t q_dim,
                                   int64_t kv_dim, int64_t ffn, float *norms, vxm_layer_weights_q8_0 *out) {
    if (!g || !prefix || !out || !norms || layer < 0 || hidden <= 0 || q_dim <= 0 || kv_dim <= 0 || ffn <= 0)
        return VXM_ERR_INVALID_ARG;
    // ne = [K, N] of q, k, v, o, gate, up, down: the sizes the upload reads
    // (ggml_mul_mat refuses a weight whose K differs from the activation's)
    const int64_t want[7][2] = {{hidden, q_dim}, {hidden, kv_dim}, {hidden, kv_dim}, {q_dim, hidden},
                                {hidden, ffn},   {hidden, ffn},    {ffn, hidden}};
    static const char *const kSuffix[9] = {
        "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.o_proj.weight", "mlp.gate_proj.weight",    "mlp.up_proj.weight",
        "mlp.down_proj.weight",    "input_layernorm.weight",  "post_attention_layernorm.weight"};
    const void *proj[7];
    for (int s = 0; s < 9; s++) {
        char name[256];
        snprintf(name, sizeof(name), "%s.%d.%s", prefix, layer, kSuffix[s]);
        const int64_t idx = vxm_gguf_find_tensor(g, name);
        if (idx < 0) return fail(g, nullptr, 0, VXM_ERR_MODEL_FORMAT, "gguf: tensor %s is missing", name);
        const vxm_gguf_tensor_info &t = g->tensors[idx].info;
        if (s < 7) {
            if (t.type != VXM_GGML_Q8_0 || t.n_dims != 2)
                return fail(g, nullptr, 0, VXM_ERR_NOT_IMPLEMENTED, "gguf: %s is not a 2-D Q8_0 tensor", name);
            if (t.ne[0] != want[s][0] || t.ne[1] != want[s][1])
                return fail(g, nullptr, 0, VXM_ERR_MODEL_FORMAT, "gguf: %s has ne = [%lld, %lld], expected [%lld, %lld]",
                            name, (long long)t.ne[0], (long long)t.ne[1], (long long)want[s][0],
                            (long long)want[s][1]);
            proj[s] = t.data;
        } else {
            if (t.n_elements != hidden)
                return fail(g, nullptr, 0, VXM_ERR_MODEL_FORMAT, "gguf: %s has %lld elements, expected %lld", name,
                            (long long)t.n_elements, (long long)hidden);
            const int rc = vxm_gguf_tensor_f32(g, idx, norms + (s - 7) * hidden, hidden);
            if (rc) return fail(g, nullptr, 0, rc, "gguf: %s has an unsupported type %d", name, t.type);
        }
    }
    *out = vxm_layer_weights_q8_0{proj[0], proj[1], proj[2], proj[3], proj[4], proj[5], proj[6],
                                  norms, norms + hidden};
    return VXM_OK;
}

extern "C" int vxm_gguf_minicpm4_config(vxm_gguf *g, int32_t residual, vxm_minicpm4_config *cfg) {
    if (!g || !cfg) return VXM_ERR_INVALID_ARG;
    const char *arch = vxm_gguf_get_str(g, "general.architecture", "");
    if (strcmp(arch, "voxcpm2") != 0)
        return fail(g, nullptr, 0, VXM_ERR_UNSUPPORTED_ARCH, "gguf: architecture '%s', expected 'voxcpm2'", arch);
    // defaults of vcpm_model_config_default (src/model_loader.c:52-97)
    const int32_t hidden = vxm_gguf_get_i32(g, "voxcpm.hidden_size", 2048);
    vxm_minicpm4_config c{};
    c.intermediate_size = vxm_gguf_get_i32(g, "voxcpm.intermediate_size", 8192);
    c.head_dim = vxm_gguf_get_i32(g, "voxcpm.head_dim", 128);
    c.rms_norm_eps = vxm_gguf_get_f32(g, "voxcpm.rms_norm_eps", 1.0e-6f);
    // a converter bug stored eps as 0; the reference substitutes 1e-5 (src/model_loader.c:203-213)
    if (c.rms_norm_eps < 1.0e-7f) c.rms_norm_eps = 1.0e-5f;
    const bool mup = vxm_gguf_get_i32(g, "voxcpm.use_mup", 0) != 0;
    if (!residual) {
        c.hidden_size = hidden;
        c.n_layers = vxm_gguf_get_i32(g, "voxcpm.num_hidden_layers", 24);
        c.n_heads = vxm_gguf_get_i32(g, "voxcpm.num_attention_heads", 16);
        c.n_kv_heads = vxm_gguf_get_i32(g, "voxcpm.num_kv_heads", 4);
        c.rope_theta = vxm_gguf_get_i32(g, "voxcpm.rope_theta", 1000000);
        c.no_rope = 0;
        c.scale_depth = mup ? vxm_gguf_get_f32(g, "voxcpm.scale_depth", 0.0f) : 0.0f;
    } else {   // the RALM: res_* keys, no rope (src/gen_prompt.c:147-178, src/ralm.c:15-29)
        c.hidden_size = vxm_gguf_get_i32(g, "voxcpm.res_hidden_size", 2048);
        c.n_layers = vxm_gguf_get_i32(g, "voxcpm.res_num_layers", 8);
        c.n_heads = vxm_gguf_get_i32(g, "voxcpm.res_num_heads", 16);
        c.n_kv_heads = vxm_gguf_get_i32(g, "voxcpm.res_num_kv_heads", 4);
        c.rope_theta = 0;
        c.no_rope = 1;
        c.scale_depth = mup ? vxm_gguf_get_f32(g, "voxcpm.res_scale_depth", 0.0f) : 0.0f;
    }
    c.rope_freq_factors = nullptr;
    *cfg = c;
    return VXM_OK;
}
