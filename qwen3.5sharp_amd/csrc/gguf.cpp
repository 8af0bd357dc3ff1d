// GGUF reader and the mixers' F32 weight upload: GgufFile
// (src/Qwen35Sharp.Gguf/GgufFile.cs:27-170, the published GGUF v2/v3 layout)
// and the F32 branch of Qwen35Model.LoadWeights (Qwen35Model.cs:463-474) for
// the tensors the token mixers read.  The file is memory-mapped read-only;
// tensor data pointers point into the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cctype>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/q35mix.h"

int q35_set_error(int code, const char* msg);
int q35_check_mixer_dims(const q35m_ctx* ctx, int num_layers, const unsigned char* is_recurrent, int conv_dim,
                         int n_v_heads, int v_head_dim, int head_dim);

namespace {

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return q35_set_error(code, buf);
}

}  // namespace

namespace {

enum : uint32_t { kMagic = 0x46554747u, kDefaultAlignment = 32 };
// GGUF metadata value types (GgufValueType).
enum ValueType { U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 };

struct Value {
    int type = -1;
    int64_t i = 0;      // integer and bool types
    double f = 0.0;     // F32 / F64
    std::string s;      // STRING
};

struct Tensor {
    int type = 0;
    int n_dims = 0;
    int64_t dims[4] = {0, 0, 0, 0};
    uint64_t offset = 0;
};

// Bytes of n elements of a ggml tensor type (block formats by their block
// size); 0 for a type this reader does not size.
uint64_t type_bytes(int type, uint64_t n) {
    switch (type) {
        case 0: return 4 * n;                      // F32
        case 1: return 2 * n;                      // F16
        case 8: return n % 32 ? 0 : n / 32 * 34;   // Q8_0
        case 12: return n % 256 ? 0 : n / 256 * 144;  // Q4_K
        case 13: return n % 256 ? 0 : n / 256 * 176;  // Q5_K
        case 14: return n % 256 ? 0 : n / 256 * 210;  // Q6_K
        case 15: return n % 256 ? 0 : n / 256 * 292;  // Q8_K
        case 23: return n % 256 ? 0 : n / 256 * 136;  // IQ4_XS
        case 40: return n % 512 ? 0 : n / 512 * 130;  // Q2_0C
        case 43: return n % 256 ? 0 : n / 256 * 42;   // STQ1_0
        default: return 0;
    }
}

struct Cursor {
    const unsigned char* p;
    uint64_t len, pos = 0;
    bool ok = true;
    bool take(void* dst, uint64_t n) {
        if (!ok || n > len - pos) return ok = false;
        std::memcpy(dst, p + pos, n);
        pos += n;
        return true;
    }
    template <class T> T get() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > len - pos) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char*>(p + pos), n);
        pos += n;
        return s;
    }
};

bool read_scalar(Cursor& c, int type, Value& v) {
    v.type = type;
    switch (type) {
        case U8: v.i = c.get<uint8_t>(); break;
        case I8: v.i = c.get<int8_t>(); break;
        case U16: v.i = c.get<uint16_t>(); break;
        case I16: v.i = c.get<int16_t>(); break;
        case U32: v.i = c.get<uint32_t>(); break;
        case I32: v.i = c.get<int32_t>(); break;
        case F32: v.f = c.get<float>(); break;
        case BOOL: v.i = c.get<uint8_t>() != 0; break;
        case STRING: v.s = c.str(); break;
        case U64: v.i = (int64_t)c.get<uint64_t>(); break;
        case I64: v.i = c.get<int64_t>(); break;
        case F64: v.f = c.get<double>(); break;
        default: return false;
    }
    return c.ok;
}

}  // namespace

struct q35m_gguf {
    void* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    const unsigned char* data = nullptr;   // start of the tensor data section
    std::map<std::string, Value> kv;
    std::map<std::string, Tensor> tensors;
};

// GgufFile.CanonicalTensorType (src/Qwen35Sharp.Gguf/GgufFile.cs:171-181):
// files written before STQ1_0 got its type number (43) store it as raw type
// 42, which is now plain Q2_0; only a file with general.file_type 41 whose
// general.name contains "Stride16" (any case) is read as STQ1_0.
static int canonical_type(const q35m_gguf* g, int raw) {
    if (raw != 42) return raw;
    auto ft = g->kv.find("general.file_type");
    auto nm = g->kv.find("general.name");
    if (ft == g->kv.end() || nm == g->kv.end() || nm->second.type != STRING) return raw;
    const int t = ft->second.type;
    if (t == F32 || t == F64 || t == STRING || t == ARRAY || ft->second.i != 41) return raw;
    std::string name = nm->second.s;
    for (char& ch : name) ch = (char)std::tolower((unsigned char)ch);
    return name.find("stride16") != std::string::npos ? 43 : raw;
}

static int parse(q35m_gguf* g) {
    Cursor c{static_cast<const unsigned char*>(g->map), g->size};
    if (c.get<uint32_t>() != kMagic || !c.ok) return fail(Q35M_ERR_INVALID, "not a GGUF file (magic)");
    g->version = c.get<uint32_t>();
    if (g->version < 2 || g->version > 3)
        return fail(Q35M_ERR_UNSUPPORTED, "GGUF version %u is not supported (need 2 or 3)", g->version);
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > INT32_MAX || n_kv > INT32_MAX)
        return fail(Q35M_ERR_INVALID, "GGUF header counts are implausible");
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = c.str();
        if (!c.ok || key.empty()) return fail(Q35M_ERR_INVALID, "GGUF key %llu unreadable", (unsigned long long)i);
        const int type = (int)c.get<uint32_t>();
        Value v;
        if (type == ARRAY) {
            // arrays are skipped element by element (no nested arrays)
            const int et = (int)c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (et == ARRAY || !c.ok) return fail(Q35M_ERR_INVALID, "GGUF array '%s' unreadable", key.c_str());
            for (uint64_t k = 0; k < n; k++) {
                Value e;
                if (!read_scalar(c, et, e)) return fail(Q35M_ERR_INVALID, "GGUF array '%s' unreadable", key.c_str());
            }
            v.type = ARRAY;
            v.i = (int64_t)n;
        } else if (!read_scalar(c, type, v)) {
            return fail(Q35M_ERR_INVALID, "GGUF value '%s' unreadable (type %d)", key.c_str(), type);
        }
        g->kv[key] = v;
    }
    uint64_t alignment = kDefaultAlignment;
    auto a = g->kv.find("general.alignment");
    if (a != g->kv.end()) {
        const int t = a->second.type;
        if (t == F32 || t == F64 || t == STRING || t == ARRAY || t == BOOL || a->second.i < 0)
            return fail(Q35M_ERR_INVALID, "GGUF general.alignment is not an unsigned integer");
        alignment = (uint64_t)a->second.i;
    }
    if (alignment == 0 || (alignment & (alignment - 1)))
        return fail(Q35M_ERR_INVALID, "GGUF alignment %llu is not a power of two", (unsigned long long)alignment);
    for (uint64_t i = 0; i < n_tensors; i++) {
        std::string name = c.str();
        Tensor t;
        t.n_dims = (int)c.get<uint32_t>();
        if (!c.ok || t.n_dims < 1 || t.n_dims > 4)
            return fail(Q35M_ERR_INVALID, "tensor '%s' has an invalid dim count", name.c_str());
        for (int d = 0; d < t.n_dims; d++) {
            t.dims[d] = c.get<int64_t>();
            if (t.dims[d] < 0) return fail(Q35M_ERR_INVALID, "tensor '%s' dim %d is negative", name.c_str(), d);
        }
        t.type = canonical_type(g, c.get<int32_t>());
        t.offset = c.get<uint64_t>();
        if (!c.ok) return fail(Q35M_ERR_INVALID, "tensor info %llu unreadable", (unsigned long long)i);
        g->tensors[name] = t;
    }
    uint64_t pos = c.pos;
    if (n_tensors > 0) pos = (pos + alignment - 1) & ~(alignment - 1);
    if (pos > g->size) return fail(Q35M_ERR_INVALID, "GGUF data section starts past the end of the file");
    g->data = static_cast<const unsigned char*>(g->map) + pos;
    return Q35M_OK;
}

int q35m_gguf_open(const char* path, q35m_gguf** out) {
    if (!path || !out) return fail(Q35M_ERR_INVALID, "null pointer");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(Q35M_ERR_INVALID, "cannot open '%s'", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail(Q35M_ERR_INVALID, "'%s' is too short for a GGUF header", path);
    }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return fail(Q35M_ERR_INVALID, "cannot map '%s'", path);
    q35m_gguf* g = new q35m_gguf;
    g->map = m;
    g->size = (size_t)st.st_size;
    const int r = parse(g);
    if (r) {
        q35m_gguf_close(g);
        return r;
    }
    *out = g;
    return Q35M_OK;
}

int q35m_gguf_close(q35m_gguf* g) {
    if (!g) return fail(Q35M_ERR_INVALID, "null GGUF handle");
    if (g->map) munmap(g->map, g->size);
    delete g;
    return Q35M_OK;
}

int q35m_gguf_tensor(const q35m_gguf* g, const char* name, int* type, int64_t dims[4], int* n_dims,
                     const void** data, size_t* bytes) {
    if (!g || !name) return fail(Q35M_ERR_INVALID, "null pointer");
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) return fail(Q35M_ERR_RANGE, "no tensor '%s'", name);
    const Tensor& t = it->second;
    // Element count and byte size with overflow checks: a header can claim
    // dims whose product wraps a 64-bit count.
    uint64_t n = 1;
    for (int d = 0; d < t.n_dims; d++) {
        const uint64_t dd = (uint64_t)t.dims[d];
        if (dd != 0 && n > UINT64_MAX / dd)
            return fail(Q35M_ERR_INVALID, "tensor '%s' has an element count that overflows", name);
        n *= dd;
    }
    if (n > UINT64_MAX / 4) return fail(Q35M_ERR_INVALID, "tensor '%s' is too large", name);
    const uint64_t nb = type_bytes(t.type, n);
    const uint64_t avail = g->size - (uint64_t)(g->data - static_cast<const unsigned char*>(g->map));
    // The offset is checked for every type, the extent for the sized ones.
    if (t.offset > avail || (nb && nb > avail - t.offset))
        return fail(Q35M_ERR_INVALID, "tensor '%s' runs past the end of the file", name);
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = d < t.n_dims ? t.dims[d] : 1;
    if (data) *data = g->data + t.offset;
    if (bytes) *bytes = (size_t)nb;
    return Q35M_OK;
}

int q35m_gguf_int(const q35m_gguf* g, const char* key, int64_t* value) {
    if (!g || !key || !value) return fail(Q35M_ERR_INVALID, "null pointer");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(Q35M_ERR_RANGE, "no key '%s'", key);
    const int t = it->second.type;
    if (t == F32 || t == F64 || t == STRING || t == ARRAY)
        return fail(Q35M_ERR_INVALID, "key '%s' is not an integer", key);
    *value = it->second.i;
    return Q35M_OK;
}

int q35m_gguf_float(const q35m_gguf* g, const char* key, double* value) {
    if (!g || !key || !value) return fail(Q35M_ERR_INVALID, "null pointer");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(Q35M_ERR_RANGE, "no key '%s'", key);
    if (it->second.type != F32 && it->second.type != F64)
        return fail(Q35M_ERR_INVALID, "key '%s' is not a float", key);
    *value = it->second.f;
    return Q35M_OK;
}

int q35m_gguf_string(const q35m_gguf* g, const char* key, const char** value) {
    if (!g || !key || !value) return fail(Q35M_ERR_INVALID, "null pointer");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(Q35M_ERR_RANGE, "no key '%s'", key);
    if (it->second.type != STRING) return fail(Q35M_ERR_INVALID, "key '%s' is not a string", key);
    *value = it->second.s.c_str();
    return Q35M_OK;
}

// One F32 tensor of exactly n elements, or an error naming it.
static int f32_tensor(const q35m_gguf* g, const std::string& name, uint64_t n, const float** out) {
    int type = 0;
    int64_t dims[4];
    int nd = 0;
    const void* p = nullptr;
    size_t bytes = 0;
    int r = q35m_gguf_tensor(g, name.c_str(), &type, dims, &nd, &p, &bytes);
    if (r) return r;
    if (type != 0) return fail(Q35M_ERR_UNSUPPORTED, "tensor '%s' must be F32 (type %d)", name.c_str(), type);
    if (bytes != 4 * n)
        return fail(Q35M_ERR_INVALID, "tensor '%s' holds %zu bytes, %llu expected", name.c_str(), bytes,
                    (unsigned long long)(4 * n));
    *out = static_cast<const float*>(p);
    return Q35M_OK;
}

int q35m_load_mixer_weights(q35m_ctx* ctx, const q35m_gguf* g, int num_layers, const unsigned char* is_recurrent,
                            int conv_dim, int n_v_heads, int v_head_dim, int head_dim) {
    if (!ctx || !g || !is_recurrent) return fail(Q35M_ERR_INVALID, "null pointer");
    // The setters copy context-sized byte counts from the mapped tensors, so
    // the sizes the tensors are checked against must be the context's.
    int r = q35_check_mixer_dims(ctx, num_layers, is_recurrent, conv_dim, n_v_heads, v_head_dim, head_dim);
    if (r) return r;
    for (int l = 0; l < num_layers; l++) {
        const std::string b = "blk." + std::to_string(l) + ".";
        if (is_recurrent[l]) {
            const float *cw, *sa, *dt, *sn;
            if ((r = f32_tensor(g, b + "ssm_conv1d.weight", 4ull * conv_dim, &cw))) return r;
            if ((r = f32_tensor(g, b + "ssm_a", (uint64_t)n_v_heads, &sa))) return r;
            if ((r = f32_tensor(g, b + "ssm_dt.bias", (uint64_t)n_v_heads, &dt))) return r;
            if ((r = f32_tensor(g, b + "ssm_norm.weight", (uint64_t)v_head_dim, &sn))) return r;
            if ((r = q35m_set_deltanet_weights(ctx, l, cw, sa, dt, sn))) return r;
        } else {
            const float *qn, *kn;
            if ((r = f32_tensor(g, b + "attn_q_norm.weight", (uint64_t)head_dim, &qn))) return r;
            if ((r = f32_tensor(g, b + "attn_k_norm.weight", (uint64_t)head_dim, &kn))) return r;
            if ((r = q35m_set_attn_weights(ctx, l, qn, kn))) return r;
        }
    }
    return Q35M_OK;
}
