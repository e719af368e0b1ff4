// gguf.cpp -- GGUF v3 reader (memory-mapped) and the uploads of its Q6_K
// tensors to the device: the input format in front of the quantized-matmul
// path (crates/llamd-gguf/src/lib.rs, the upload side of
// crates/llamd-runtime/src/device.rs:224-256).
//
// Layout (ggml's gguf.h):
//   "GGUF" | version u32 | n_tensors u64 | n_kv u64
//   n_kv     x  key(string) type(u32) value
//   n_tensors x name(string) n_dims(u32) dims[n_dims](u64) type(u32) offset(u64)
//   padding to general.alignment (default 32), then the tensor data.
// Strings are a u64 length and unterminated bytes. Everything little-endian.
//
// Every count and length in the file is untrusted. The rules follow the
// reference parser (lib.rs:141-236, 293-375): header counts larger than the
// file are refused before anything is reserved; array lengths are checked
// against the bytes that remain; nested arrays, unknown value types, more
// than 4 dims and a non-power-of-two alignment are refused; a tensor's bytes
// must lie inside the file and its element count must fill whole blocks of
// its type (lib.rs:256-278). Metadata keys are unique (a later duplicate
// replaces an earlier one, as in the reference's BTreeMap) and listed in
// byte order of the key.
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "../../../include/llamd_hip.h"
#include "../errors.hpp"

using llamd::set_error;

namespace {

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12,
};

// bytes of a fixed-size value type; 0 for string / array / unknown
size_t scalar_size(uint32_t t) {
    switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
    }
}

struct Kv {
    std::string key;
    uint32_t type = 0, arr_type = 0;
    uint64_t arr_len = 0;
    size_t pos = 0;                // scalar / string: where the value starts
    std::vector<size_t> elems;     // array: where each element starts
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0, type = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
};

struct Gguf {
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<Kv> kvs;           // sorted by key
    std::vector<Tensor> tensors;   // file order
    ~Gguf() {
        if (map) munmap((void *)map, size);
    }
};

struct Reader {
    const uint8_t *b;
    size_t n, p = 0;
    bool take(size_t k, const uint8_t **out) {
        if (k > n - p) {
            set_error("gguf: truncated: wanted %zu bytes at %zu, file has %zu", k, p, n);
            return false;
        }
        *out = b + p;
        p += k;
        return true;
    }
    bool u32(uint32_t *v) {
        const uint8_t *s;
        if (!take(4, &s)) return false;
        memcpy(v, s, 4);
        return true;
    }
    bool u64(uint64_t *v) {
        const uint8_t *s;
        if (!take(8, &s)) return false;
        memcpy(v, s, 8);
        return true;
    }
    bool string(std::string *out) {
        uint64_t len;
        if (!u64(&len)) return false;
        const uint8_t *s;
        if (len > n - p) {
            set_error("gguf: truncated: string of %llu bytes at %zu, file has %zu",
                      (unsigned long long)len, p, n);
            return false;
        }
        if (!take((size_t)len, &s)) return false;
        if (out) out->assign((const char *)s, (size_t)len);
        return true;
    }
    // skips one value of type t, recording where it starts
    bool value(uint32_t t, Kv *kv) {
        if (kv) kv->pos = p;
        if (const size_t sz = scalar_size(t)) {
            const uint8_t *s;
            return take(sz, &s);
        }
        if (t == T_STRING) return string(nullptr);
        if (t == T_ARRAY) {
            uint32_t inner;
            uint64_t cnt;
            if (!u32(&inner) || !u64(&cnt)) return false;
            if (inner == T_ARRAY) return set_error("gguf array: nested arrays are unsupported") == 0;
            const uint64_t remaining = n - p;
            if (cnt > remaining)
                return set_error("gguf array: %llu elements declared, only %llu bytes remain",
                                 (unsigned long long)cnt, (unsigned long long)remaining) == 0;
            if (kv) {
                kv->arr_type = inner;
                kv->arr_len = cnt;
                kv->elems.reserve((size_t)(cnt < 65536 ? cnt : 65536));  // cnt is untrusted
            }
            for (uint64_t i = 0; i < cnt; ++i) {
                if (kv) kv->elems.push_back(p);
                if (!value(inner, nullptr)) return false;
            }
            return true;
        }
        return set_error("gguf value: unknown type %u", t) == 0;
    }
};

bool parse(Gguf &g) {
    Reader r{g.map, g.size};
    const uint8_t *magic;
    if (!r.take(4, &magic)) return false;
    if (memcmp(magic, "GGUF", 4) != 0)
        return set_error("gguf header: magic is %02x %02x %02x %02x, expected \"GGUF\"", magic[0],
                         magic[1], magic[2], magic[3]) == 0;
    if (!r.u32(&g.version)) return false;
    if (g.version != 3)
        return set_error("gguf version: version %u; this parser implements 3", g.version) == 0;
    uint64_t n_tensors, n_kv;
    if (!r.u64(&n_tensors) || !r.u64(&n_kv)) return false;
    if (n_tensors > g.size || n_kv > g.size)
        return set_error("gguf header: %llu kv / %llu tensors exceeds the %zu-byte file",
                         (unsigned long long)n_kv, (unsigned long long)n_tensors, g.size) == 0;
    std::map<std::string, Kv> kv;
    for (uint64_t i = 0; i < n_kv; ++i) {
        Kv e;
        if (!r.string(&e.key) || !r.u32(&e.type)) return false;
        if (!r.value(e.type, &e)) return false;
        kv[e.key] = std::move(e);
    }
    g.kvs.reserve(kv.size());
    for (auto &it : kv) g.kvs.push_back(std::move(it.second));
    g.tensors.reserve((size_t)(n_tensors < 4096 ? n_tensors : 4096));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        if (!r.string(&t.name) || !r.u32(&t.n_dims)) return false;
        if (t.n_dims > 4)
            return set_error("tensor info: %s claims %u dimensions; ggml allows at most 4",
                             t.name.c_str(), t.n_dims) == 0;
        for (uint32_t d = 0; d < t.n_dims; ++d)
            if (!r.u64(&t.dims[d])) return false;
        if (!r.u32(&t.type) || !r.u64(&t.offset)) return false;
        g.tensors.push_back(std::move(t));
    }
    g.data_offset = r.p;  // the header's end; open() aligns it
    return true;
}

const Kv *find_kv(const Gguf &g, const char *key) {
    size_t lo = 0, hi = g.kvs.size();
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        const int c = g.kvs[mid].key.compare(key);
        if (c == 0) return &g.kvs[mid];
        if (c < 0) lo = mid + 1; else hi = mid;
    }
    return nullptr;
}

uint64_t read_bits(const uint8_t *p, size_t sz) {
    uint64_t v = 0;
    memcpy(&v, p, sz);
    return v;
}

// Value::as_u64 (lib.rs:55-67): unsigned types, and signed ones when >= 0
bool as_u64(const Gguf &g, const Kv &e, uint64_t *out) {
    const size_t sz = scalar_size(e.type);
    if (!sz || e.type == T_F32 || e.type == T_F64 || e.type == T_BOOL) return false;
    const uint64_t b = read_bits(g.map + e.pos, sz);
    int64_t s;
    switch (e.type) {
    case T_U8: case T_U16: case T_U32: case T_U64: *out = b; return true;
    case T_I8: s = (int8_t)b; break;
    case T_I16: s = (int16_t)b; break;
    case T_I32: s = (int32_t)b; break;
    default: s = (int64_t)b; break;
    }
    if (s < 0) return false;
    *out = (uint64_t)s;
    return true;
}

// QuantType::from_ggml + bytes_for (crates/llamd-quant/src/lib.rs:55-101)
bool type_bytes(uint32_t type, uint64_t n, const char *name, uint64_t *bytes) {
    uint64_t be, bb;
    switch (type) {
    case 0: be = 1; bb = 4; break;      // F32
    case 1: be = 1; bb = 2; break;      // F16
    case 8: be = 32; bb = 34; break;    // Q8_0
    case 14: be = 256; bb = 210; break; // Q6_K
    default:
        return set_error("ggml quantization type: type %u is not implemented yet (tensor %s)", type,
                         name) == 0;
    }
    if (n % be)
        return set_error("tensor length: %llu elements is not a multiple of the %llu-element block "
                         "(tensor %s)", (unsigned long long)n, (unsigned long long)be, name) == 0;
    *bytes = n / be * bb;
    return true;
}

bool elems_of(const Tensor &t, uint64_t *n) {
    uint64_t e = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
        if (t.dims[d] && e > UINT64_MAX / t.dims[d])
            return set_error("tensor: %s has too many elements", t.name.c_str()) == 0;
        e *= t.dims[d];
    }
    *n = e;
    return true;
}

// Gguf::tensor_data (lib.rs:256-278)
const uint8_t *tensor_bytes(const Gguf &g, const Tensor &t, uint64_t *nbytes) {
    uint64_t n, len;
    if (!elems_of(t, &n) || !type_bytes(t.type, n, t.name.c_str(), &len)) return nullptr;
    const uint64_t start = g.data_offset + t.offset;
    if (start < g.data_offset || start > g.size || len > g.size - start) {
        set_error("tensor: %s spans %llu..%llu, past the %zu-byte file", t.name.c_str(),
                  (unsigned long long)start, (unsigned long long)(start + len), g.size);
        return nullptr;
    }
    *nbytes = len;
    return g.map + start;
}

const Tensor *find_tensor(const Gguf &g, const char *name) {
    for (const Tensor &t : g.tensors)
        if (t.name == name) return &t;
    return nullptr;
}

bool copy_out(const std::string &s, char *buf, size_t cap) {
    if (!buf) return true;
    if (s.size() + 1 > cap) return set_error("gguf: a %zu-byte name does not fit the buffer", s.size()) == 0;
    memcpy(buf, s.data(), s.size());
    buf[s.size()] = '\0';
    return true;
}

}  // namespace

extern "C" {

void *llamd_gguf_open(const char *path) {
    if (!path) { set_error("gguf: null path"); return nullptr; }
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) { set_error("gguf: cannot open %s", path); return nullptr; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        set_error("gguf: %s is empty or unreadable", path);
        return nullptr;
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) { set_error("gguf: cannot map %s", path); return nullptr; }
    Gguf *g = new Gguf();
    g->map = (const uint8_t *)m;
    g->size = (size_t)st.st_size;
    if (!parse(*g)) { delete g; return nullptr; }
    // general.alignment (lib.rs:207-216), then the data section (lib.rs:218-229)
    if (const Kv *a = find_kv(*g, "general.alignment")) {
        uint64_t v;
        if (as_u64(*g, *a, &v)) g->alignment = v;
    }
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1))) {
        set_error("general.alignment: %llu is not a power of two", (unsigned long long)g->alignment);
        delete g;
        return nullptr;
    }
    const uint64_t end = g->data_offset;
    g->data_offset = (end + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_offset < end || g->data_offset > g->size) {
        set_error("gguf layout: data section starts at %llu, past the %zu-byte file",
                  (unsigned long long)g->data_offset, g->size);
        delete g;
        return nullptr;
    }
    return g;
}

void llamd_gguf_close(void *h) { delete (Gguf *)h; }

int llamd_gguf_header(void *h, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv,
                      uint64_t *alignment, uint64_t *data_offset, uint64_t *file_size) {
    const Gguf *g = (const Gguf *)h;
    if (!g) return set_error("gguf: null handle");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kvs.size();
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (file_size) *file_size = g->size;
    return 0;
}

int llamd_gguf_kv(void *h, uint64_t i, char *key, size_t cap, uint32_t *type, uint32_t *arr_type,
                  uint64_t *arr_len) {
    const Gguf *g = (const Gguf *)h;
    if (!g) return set_error("gguf: null handle");
    if (i >= g->kvs.size()) return set_error("gguf: metadata index %llu of %zu", (unsigned long long)i, g->kvs.size());
    const Kv &e = g->kvs[i];
    if (!copy_out(e.key, key, cap)) return -1;
    if (type) *type = e.type;
    if (arr_type) *arr_type = e.type == T_ARRAY ? e.arr_type : 0;
    if (arr_len) *arr_len = e.type == T_ARRAY ? e.arr_len : 0;
    return 0;
}

int64_t llamd_gguf_find_kv(void *h, const char *key) {
    const Gguf *g = (const Gguf *)h;
    if (!g || !key) return set_error("gguf: null argument");
    const Kv *e = find_kv(*g, key);
    return e ? (int64_t)(e - g->kvs.data()) : -1;
}

// a fixed-size value: the scalar itself (elem ignored) or element elem of an array
int llamd_gguf_kv_bits(void *h, uint64_t i, uint64_t elem, uint64_t *bits) {
    const Gguf *g = (const Gguf *)h;
    if (!g || !bits) return set_error("gguf: null argument");
    if (i >= g->kvs.size()) return set_error("gguf: metadata index %llu of %zu", (unsigned long long)i, g->kvs.size());
    const Kv &e = g->kvs[i];
    const uint32_t t = e.type == T_ARRAY ? e.arr_type : e.type;
    const size_t sz = scalar_size(t);
    if (!sz) return set_error("gguf: %s is not a number or bool", e.key.c_str());
    size_t pos = e.pos;
    if (e.type == T_ARRAY) {
        if (elem >= e.arr_len) return set_error("gguf: %s has %llu elements", e.key.c_str(), (unsigned long long)e.arr_len);
        pos = e.elems[(size_t)elem];
    }
    *bits = read_bits(g->map + pos, sz);
    return 0;
}

// a string: the scalar (elem ignored) or element elem of a string array.
// *len receives the byte length; buf (optional) receives the bytes + NUL.
int llamd_gguf_kv_str(void *h, uint64_t i, uint64_t elem, char *buf, size_t cap, uint64_t *len) {
    const Gguf *g = (const Gguf *)h;
    if (!g) return set_error("gguf: null handle");
    if (i >= g->kvs.size()) return set_error("gguf: metadata index %llu of %zu", (unsigned long long)i, g->kvs.size());
    const Kv &e = g->kvs[i];
    size_t pos = e.pos;
    if (e.type == T_ARRAY) {
        if (e.arr_type != T_STRING) return set_error("gguf: %s is not a string array", e.key.c_str());
        if (elem >= e.arr_len) return set_error("gguf: %s has %llu elements", e.key.c_str(), (unsigned long long)e.arr_len);
        pos = e.elems[(size_t)elem];
    } else if (e.type != T_STRING) {
        return set_error("gguf: %s is not a string", e.key.c_str());
    }
    const uint64_t n = read_bits(g->map + pos, 8);
    if (len) *len = n;
    if (buf) {
        if (n + 1 > cap) return set_error("gguf: a %llu-byte string does not fit the buffer", (unsigned long long)n);
        memcpy(buf, g->map + pos + 8, (size_t)n);
        buf[n] = '\0';
    }
    return 0;
}

// Value::as_u64 of a key (lib.rs:55-67); -1 if absent or not an integer >= 0
int llamd_gguf_get_u64(void *h, const char *key, uint64_t *out) {
    const Gguf *g = (const Gguf *)h;
    if (!g || !key || !out) return set_error("gguf: null argument");
    const Kv *e = find_kv(*g, key);
    if (!e) return set_error("gguf: %s is absent", key);
    if (!as_u64(*g, *e, out)) return set_error("gguf: %s is not a non-negative integer", key);
    return 0;
}

// Value::as_f32 of a key (lib.rs:68-74): F32, or F64 rounded to f32
int llamd_gguf_get_f32(void *h, const char *key, float *out) {
    const Gguf *g = (const Gguf *)h;
    if (!g || !key || !out) return set_error("gguf: null argument");
    const Kv *e = find_kv(*g, key);
    if (!e) return set_error("gguf: %s is absent", key);
    if (e->type == T_F32) {
        memcpy(out, g->map + e->pos, 4);
    } else if (e->type == T_F64) {
        double d;
        memcpy(&d, g->map + e->pos, 8);
        *out = (float)d;
    } else {
        return set_error("gguf: %s is not a float", key);
    }
    return 0;
}

int llamd_gguf_tensor(void *h, uint64_t i, char *name, size_t cap, uint32_t *n_dims,
                      uint64_t dims[4], uint32_t *type, uint64_t *offset) {
    const Gguf *g = (const Gguf *)h;
    if (!g) return set_error("gguf: null handle");
    if (i >= g->tensors.size()) return set_error("gguf: tensor index %llu of %zu", (unsigned long long)i, g->tensors.size());
    const Tensor &t = g->tensors[i];
    if (!copy_out(t.name, name, cap)) return -1;
    if (n_dims) *n_dims = t.n_dims;
    if (dims) for (int d = 0; d < 4; ++d) dims[d] = d < (int)t.n_dims ? t.dims[d] : 1;
    if (type) *type = t.type;
    if (offset) *offset = t.offset;
    return 0;
}

int64_t llamd_gguf_find_tensor(void *h, const char *name) {
    const Gguf *g = (const Gguf *)h;
    if (!g || !name) return set_error("gguf: null argument");
    const Tensor *t = find_tensor(*g, name);
    return t ? (int64_t)(t - g->tensors.data()) : -1;
}

const void *llamd_gguf_tensor_data(void *h, uint64_t i, uint64_t *nbytes) {
    const Gguf *g = (const Gguf *)h;
    if (!g) { set_error("gguf: null handle"); return nullptr; }
    if (i >= g->tensors.size()) { set_error("gguf: tensor index %llu of %zu", (unsigned long long)i, g->tensors.size()); return nullptr; }
    uint64_t n = 0;
    const uint8_t *p = tensor_bytes(*g, g->tensors[i], &n);
    if (p && nbytes) *nbytes = n;
    return p;
}

// A Q6_K tensor to the device in the tiled layout, no dequantization
// (device.rs:236-248): 2D [k, rows] as one matrix; 3D [k, rows, n_expert] as
// n_expert expert matrices (the expert index is the slowest axis,
// model.rs:181-227).
void *llamd_gguf_upload_q6k(void *h, const char *name) {
    const Gguf *g = (const Gguf *)h;
    if (!g || !name) { set_error("gguf: null argument"); return nullptr; }
    const Tensor *t = find_tensor(*g, name);
    if (!t) { set_error("gguf: tensor %s is absent", name); return nullptr; }
    if (t->type != 14) { set_error("planar upload: %s is type %u, not Q6_K", name, t->type); return nullptr; }
    if (t->n_dims < 2 || t->n_dims > 3) { set_error("upload: %s has %u dims, expected 2 or 3", name, t->n_dims); return nullptr; }
    uint64_t nbytes;
    const uint8_t *p = tensor_bytes(*g, *t, &nbytes);
    if (!p) return nullptr;
    const uint64_t k = t->dims[0], rows = t->dims[1], ne = t->n_dims == 3 ? t->dims[2] : 1;
    if (k % 256 || rows == 0 || rows > INT32_MAX || ne > INT32_MAX || k / 256 > INT32_MAX) {
        set_error("upload: %s has shape [%llu, %llu, %llu]", name, (unsigned long long)k,
                  (unsigned long long)rows, (unsigned long long)ne);
        return nullptr;
    }
    if (t->n_dims == 2) return llamd_rocm_upload_q6k(p, (int)rows, (int)(k / 256));
    return llamd_rocm_upload_q6k_experts(p, (int)ne, (int)rows, (int)(k / 256));
}

// One Qwen3-MoE FFN layer from the file: router blk.L.ffn_gate_inp.weight (F32
// [n_embd, n_expert]) and the Q6_K expert tensors blk.L.ffn_{gate,up}_exps
// ([n_embd, n_ff, n_expert]) and ffn_down_exps ([n_ff, n_embd, n_expert]);
// n_expert_used from {arch}.expert_used_count (hparams.rs:77-135).
void *llamd_gguf_moe_create(void *h, int layer) {
    const Gguf *g = (const Gguf *)h;
    if (!g || layer < 0) { set_error("gguf: bad argument"); return nullptr; }
    const Kv *ak = find_kv(*g, "general.architecture");
    if (!ak || ak->type != T_STRING) { set_error("hparams: general.architecture is absent"); return nullptr; }
    const uint64_t alen = read_bits(g->map + ak->pos, 8);
    const std::string arch((const char *)g->map + ak->pos + 8, (size_t)alen);
    uint64_t used = 0;
    const std::string used_key = arch + ".expert_used_count";
    const Kv *uk = find_kv(*g, used_key.c_str());
    if (!uk || !as_u64(*g, *uk, &used)) { set_error("hparams: %s is absent", used_key.c_str()); return nullptr; }
    const std::string b = "blk." + std::to_string(layer) + ".";
    const Tensor *tr = find_tensor(*g, (b + "ffn_gate_inp.weight").c_str());
    const Tensor *tg = find_tensor(*g, (b + "ffn_gate_exps.weight").c_str());
    const Tensor *tu = find_tensor(*g, (b + "ffn_up_exps.weight").c_str());
    const Tensor *td = find_tensor(*g, (b + "ffn_down_exps.weight").c_str());
    if (!tr || !tg || !tu || !td) { set_error("moe layer: blk.%d lacks a router or expert tensor", layer); return nullptr; }
    if (tr->type != 0 || tr->n_dims != 2) { set_error("moe layer: %s must be F32 [n_embd, n_expert]", tr->name.c_str()); return nullptr; }
    const uint64_t n_embd = tr->dims[0], n_expert = tr->dims[1];
    for (const Tensor *t : {tg, tu, td}) {
        if (t->type != 14 || t->n_dims != 3 || t->dims[2] != n_expert) {
            set_error("moe layer: %s must be Q6_K [., ., %llu]", t->name.c_str(), (unsigned long long)n_expert);
            return nullptr;
        }
    }
    const uint64_t n_ff = tg->dims[1];
    if (tg->dims[0] != n_embd || tu->dims[0] != n_embd || tu->dims[1] != n_ff ||
        td->dims[0] != n_ff || td->dims[1] != n_embd) {
        set_error("moe layer: blk.%d expert shapes disagree with the router's n_embd %llu", layer,
                  (unsigned long long)n_embd);
        return nullptr;
    }
    if (n_embd > INT32_MAX || n_ff > INT32_MAX || n_expert > INT32_MAX || used > n_expert) {
        set_error("moe layer: blk.%d shape out of range", layer);
        return nullptr;
    }
    uint64_t nb;
    const void *router = tensor_bytes(*g, *tr, &nb);
    const void *gate = router ? tensor_bytes(*g, *tg, &nb) : nullptr;
    const void *up = gate ? tensor_bytes(*g, *tu, &nb) : nullptr;
    const void *down = up ? tensor_bytes(*g, *td, &nb) : nullptr;
    if (!down) return nullptr;
    return llamd_hip_moe_create((const float *)router, gate, up, down, (int)n_embd, (int)n_ff,
                                (int)n_expert, (int)used);
}

}  // extern "C"

