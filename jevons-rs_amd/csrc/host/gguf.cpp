// GGUF v2/v3 reader: metadata, tensor directory and bounded tensor reads, the counterpart of
// crates/jevons-formats/src/gguf.rs:1-372, plus the read -> upload step of the model loader
// (crates/jevons-gemma4-diffusion/src/model.rs:302-351). The on-disk GGML block bytes are
// handed to jv_qmatrix_upload unchanged.

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "jevons_qmm.h"

extern "C" jv_status jv_internal_fail(jv_status st, const char *msg);

namespace {

constexpr uint64_t kMaxString = 1ull << 24;
constexpr uint64_t kMaxArray = 1ull << 26;
constexpr uint32_t kMaxDims = 4;

// One metadata value: the scalar kinds as integers or floats, strings as text; arrays keep
// their element count only (the path reads no array-valued keys).
struct Value {
    uint32_t kind = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    bool is_unsigned = false, is_signed = false, is_float = false, is_bool = false;
    std::string s;
    uint64_t array_len = 0;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;  // GGML order: dims[0] is the contiguous row length
    uint32_t type = 0;
    uint64_t offset = 0;         // absolute file offset
    uint64_t bytes = 0;          // 0 for types without a block size
};

jv_status bad(const std::string &m) { return jv_internal_fail(JV_ERR_INVALID, ("Invalid GGUF file: " + m).c_str()); }

// Block (elements, bytes) of the GGML types this library decodes (gguf.rs:134-144).
bool block_of(uint32_t type, uint64_t *elems, uint64_t *bytes) {
    uint32_t e, b;
    if (jv_type_block(type, &e, &b) != JV_OK) return false;
    *elems = e;
    *bytes = b;
    return true;
}

struct Cursor {
    const std::vector<uint8_t> &buf;
    size_t pos = 0;
    bool ok = true;
    explicit Cursor(const std::vector<uint8_t> &b) : buf(b) {}
    bool take(void *dst, size_t n) {
        if (!ok || pos + n > buf.size()) return ok = false;
        memcpy(dst, buf.data() + pos, n);
        pos += n;
        return true;
    }
    uint32_t u32() { uint32_t v = 0; take(&v, 4); return v; }
    uint64_t u64() { uint64_t v = 0; take(&v, 8); return v; }
};

}  // namespace

struct jv_gguf {
    int fd = -1;
    uint64_t file_len = 0;
    std::map<std::string, Value> metadata;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> by_name;
};

namespace {

// Reads the whole header into memory in growing chunks (it precedes the aligned data section).
jv_status parse(jv_gguf *g) {
    std::vector<uint8_t> head;
    size_t want = 1 << 20;
    for (;;) {
        head.resize(std::min<uint64_t>(want, g->file_len));
        if (pread(g->fd, head.data(), head.size(), 0) != (ssize_t)head.size())
            return jv_internal_fail(JV_ERR_INVALID, "I/O error reading the model header");
        Cursor c(head);
        char magic[4];
        if (!c.take(magic, 4)) return bad("truncated header");
        if (memcmp(magic, "GGUF", 4) != 0) return bad("bad magic");
        const uint32_t version = c.u32();
        if (c.ok && (version < 2 || version > 3)) return bad("unsupported version " + std::to_string(version));
        const uint64_t tensor_count = c.u64(), kv_count = c.u64();
        if (c.ok && (tensor_count > (1u << 20) || kv_count > (1u << 20))) return bad("implausible header counts");
        std::map<std::string, Value> meta;
        std::vector<Tensor> infos;
        std::string err;
        auto str = [&](std::string &out) {
            const uint64_t len = c.u64();
            if (!c.ok) return false;
            if (len > kMaxString) { err = "string is too long"; return false; }
            out.resize(len);
            return len == 0 || c.take(&out[0], len);
        };
        std::function<bool(uint32_t, int, Value &)> value = [&](uint32_t kind, int depth, Value &v) -> bool {
            v.kind = kind;
            switch (kind) {
            case 0: { uint8_t x = 0; c.take(&x, 1); v.u = x; v.is_unsigned = true; break; }
            case 1: { int8_t x = 0; c.take(&x, 1); v.i = x; v.is_signed = true; break; }
            case 2: { uint16_t x = 0; c.take(&x, 2); v.u = x; v.is_unsigned = true; break; }
            case 3: { int16_t x = 0; c.take(&x, 2); v.i = x; v.is_signed = true; break; }
            case 4: v.u = c.u32(); v.is_unsigned = true; break;
            case 5: { int32_t x = 0; c.take(&x, 4); v.i = x; v.is_signed = true; break; }
            case 6: { float x = 0; c.take(&x, 4); v.f = x; v.is_float = true; break; }
            case 7: {
                uint8_t x = 0;
                c.take(&x, 1);
                if (c.ok && x > 1) { err = "invalid boolean"; return false; }
                v.u = x;
                v.is_bool = true;
                break;
            }
            case 8: return str(v.s);
            case 9: {
                if (depth > 0) { err = "nested arrays are not supported"; return false; }
                const uint32_t inner = c.u32();
                const uint64_t len = c.u64();
                if (!c.ok) return false;
                if (len > kMaxArray) { err = "array is too long"; return false; }
                v.array_len = len;
                Value e;
                for (uint64_t i = 0; i < len && c.ok; ++i)
                    if (!value(inner, depth + 1, e)) return false;
                break;
            }
            case 10: v.u = c.u64(); v.is_unsigned = true; break;
            case 11: { int64_t x = 0; c.take(&x, 8); v.i = x; v.is_signed = true; break; }
            case 12: { double x = 0; c.take(&x, 8); v.f = x; v.is_float = true; break; }
            default: err = "unknown metadata type " + std::to_string(kind); return false;
            }
            return c.ok;
        };
        bool done = c.ok;
        for (uint64_t i = 0; done && i < kv_count; ++i) {
            std::string key;
            Value v;
            if (!str(key)) { done = false; break; }
            const uint32_t kind = c.u32();
            if (!c.ok || !value(kind, 0, v)) { done = false; break; }
            if (!meta.emplace(key, v).second) return bad("duplicate metadata key");
        }
        for (uint64_t i = 0; done && i < tensor_count; ++i) {
            Tensor t;
            if (!str(t.name)) { done = false; break; }
            const uint32_t nd = c.u32();
            if (!c.ok) { done = false; break; }
            if (nd == 0 || nd > kMaxDims)
                return bad("tensor " + t.name + " has " + std::to_string(nd) + " dimensions");
            for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.u64());
            t.type = c.u32();
            t.offset = c.u64();
            if (!c.ok) { done = false; break; }
            infos.push_back(std::move(t));
        }
        if (!err.empty()) return bad(err);
        if (!done || !c.ok) {
            if (head.size() >= g->file_len) return bad("truncated header");
            want *= 4;  // the header is longer than what was read: read more
            continue;
        }
        uint64_t alignment = 32;
        auto al = meta.find("general.alignment");
        if (al != meta.end()) {
            const Value &v = al->second;
            const bool ok = (v.is_unsigned && v.u > 0 && (v.u & (v.u - 1)) == 0) ||
                            (v.is_signed && v.i > 0 && ((uint64_t)v.i & ((uint64_t)v.i - 1)) == 0);
            if (!ok) return bad("invalid alignment");
            alignment = v.is_unsigned ? v.u : (uint64_t)v.i;
        }
        const uint64_t data_start = (c.pos + alignment - 1) / alignment * alignment;
        for (Tensor &t : infos) {
            uint64_t elements = 1;
            for (uint64_t d : t.dims) {
                if (d != 0 && elements > UINT64_MAX / d) return bad("tensor " + t.name + " is too large");
                elements *= d;
            }
            uint64_t be, bb;
            if (block_of(t.type, &be, &bb)) {
                if (t.dims[0] % be != 0) return bad("tensor " + t.name + " rows are not block aligned");
                t.bytes = elements / be * bb;
            }
            const uint64_t start = data_start + t.offset;
            if (t.offset % alignment != 0 || start < data_start || start + t.bytes < start || start + t.bytes > g->file_len)
                return bad("tensor " + t.name + " is out of bounds");
            t.offset = start;
            if (!g->by_name.emplace(t.name, g->tensors.size()).second) return bad("duplicate tensor name");
            g->tensors.push_back(t);
        }
        g->metadata = std::move(meta);
        return JV_OK;
    }
}

const Value *meta_of(const jv_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->metadata.find(key);
    return it == g->metadata.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

jv_status jv_gguf_open(const char *path, jv_gguf **out) {
    if (!out || !path) return jv_internal_fail(JV_ERR_INVALID, "null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return jv_internal_fail(JV_ERR_INVALID, (std::string("I/O error reading the model: cannot open ") + path).c_str());
    struct stat st {};
    if (fstat(fd, &st) != 0) {
        close(fd);
        return jv_internal_fail(JV_ERR_INVALID, "I/O error reading the model: stat failed");
    }
    auto *g = new jv_gguf();
    g->fd = fd;
    g->file_len = (uint64_t)st.st_size;
    const jv_status s = parse(g);
    if (s != JV_OK) {
        close(fd);
        delete g;
        return s;
    }
    *out = g;
    return JV_OK;
}

void jv_gguf_close(jv_gguf *g) {
    if (!g) return;
    if (g->fd >= 0) close(g->fd);
    delete g;
}

size_t jv_gguf_tensor_count(const jv_gguf *g) { return g ? g->tensors.size() : 0; }

jv_status jv_gguf_tensor_info(const jv_gguf *g, size_t index, const char **name, uint32_t *ggml_type,
                              uint32_t *n_dims, uint64_t dims[4], uint64_t *offset, uint64_t *bytes) {
    if (!g || index >= g->tensors.size()) return jv_internal_fail(JV_ERR_INVALID, "tensor index out of range");
    const Tensor &t = g->tensors[index];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (n_dims) *n_dims = (uint32_t)t.dims.size();
    if (dims)
        for (uint32_t d = 0; d < 4; ++d) dims[d] = d < t.dims.size() ? t.dims[d] : 1;
    if (offset) *offset = t.offset;
    if (bytes) *bytes = t.bytes;
    return JV_OK;
}

jv_status jv_gguf_find(const jv_gguf *g, const char *name, size_t *index) {
    if (!g || !name || !index) return jv_internal_fail(JV_ERR_INVALID, "null argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return jv_internal_fail(JV_ERR_INVALID, (std::string("Missing tensor ") + name).c_str());
    *index = it->second;
    return JV_OK;
}

jv_status jv_gguf_u64(const jv_gguf *g, const char *key, uint64_t *out) {
    const Value *v = meta_of(g, key);
    if (!v) return jv_internal_fail(JV_ERR_INVALID, (std::string("Missing GGUF metadata key ") + (key ? key : "")).c_str());
    if (v->is_unsigned) *out = v->u;
    else if (v->is_signed && v->i >= 0) *out = (uint64_t)v->i;
    else return jv_internal_fail(JV_ERR_INVALID, (std::string("Invalid GGUF file: ") + key + " is not an unsigned integer").c_str());
    return JV_OK;
}

jv_status jv_gguf_f32(const jv_gguf *g, const char *key, float *out) {
    const Value *v = meta_of(g, key);
    if (!v) return jv_internal_fail(JV_ERR_INVALID, (std::string("Missing GGUF metadata key ") + (key ? key : "")).c_str());
    if (!v->is_float) return jv_internal_fail(JV_ERR_INVALID, (std::string("Invalid GGUF file: ") + key + " is not a float").c_str());
    *out = (float)v->f;
    return JV_OK;
}

jv_status jv_gguf_str(const jv_gguf *g, const char *key, const char **out) {
    const Value *v = meta_of(g, key);
    if (!v) return jv_internal_fail(JV_ERR_INVALID, (std::string("Missing GGUF metadata key ") + (key ? key : "")).c_str());
    if (v->kind != 8) return jv_internal_fail(JV_ERR_INVALID, (std::string("Invalid GGUF file: ") + key + " is not a string").c_str());
    *out = v->s.c_str();
    return JV_OK;
}

jv_status jv_gguf_read(const jv_gguf *g, size_t index, uint64_t start, uint64_t len, void *dst) {
    if (!g || index >= g->tensors.size()) return jv_internal_fail(JV_ERR_INVALID, "tensor index out of range");
    const Tensor &t = g->tensors[index];
    uint64_t be, bb;
    if (!block_of(t.type, &be, &bb))
        return jv_internal_fail(JV_ERR_UNSUPPORTED,
                                ("Invalid GGUF file: tensor " + t.name + " has unsupported type " + std::to_string(t.type)).c_str());
    if (start + len < start || start + len > t.bytes)
        return jv_internal_fail(JV_ERR_INVALID, ("Invalid GGUF file: range is outside tensor " + t.name).c_str());
    if (len && !dst) return jv_internal_fail(JV_ERR_INVALID, "null buffer");
    uint8_t *p = (uint8_t *)dst;
    uint64_t done = 0;
    while (done < len) {
        const ssize_t r = pread(g->fd, p + done, (size_t)std::min<uint64_t>(len - done, 1ull << 30), (off_t)(t.offset + start + done));
        if (r <= 0) return jv_internal_fail(JV_ERR_INVALID, "I/O error reading the model");
        done += (uint64_t)r;
    }
    return JV_OK;
}

jv_status jv_gguf_upload(jv_ctx *ctx, const jv_gguf *g, const char *name, jv_qmatrix **out) {
    if (!out) return jv_internal_fail(JV_ERR_INVALID, "null output pointer");
    *out = nullptr;
    size_t index;
    jv_status st = jv_gguf_find(g, name, &index);
    if (st != JV_OK) return st;
    const Tensor &t = g->tensors[index];
    if (t.dims.size() < 2 || t.dims.size() > 3)
        return jv_internal_fail(JV_ERR_INVALID, ("tensor " + t.name + " is not a matrix or an expert stack").c_str());
    std::vector<uint8_t> raw(t.bytes);
    st = jv_gguf_read(g, index, 0, t.bytes, raw.data());
    if (st != JV_OK) return st;
    const size_t k = (size_t)t.dims[0], n = (size_t)t.dims[1], experts = t.dims.size() == 3 ? (size_t)t.dims[2] : 1;
    return jv_qmatrix_upload(ctx, t.type, n, k, experts, raw.data(), raw.size(), out);
}

}  // extern "C"
