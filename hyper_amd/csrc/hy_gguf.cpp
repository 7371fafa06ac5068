// GGUF expert loading: a read-only GGUF (v2, v3) reader over memory-mapped files -- metadata, the tensor table and
// zero-copy tensor views -- and the lookup of one layer's expert tensors, which hy_upload_experts then places on the
// device.  Replaces class GGUF (src/gguf.h:38-70, src/gguf.cpp:84-285) and expert_tensors (src/experts.cu:12-22).
//
// File layout (GGUF v2/v3, little endian): "GGUF", u32 version, u64 tensor count, u64 key/value count; the
// key/value pairs (string key, u32 value type, value); the tensor table (string name, u32 n_dims, u64 ne[n_dims],
// u32 type, u64 offset); then, from the header's end rounded up to general.alignment (32 by default), the tensor
// data, each tensor at its offset.  A string is a u64 length and its bytes; an array a u32 element type, a u64 count
// and the elements.
#include "hy_error.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <vector>

using hy::set_error;

namespace {

// GGML block geometry of the tensor types a model file may hold (the set src/gguf.cpp:43-82 accepts)
bool ggml_block(uint32_t type, size_t &bytes, int64_t &elems) {
    switch (type) {
    case 0: bytes = 4; elems = 1; return true;            // F32
    case 1: bytes = 2; elems = 1; return true;            // F16
    case 30: bytes = 2; elems = 1; return true;           // BF16
    case 26: bytes = 4; elems = 1; return true;           // I32
    case 27: bytes = 8; elems = 1; return true;           // I64
    case 2: bytes = 18; elems = 32; return true;          // Q4_0
    case 3: bytes = 20; elems = 32; return true;          // Q4_1
    case 6: bytes = 22; elems = 32; return true;          // Q5_0
    case 7: bytes = 24; elems = 32; return true;          // Q5_1
    case 8: bytes = 34; elems = 32; return true;          // Q8_0
    case 20: bytes = 18; elems = 32; return true;         // IQ4_NL
    case 39: bytes = 17; elems = 32; return true;         // MXFP4
    case 10: bytes = 84; elems = 256; return true;        // Q2_K
    case 11: bytes = 110; elems = 256; return true;       // Q3_K
    case 12: bytes = 144; elems = 256; return true;       // Q4_K
    case 13: bytes = 176; elems = 256; return true;       // Q5_K
    case 14: bytes = 210; elems = 256; return true;       // Q6_K
    case 16: bytes = 66; elems = 256; return true;        // IQ2_XXS
    case 17: bytes = 74; elems = 256; return true;        // IQ2_XS
    case 18: bytes = 98; elems = 256; return true;        // IQ3_XXS
    case 19: bytes = 50; elems = 256; return true;        // IQ1_S
    case 21: bytes = 110; elems = 256; return true;       // IQ3_S
    case 22: bytes = 82; elems = 256; return true;        // IQ2_S
    case 23: bytes = 136; elems = 256; return true;       // IQ4_XS
    default: return false;
    }
}

// a metadata value: integers (and booleans) as int64, floats as double, strings, and arrays of one of these
struct Value {
    enum Kind { INT, BOOL, FLOAT, STR, INT_ARR, FLOAT_ARR, STR_ARR } kind = INT;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    std::vector<int64_t> ia;
    std::vector<double> fa;
    std::vector<std::string> sa;
};

enum : uint32_t { V_U8 = 0, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 };

// bounds-checked reads from the mapped header; the first failure sticks and names what was being read
struct Reader {
    const uint8_t *p, *end;
    std::string err;
    bool need(size_t n, const char *what) {
        if (!err.empty()) return false;
        if ((size_t) (end - p) < n) { err = std::string("truncated ") + what; return false; }
        return true;
    }
    template <class T> T num(const char *what) {
        T v{};
        if (need(sizeof(T), what)) { std::memcpy(&v, p, sizeof(T)); p += sizeof(T); }
        return v;
    }
    std::string str(const char *what) {
        const uint64_t n = num<uint64_t>(what);
        if (!need(n, what)) return {};
        std::string s((const char *) p, (size_t) n);
        p += n;
        return s;
    }
    bool integer(uint32_t t, int64_t &v) {   // one integer or boolean element of type t
        switch (t) {
        case V_U8: case V_BOOL: v = num<uint8_t>("value"); return true;
        case V_I8: v = num<int8_t>("value"); return true;
        case V_U16: v = num<uint16_t>("value"); return true;
        case V_I16: v = num<int16_t>("value"); return true;
        case V_U32: v = num<uint32_t>("value"); return true;
        case V_I32: v = num<int32_t>("value"); return true;
        case V_U64: v = (int64_t) num<uint64_t>("value"); return true;
        case V_I64: v = num<int64_t>("value"); return true;
        default: return false;
        }
    }
    bool value(uint32_t t, Value &out) {
        int64_t iv;
        if (t == V_BOOL) { out.kind = Value::BOOL; out.i = num<uint8_t>("value"); return err.empty(); }
        if (integer(t, iv)) { out.kind = Value::INT; out.i = iv; return err.empty(); }
        switch (t) {
        case V_F32: out.kind = Value::FLOAT; out.f = num<float>("value"); return err.empty();
        case V_F64: out.kind = Value::FLOAT; out.f = num<double>("value"); return err.empty();
        case V_STR: out.kind = Value::STR; out.s = str("string"); return err.empty();
        case V_ARR: {
            const uint32_t at = num<uint32_t>("array type");
            const uint64_t n = num<uint64_t>("array length");
            if (!err.empty()) return false;
            if (n > (uint64_t) (end - p)) { err = "truncated array"; return false; }   // every element takes >= 1 byte
            if (at == V_STR) {
                out.kind = Value::STR_ARR;
                out.sa.reserve((size_t) n);
                for (uint64_t k = 0; k < n && err.empty(); ++k) out.sa.push_back(str("string"));
            } else if (at == V_F32 || at == V_F64) {
                out.kind = Value::FLOAT_ARR;
                out.fa.reserve((size_t) n);
                for (uint64_t k = 0; k < n && err.empty(); ++k) out.fa.push_back(at == V_F32 ? (double) num<float>("value") : num<double>("value"));
            } else {
                out.kind = Value::INT_ARR;
                out.ia.reserve((size_t) n);
                for (uint64_t k = 0; k < n && err.empty(); ++k) {
                    if (!integer(at, iv)) { err = "array of unsupported element type " + std::to_string(at); return false; }
                    out.ia.push_back(iv);
                }
            }
            return err.empty();
        }
        default: err = "unknown value type " + std::to_string(t); return false;
        }
    }
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    int32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    const uint8_t *data = nullptr;
    size_t nbytes = 0;
};

struct Mapping {
    int fd = -1;
    void *p = MAP_FAILED;
    size_t size = 0;
};

} // namespace

struct hy_gguf {
    std::vector<Mapping> maps;
    std::map<std::string, Value> kv;       // the first shard's metadata
    std::vector<Tensor> tensors;           // every shard's, in file order
    std::map<std::string, size_t> index;   // name -> position in tensors
    std::string arch;

    ~hy_gguf() {
        for (Mapping &m : maps) {
            if (m.p != MAP_FAILED) munmap(m.p, m.size);
            if (m.fd >= 0) close(m.fd);
        }
    }

    // map one file and read its header; metadata is kept for the first shard only (src/gguf.cpp:205)
    int load(const std::string &path, bool first) {
        Mapping m;
        m.fd = open(path.c_str(), O_RDONLY);
        if (m.fd < 0) { set_error("hy_gguf_open: cannot open %s", path.c_str()); return HY_EINVAL; }
        struct stat st;
        if (fstat(m.fd, &st) != 0 || st.st_size <= 0) { close(m.fd); set_error("hy_gguf_open: cannot stat %s", path.c_str()); return HY_EINVAL; }
        m.size = (size_t) st.st_size;
        m.p = mmap(nullptr, m.size, PROT_READ, MAP_SHARED, m.fd, 0);
        if (m.p == MAP_FAILED) { close(m.fd); set_error("hy_gguf_open: mmap of %s failed", path.c_str()); return HY_EINVAL; }
        maps.push_back(m);
        const uint8_t *base = (const uint8_t *) m.p;
        Reader r{base, base + m.size, {}};
        auto fail = [&](const std::string &what) { set_error("hy_gguf_open: %s: %s", path.c_str(), what.c_str()); return HY_EINVAL; };
        if (r.num<uint32_t>("magic") != 0x46554747u) return fail(r.err.empty() ? "not a GGUF file (bad magic)" : r.err);
        const uint32_t version = r.num<uint32_t>("version");
        if (r.err.empty() && version < 2) return fail("GGUF version " + std::to_string(version) + " is not supported (2 or later)");
        const uint64_t n_tensors = r.num<uint64_t>("tensor count"), n_kv = r.num<uint64_t>("key/value count");
        if (!r.err.empty()) return fail(r.err);
        std::map<std::string, Value> meta;
        for (uint64_t k = 0; k < n_kv; ++k) {
            std::string key = r.str("key");
            const uint32_t t = r.num<uint32_t>("value type");
            Value v;
            if (!r.err.empty() || !r.value(t, v)) return fail(r.err + (key.empty() ? "" : " (key " + key + ")"));
            meta[key] = std::move(v);
        }
        uint64_t alignment = 32;
        if (auto it = meta.find("general.alignment"); it != meta.end() && it->second.kind == Value::INT) alignment = (uint64_t) it->second.i;
        if (alignment == 0) return fail("general.alignment is 0");
        std::vector<std::pair<size_t, uint64_t>> offsets;
        for (uint64_t k = 0; k < n_tensors; ++k) {
            Tensor t;
            t.name = r.str("tensor name");
            const uint32_t nd = r.num<uint32_t>("tensor dims");
            if (r.err.empty() && (nd < 1 || nd > 4)) return fail("tensor " + t.name + " has " + std::to_string(nd) + " dimensions");
            t.n_dims = (int32_t) nd;
            for (uint32_t d = 0; d < nd; ++d) t.ne[d] = (int64_t) r.num<uint64_t>("tensor shape");
            t.type = r.num<uint32_t>("tensor type");
            const uint64_t off = r.num<uint64_t>("tensor offset");
            if (!r.err.empty()) return fail(r.err);
            if (index.count(t.name)) return fail("tensor " + t.name + " appears twice");
            index[t.name] = tensors.size();
            offsets.emplace_back(tensors.size(), off);
            tensors.push_back(std::move(t));
        }
        const uint64_t head = (uint64_t) (r.p - base), data0 = (head + alignment - 1) / alignment * alignment;
        for (auto &[i, off] : offsets) {
            Tensor &t = tensors[i];
            size_t bb;
            int64_t be;
            if (!ggml_block(t.type, bb, be)) {
                set_error("hy_gguf_open: %s: tensor %s has unsupported type %u", path.c_str(), t.name.c_str(), t.type);
                return HY_EUNSUPPORTED_TYPE;
            }
            int64_t nel = 1;
            for (int d = 0; d < t.n_dims; ++d) {
                if (t.ne[d] <= 0 || nel > INT64_MAX / t.ne[d]) return fail("tensor " + t.name + " has a bad shape");
                nel *= t.ne[d];
            }
            if (t.ne[0] % be) return fail("tensor " + t.name + ": row of " + std::to_string(t.ne[0]) + " values is not whole blocks");
            const size_t row = (size_t) (t.ne[0] / be) * bb, rows = (size_t) (nel / t.ne[0]);
            if (rows && row > SIZE_MAX / rows) return fail("tensor " + t.name + " has a bad shape");
            t.nbytes = row * rows;
            if (off > m.size || data0 > m.size - off || t.nbytes > m.size - data0 - off) return fail("tensor " + t.name + " lies outside the file");
            t.data = base + data0 + off;
        }
        if (first) kv = std::move(meta);
        return HY_OK;
    }

    const Value *find(const char *key) const {
        if (!key) return nullptr;
        auto it = kv.find(key);
        return it == kv.end() ? nullptr : &it->second;
    }
};

static void fill(const Tensor &t, hy_gguf_tensor_info *out) {
    out->name = t.name.c_str();
    out->data = t.data;
    out->nbytes = t.nbytes;
    out->type = (int32_t) t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
}

extern "C" {

int hy_gguf_open(const char *path, hy_gguf **out) {
    if (!path || !out) { set_error("hy_gguf_open: null argument"); return HY_EINVAL; }
    *out = nullptr;
    hy_gguf *g = new (std::nothrow) hy_gguf;
    if (!g) { set_error("hy_gguf_open: out of host memory"); return HY_EINVAL; }
    const std::string p(path);
    // a split model: <name>-00001-of-0000N.gguf names N shards, numbered in the same five-digit field
    const size_t at = p.rfind("-00001-of-");
    int rc = HY_OK;
    if (at != std::string::npos && p.size() > at + 15) {
        const int n = std::atoi(p.substr(at + 10, 5).c_str());
        if (n < 1 || n > 99999) { delete g; set_error("hy_gguf_open: bad shard count in %s", path); return HY_EINVAL; }
        for (int i = 1; i <= n && rc == HY_OK; ++i) {
            char num[8];
            std::snprintf(num, sizeof num, "%05d", i);
            std::string shard = p;
            shard.replace(at + 1, 5, num);
            rc = g->load(shard, i == 1);
        }
    } else {
        rc = g->load(p, true);
    }
    if (rc == HY_OK) {
        const Value *a = g->find("general.architecture");   // required, as src/gguf.cpp:150
        if (!a || a->kind != Value::STR) { set_error("hy_gguf_open: %s: missing key general.architecture", path); rc = HY_EINVAL; }
        else g->arch = a->s;
    }
    if (rc != HY_OK) { delete g; return rc; }
    *out = g;
    return HY_OK;
}

int hy_gguf_close(hy_gguf *g) {
    delete g;
    return HY_OK;
}

const char *hy_gguf_arch(const hy_gguf *g) { return g ? g->arch.c_str() : ""; }

int hy_gguf_has(const hy_gguf *g, const char *key) { return g && g->find(key) ? 1 : 0; }

int hy_gguf_get_int(const hy_gguf *g, const char *key, int64_t *out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out) { set_error("hy_gguf_get_int: missing key %s", key ? key : "(null)"); return HY_EINVAL; }
    if (v->kind != Value::INT && v->kind != Value::BOOL) { set_error("hy_gguf_get_int: key is not an int: %s", key); return HY_EINVAL; }
    *out = v->i;
    return HY_OK;
}

int hy_gguf_get_float(const hy_gguf *g, const char *key, double *out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out) { set_error("hy_gguf_get_float: missing key %s", key ? key : "(null)"); return HY_EINVAL; }
    if (v->kind == Value::FLOAT) *out = v->f;
    else if (v->kind == Value::INT) *out = (double) v->i;
    else { set_error("hy_gguf_get_float: key is not a float: %s", key); return HY_EINVAL; }
    return HY_OK;
}

int hy_gguf_get_str(const hy_gguf *g, const char *key, const char **out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out) { set_error("hy_gguf_get_str: missing key %s", key ? key : "(null)"); return HY_EINVAL; }
    if (v->kind != Value::STR) { set_error("hy_gguf_get_str: key is not a string: %s", key); return HY_EINVAL; }
    *out = v->s.c_str();
    return HY_OK;
}

int hy_gguf_get_int_arr(const hy_gguf *g, const char *key, int64_t *out, size_t cap, size_t *n) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !n) { set_error("hy_gguf_get_int_arr: missing key %s", key ? key : "(null)"); return HY_EINVAL; }
    if (v->kind == Value::INT) {   // a scalar reads as one element (src/gguf.cpp:266)
        *n = 1;
        if (out && cap >= 1) out[0] = v->i;
        return HY_OK;
    }
    if (v->kind != Value::INT_ARR) { set_error("hy_gguf_get_int_arr: key is not an int array: %s", key); return HY_EINVAL; }
    *n = v->ia.size();
    for (size_t i = 0; out && i < v->ia.size() && i < cap; ++i) out[i] = v->ia[i];
    return HY_OK;
}

int hy_gguf_get_float_arr(const hy_gguf *g, const char *key, double *out, size_t cap, size_t *n) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !n) { set_error("hy_gguf_get_float_arr: missing key %s", key ? key : "(null)"); return HY_EINVAL; }
    if (v->kind == Value::FLOAT_ARR) {
        *n = v->fa.size();
        for (size_t i = 0; out && i < v->fa.size() && i < cap; ++i) out[i] = v->fa[i];
        return HY_OK;
    }
    double f;   // otherwise a scalar float (or int) reads as one element (src/gguf.cpp:274)
    const int rc = hy_gguf_get_float(g, key, &f);
    if (rc != HY_OK) return rc;
    *n = 1;
    if (out && cap >= 1) out[0] = f;
    return HY_OK;
}

int hy_gguf_n_tensors(const hy_gguf *g) { return g ? (int) g->tensors.size() : 0; }

int hy_gguf_tensor_at(const hy_gguf *g, int i, hy_gguf_tensor_info *out) {
    if (!g || !out || i < 0 || i >= (int) g->tensors.size()) { set_error("hy_gguf_tensor_at: no tensor %d", i); return HY_EINVAL; }
    fill(g->tensors[(size_t) i], out);
    return HY_OK;
}

int hy_gguf_tensor(const hy_gguf *g, const char *name, hy_gguf_tensor_info *out) {
    if (!g || !name || !out) { set_error("hy_gguf_tensor: null argument"); return HY_EINVAL; }
    auto it = g->index.find(name);
    if (it == g->index.end()) { set_error("hy_gguf_tensor: missing tensor %s", name); return HY_EINVAL; }
    fill(g->tensors[it->second], out);
    return HY_OK;
}

int hy_gguf_expert_tensors(const hy_gguf *g, int il, int E, hy_expert_tensors *out) {
    if (!g || !out || E <= 0 || il < 0) { set_error("hy_gguf_expert_tensors: bad argument (layer %d, E %d)", il, E); return HY_EINVAL; }
    const std::string pre = "blk." + std::to_string(il) + ".";
    hy_gguf_tensor_info t[3];
    const char *names[3] = {"ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"};
    for (int i = 0; i < 3; ++i) {
        const int rc = hy_gguf_tensor(g, (pre + names[i]).c_str(), &t[i]);
        if (rc != HY_OK) return rc;
    }
    if (t[0].type != t[1].type) { set_error("hy_gguf_expert_tensors: expert gate/up types differ in layer %d", il); return HY_EBAD_SHAPE; }
    if (t[0].nbytes != t[1].nbytes || t[0].nbytes % (size_t) E || t[2].nbytes % (size_t) E) {
        set_error("hy_gguf_expert_tensors: layer %d: tensor sizes %zu / %zu / %zu do not split into %d experts", il, t[0].nbytes,
                  t[1].nbytes, t[2].nbytes, E);
        return HY_EBAD_SHAPE;
    }
    out->gate = t[0].data;
    out->up = t[1].data;
    out->down = t[2].data;
    out->gb = t[0].nbytes / (size_t) E;
    out->db = t[2].nbytes / (size_t) E;
    out->E = E;
    out->tg = t[0].type;
    out->td = t[2].type;
    return HY_OK;
}

} // extern "C"
