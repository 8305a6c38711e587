// GGUF v3 reader and device tensor store (host code).
//
// qw35_hip_gguf_parse restates the reference loader's parse_mapping
// (qw35-server/src/loader/tensors.rs:23-121) over a host image of the file:
// magic and version 3 only, metadata values walked with the same type table
// and array nesting limit (loader/metadata.rs:206-288), general.alignment
// (u32, 0 = keep 32), 1..8 dimensions, the byte size of every type by
// tensor_nbytes (tensors.rs:123-172), data section at the aligned end of the
// tensor infos, and every tensor inside the file.  The descriptors are filled
// as bridge.rs:279-290 fills qw35_metal_tensor_desc: dims padded with 1 to
// four entries, n_dims the true count, name pointing into the image.
//
// qw35_hip_store_* replace Qw35TensorStore (Qw35TensorStore.m:58-153): the
// reference wraps the model mmap in Metal buffers without a copy; HBM is not
// the host's memory, so the store copies the image once (bytes 0 .. end of the
// last tensor) into one device allocation and hands out weight views by name.
#include "qw35_kernels.h"

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/qw35_hip.h"

namespace {

void gg_err(char* err, uintptr_t err_len, const char* fmt, ...) {
    if (!err || err_len == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, (size_t)err_len, fmt, ap);
    va_end(ap);
}

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint32_t kGgufVersion = 3;

struct Cursor {
    const uint8_t* p;
    uint64_t n;
    uint64_t pos = 0;
    const char* fail = nullptr;

    bool take(uint64_t len, const uint8_t** out) {
        if (fail) return false;
        if (len > n - pos) {
            fail = "unexpected end of GGUF file";
            return false;
        }
        if (out) *out = p + pos;
        pos += len;
        return true;
    }
    bool u32(uint32_t* v) {
        const uint8_t* b;
        if (!take(4, &b)) return false;
        memcpy(v, b, 4);
        return true;
    }
    bool u64(uint64_t* v) {
        const uint8_t* b;
        if (!take(8, &b)) return false;
        memcpy(v, b, 8);
        return true;
    }
    bool str(const uint8_t** s, uint64_t* len) {
        return u64(len) && take(*len, s);
    }
};

// Byte size of one metadata scalar (metadata.rs:280-288), 0 if not a scalar.
uint64_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;   // u8, i8, bool
        case 2: case 3: return 2;           // u16, i16
        case 4: case 5: case 6: return 4;   // u32, i32, f32
        case 10: case 11: case 12: return 8;  // u64, i64, f64
        default: return 0;
    }
}

bool skip_value(Cursor& c, uint32_t t, int depth, char* err, uintptr_t err_len) {
    if (depth > 8) {
        gg_err(err, err_len, "metadata array nesting is too deep");
        return false;
    }
    const uint64_t sz = scalar_size(t);
    if (sz) return c.take(sz, nullptr) || (gg_err(err, err_len, "%s", c.fail), false);
    if (t == 8) {  // string
        const uint8_t* s;
        uint64_t len;
        return c.str(&s, &len) || (gg_err(err, err_len, "%s", c.fail), false);
    }
    if (t == 9) {  // array: item type, count, items
        uint32_t it;
        uint64_t len;
        if (!c.u32(&it) || !c.u64(&len)) return gg_err(err, err_len, "%s", c.fail), false;
        const uint64_t isz = scalar_size(it);
        if (isz) {
            if (len > (c.n - c.pos) / isz) return gg_err(err, err_len, "unexpected end of GGUF file"), false;
            return c.take(len * isz, nullptr) || (gg_err(err, err_len, "%s", c.fail), false);
        }
        if (it != 8 && it != 9) return gg_err(err, err_len, "unknown GGUF array item type %u", it), false;
        for (uint64_t i = 0; i < len; ++i)
            if (!skip_value(c, it, depth + 1, err, err_len)) return false;
        return true;
    }
    gg_err(err, err_len, "unknown GGUF metadata type %u", t);
    return false;
}

// tensor_nbytes (tensors.rs:123-172): 0 for an unknown type.
bool tensor_nbytes(uint32_t t, uint64_t elements, uint64_t* out) {
    if (t == 101) {  // GF2: 5 bytes per (padded) group of 16
        *out = (elements + 15) / 16 * 5;
        return true;
    }
    uint64_t be, bb;
    switch (t) {
        case 0: be = 1; bb = 4; break;
        case 1: be = 1; bb = 2; break;
        case 2: be = 32; bb = 18; break;
        case 3: be = 32; bb = 20; break;
        case 6: be = 32; bb = 22; break;
        case 7: be = 32; bb = 24; break;
        case 8: be = 32; bb = 34; break;
        case 9: be = 32; bb = 40; break;
        case 10: be = 256; bb = 84; break;
        case 11: be = 256; bb = 110; break;
        case 12: be = 256; bb = 144; break;
        case 13: be = 256; bb = 176; break;
        case 14: be = 256; bb = 210; break;
        case 15: be = 256; bb = 292; break;
        case 16: be = 256; bb = 66; break;
        case 17: be = 256; bb = 74; break;
        case 18: be = 256; bb = 98; break;
        case 19: be = 256; bb = 110; break;
        case 20: be = 32; bb = 18; break;
        case 21: be = 256; bb = 110; break;
        case 22: be = 256; bb = 82; break;
        case 23: be = 256; bb = 136; break;
        case 24: be = 1; bb = 1; break;
        case 25: be = 1; bb = 2; break;
        case 26: be = 1; bb = 4; break;
        case 27: be = 1; bb = 8; break;
        case 28: be = 1; bb = 8; break;
        case 29: be = 256; bb = 56; break;
        case 30: be = 1; bb = 2; break;
        case 100: be = 8; bb = 4; break;
        default: return false;
    }
    const uint64_t blocks = (elements + be - 1) / be;
    if (blocks > UINT64_MAX / bb) return false;
    *out = blocks * bb;
    return true;
}

struct Store {
    void* dev = nullptr;
    uint64_t bytes = 0;
    std::vector<std::string> names;
    std::vector<qw35_hip_tensor_desc> descs;
    std::unordered_map<std::string, size_t> index;  // name -> descs position
    // Sharing key and reference count (under g_stores_mu).
    const void* map = nullptr;
    uint64_t map_size = 0;
    uint32_t count = 0;
    int device = -1;
    int refs = 0;
};

// Every live store, so that creates over the same image and device share one.
std::mutex g_stores_mu;
std::vector<Store*> g_stores;

void store_free(Store* s) {
    if (s->dev) (void)hipFree(s->dev);
    delete s;
}

}  // namespace

extern "C" {

int qw35_hip_gguf_parse(const void* model_map, uint64_t model_size, qw35_hip_tensor_desc* out, uint32_t cap,
                        uint32_t* n_tensors, uint64_t* data_offset, char* err, uintptr_t err_len) {
    if (!model_map || !n_tensors) {
        gg_err(err, err_len, "gguf_parse: null model image or count");
        return 0;
    }
    Cursor c{static_cast<const uint8_t*>(model_map), model_size};
    uint32_t magic = 0, version = 0;
    uint64_t nt = 0, nkv = 0;
    if (!c.u32(&magic)) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
    if (magic != kGgufMagic) return gg_err(err, err_len, "gguf_parse: model is not a GGUF file"), 0;
    if (!c.u32(&version)) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
    if (version != kGgufVersion)
        return gg_err(err, err_len, "gguf_parse: only GGUF v3 is supported, found v%u", version), 0;
    if (!c.u64(&nt) || !c.u64(&nkv)) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
    if (nt > 0xFFFFFFFFull) return gg_err(err, err_len, "gguf_parse: tensor count %llu", (unsigned long long)nt), 0;

    uint64_t alignment = 32;
    char msg[160];
    for (uint64_t i = 0; i < nkv; ++i) {
        const uint8_t* key;
        uint64_t key_len;
        uint32_t t;
        if (!c.str(&key, &key_len) || !c.u32(&t)) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
        if (t == 4 && key_len == 17 && memcmp(key, "general.alignment", 17) == 0) {
            uint32_t a;
            if (!c.u32(&a)) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
            if (a != 0) alignment = a;
            continue;
        }
        if (!skip_value(c, t, 0, msg, sizeof msg)) return gg_err(err, err_len, "gguf_parse: %s", msg), 0;
    }

    // every tensor info takes at least 32 bytes (name length, ndim, one dim, type, offset)
    if (nt > (c.n - c.pos) / 32) return gg_err(err, err_len, "gguf_parse: unexpected end of GGUF file"), 0;
    std::vector<qw35_hip_tensor_desc> all;
    try {
        all.resize((size_t)nt);
    } catch (...) {
        return gg_err(err, err_len, "gguf_parse: %llu tensor infos do not fit in host memory",
                      (unsigned long long)nt),
               0;
    }
    for (uint64_t i = 0; i < nt; ++i) {
        const uint8_t* name;
        uint64_t name_len;
        uint32_t ndim;
        if (!c.str(&name, &name_len) || !c.u32(&ndim)) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
        const int shown = (int)(name_len < 96 ? name_len : 96);
        if (ndim == 0 || ndim > 8)
            return gg_err(err, err_len, "gguf_parse: tensor %.*s has unsupported dimension count %u", shown,
                          (const char*)name, ndim),
                   0;
        uint64_t dims[8];
        uint64_t elements = 1;
        for (uint32_t d = 0; d < ndim; ++d) {
            if (!c.u64(&dims[d])) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
            if (dims[d] != 0) {
                if (elements > UINT64_MAX / dims[d])
                    return gg_err(err, err_len, "gguf_parse: tensor %.*s element count overflow", shown,
                                  (const char*)name),
                           0;
                elements *= dims[d];
            }
        }
        uint32_t type_id;
        uint64_t rel;
        if (!c.u32(&type_id) || !c.u64(&rel)) return gg_err(err, err_len, "gguf_parse: %s", c.fail), 0;
        uint64_t bytes;
        if (!tensor_nbytes(type_id, elements, &bytes))
            return gg_err(err, err_len, "gguf_parse: tensor %.*s has unsupported GGUF type %u", shown,
                          (const char*)name, type_id),
                   0;
        qw35_hip_tensor_desc& o = all[(size_t)i];
        o.name = name;
        o.name_len = (uintptr_t)name_len;
        for (int d = 0; d < 4; ++d) o.dims[d] = d < (int)ndim ? dims[d] : 1;
        o.n_dims = ndim;
        o.type_id = type_id;
        o.abs_offset = rel;  // relative until the data section is known
        o.bytes = bytes;
        o.elements = elements;
    }
    const uint64_t rem = c.pos % alignment;
    const uint64_t data_pos = rem ? c.pos + (alignment - rem) : c.pos;
    for (qw35_hip_tensor_desc& o : all) {
        const int shown = (int)(o.name_len < 96 ? o.name_len : 96);
        if (o.abs_offset > UINT64_MAX - data_pos)
            return gg_err(err, err_len, "gguf_parse: tensor %.*s offset overflow", shown, (const char*)o.name), 0;
        o.abs_offset += data_pos;
        if (o.bytes != 0 && (o.abs_offset > model_size || o.bytes > model_size - o.abs_offset))
            return gg_err(err, err_len, "gguf_parse: tensor %.*s points outside GGUF file", shown,
                          (const char*)o.name),
                   0;
    }
    if (out)
        for (uint64_t i = 0; i < nt && i < cap; ++i) out[i] = all[(size_t)i];
    *n_tensors = (uint32_t)nt;
    if (data_offset) *data_offset = data_pos;
    return 1;
}

namespace {

// The descriptors a store was made from, field for field (names by their bytes).
bool same_descs(const Store* s, const qw35_hip_tensor_desc* descs, uint32_t count) {
    if (s->count != count) return false;
    for (uint32_t i = 0; i < count; ++i) {
        const qw35_hip_tensor_desc& a = s->descs[i];
        const qw35_hip_tensor_desc& b = descs[i];
        const uintptr_t blen = b.name ? b.name_len : 0;
        if (a.type_id != b.type_id || a.abs_offset != b.abs_offset || a.bytes != b.bytes ||
            a.elements != b.elements || a.n_dims != b.n_dims || memcmp(a.dims, b.dims, sizeof a.dims) != 0 ||
            s->names[i].size() != blen || (blen && memcmp(s->names[i].data(), b.name, blen) != 0))
            return false;
    }
    return true;
}

}  // namespace

void* qw35_hip_store_create(const void* model_map, uint64_t model_size, const qw35_hip_tensor_desc* descs,
                            uint32_t count, char* err, uintptr_t err_len) {
    if (!model_map || (!descs && count)) {
        gg_err(err, err_len, "store_create: null model image or descriptors");
        return nullptr;
    }
    uint64_t end = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const qw35_hip_tensor_desc& d = descs[i];
        if (d.abs_offset > model_size || d.bytes > model_size - d.abs_offset) {
            gg_err(err, err_len, "store_create: tensor %u points outside the model image", i);
            return nullptr;
        }
        if (d.abs_offset + d.bytes > end) end = d.abs_offset + d.bytes;
    }
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess) {
        (void)hipGetLastError();
        gg_err(err, err_len, "store_create: no current HIP device");
        return nullptr;
    }
    // Creation runs under the lock, so two first users of one image copy it once.
    std::lock_guard<std::mutex> lock(g_stores_mu);
    for (Store* o : g_stores) {
        // shared only with the same image, device and descriptors; other
        // descriptors over the same image get a store of their own
        if (o->map == model_map && o->map_size == model_size && o->device == device && same_descs(o, descs, count)) {
            ++o->refs;
            return o;
        }
    }
    Store* s = new (std::nothrow) Store();
    if (!s) {
        gg_err(err, err_len, "store_create: out of host memory");
        return nullptr;
    }
    s->map = model_map;
    s->map_size = model_size;
    s->count = count;
    s->device = device;
    s->bytes = end;
    if (end) {
        hipError_t e = hipMalloc(&s->dev, end);
        if (e == hipSuccess) e = hipMemcpy(s->dev, model_map, end, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            gg_err(err, err_len, "store_create: %llu device bytes: %s", (unsigned long long)end, hipGetErrorString(e));
            store_free(s);
            return nullptr;
        }
    }
    try {
        s->names.reserve(count);
        s->descs.assign(descs, descs + count);
        for (uint32_t i = 0; i < count; ++i) {
            s->names.emplace_back(reinterpret_cast<const char*>(descs[i].name),
                                  descs[i].name ? descs[i].name_len : 0);
            s->descs[i].name = reinterpret_cast<const uint8_t*>(s->names.back().data());
            s->index.emplace(s->names.back(), i);  // the first of duplicate names wins
        }
        g_stores.push_back(s);
    } catch (...) {
        gg_err(err, err_len, "store_create: out of host memory");
        store_free(s);
        return nullptr;
    }
    s->refs = 1;
    return s;
}

const void* qw35_hip_store_device_base(const void* store) { return store ? static_cast<const Store*>(store)->dev : nullptr; }

uint64_t qw35_hip_store_bytes(const void* store) { return store ? static_cast<const Store*>(store)->bytes : 0; }

int qw35_hip_store_weight(const void* store, const char* name, uintptr_t name_len, qw35_hip_weight* out, char* err,
                          uintptr_t err_len) {
    if (!store || !name || !out) {
        gg_err(err, err_len, "store_weight: null store, name or output");
        return 0;
    }
    const Store* s = static_cast<const Store*>(store);
    const auto it = s->index.find(std::string(name, name_len));
    if (it != s->index.end()) return qw35_hip_weight_view(&s->descs[it->second], s->dev, out, err, err_len);
    gg_err(err, err_len, "store_weight: no tensor named %.*s", (int)(name_len < 96 ? name_len : 96), name);
    return 0;
}

void qw35_hip_store_destroy(void* store) {
    Store* s = static_cast<Store*>(store);
    if (!s) return;
    std::lock_guard<std::mutex> lock(g_stores_mu);
    if (--s->refs > 0) return;
    for (size_t i = 0; i < g_stores.size(); ++i)
        if (g_stores[i] == s) {
            g_stores.erase(g_stores.begin() + (ptrdiff_t)i);
            break;
        }
    store_free(s);
}

}  // extern "C"
