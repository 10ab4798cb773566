// gguf_file.cpp - GGUF checkpoints straight into device buffers: the
// reference's parser (gguf_parse, lib/gguf/parser.c3:164-208, with its reader
// helpers :12-162) and upload_weight (lib/model/tensor.c3:48-66).
//
// The file is memory-mapped read-only; the header, the metadata key/values
// and the tensor infos are parsed once at open; tensor bytes are copied to
// the device unchanged (quantized blocks stay in their GGUF layout, which is
// what the GEMM kernels read). Unlike the reference, every read is checked
// against the file size, so a truncated or corrupt file is an error rather
// than a read past the mapping. Host code only.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "llmr_hip.h"

namespace llmr {
int set_error(int code, const char* msg);  // capi.hip: records llmr_last_error
}

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" (types.c3:6)
constexpr uint64_t kGgufAlignment = 32;        // hard-coded data alignment (types.c3:8)

int ok() { return llmr::set_error(LLMR_OK, ""); }

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return llmr::set_error(code, buf);
}

// GGMLType.block_size / type_size (types.c3:50-98): elements per block and
// bytes per block; unknown types give a zero size, as in the reference.
void ggml_block(uint32_t t, uint64_t& bs, uint64_t& ts) {
    switch (t) {
        case 0: bs = 1; ts = 4; return;      // F32
        case 1: bs = 1; ts = 2; return;      // F16
        case 2: bs = 32; ts = 18; return;    // Q4_0
        case 3: bs = 32; ts = 20; return;    // Q4_1
        case 6: bs = 32; ts = 22; return;    // Q5_0
        case 7: bs = 32; ts = 24; return;    // Q5_1
        case 8: bs = 32; ts = 34; return;    // Q8_0
        case 9: bs = 32; ts = 36; return;    // Q8_1
        case 10: bs = 256; ts = 84; return;  // Q2_K
        case 11: bs = 256; ts = 110; return; // Q3_K
        case 12: bs = 256; ts = 144; return; // Q4_K
        case 13: bs = 256; ts = 176; return; // Q5_K
        case 14: bs = 256; ts = 210; return; // Q6_K
        case 24: bs = 1; ts = 1; return;     // I8
        case 25: bs = 1; ts = 2; return;     // I16
        case 26: bs = 1; ts = 4; return;     // I32
        case 27: bs = 1; ts = 8; return;     // I64
        case 28: bs = 1; ts = 8; return;     // F64
        case 30: bs = 1; ts = 2; return;     // BF16
        default: bs = 32; ts = 0; return;
    }
}

// Byte size of one scalar metadata value of GGUFType t (types.c3:11-25);
// 0 for STRING (8) and ARRAY (9), which carry their own lengths.
uint64_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;   // UINT8, INT8, BOOL
        case 2: case 3: return 2;           // UINT16, INT16
        case 4: case 5: case 6: return 4;   // UINT32, INT32, FLOAT32
        case 10: case 11: case 12: return 8;  // UINT64, INT64, FLOAT64
        default: return 0;
    }
}

struct Kv {
    std::string key;
    uint32_t type, array_type;
    uint64_t array_len, data_off, data_len;
};
struct Tensor {
    std::string name;
    uint32_t type, n_dims;
    uint64_t ne[4], offset, data_size;
};

// Bounds-checked little-endian reader over the mapping.
struct Reader {
    const uint8_t* p;
    uint64_t size, pos;
    bool ok;
    bool need(uint64_t n) {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return {};
        std::string s((const char*)p + pos, (size_t)n);
        pos += n;
        return s;
    }
    void skip(uint64_t n) {
        if (need(n)) pos += n;
    }
    // a value of type t (arrays nested as in GGUFReader.skip_value)
    void skip_value(uint32_t t, int depth = 0) {
        if (t == 8) {
            const uint64_t n = get<uint64_t>();
            skip(n);
        } else if (t == 9) {
            const uint32_t at = get<uint32_t>();
            const uint64_t n = get<uint64_t>();
            if (depth > 4) ok = false;
            if (scalar_size(at)) {
                if (n > (size - pos) / scalar_size(at)) ok = false;
                else skip(n * scalar_size(at));
            } else {
                for (uint64_t i = 0; ok && i < n; i++) skip_value(at, depth + 1);
            }
        } else if (scalar_size(t)) {
            skip(scalar_size(t));
        } else {
            ok = false;  // unknown value type
        }
    }
};

}  // namespace

struct llmr_gguf {
    void* map;
    uint64_t size;
    uint32_t version;
    uint64_t data_base;  // file offset of the aligned tensor data section
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
};

extern "C" {

int llmr_gguf_open(const char* path, llmr_gguf** out) {
    if (!path || !out) return fail(LLMR_ERR_INVALID_ARG, "null path or output pointer");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(LLMR_ERR_INVALID_ARG, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail(LLMR_ERR_INVALID_ARG, "%s: too short for a GGUF header", path);
    }
    void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return fail(LLMR_ERR_INVALID_ARG, "cannot map %s", path);
    auto* f = new (std::nothrow) llmr_gguf{map, (uint64_t)st.st_size, 0, 0, {}, {}};
    if (!f) {
        munmap(map, (size_t)st.st_size);
        return fail(LLMR_ERR_INVALID_ARG, "out of host memory");
    }
    Reader r{(const uint8_t*)map, f->size, 0, true};
    auto bad = [&](const char* what) {
        const int e = fail(LLMR_ERR_INVALID_ARG, "%s: %s", path, what);
        llmr_gguf_close(f);
        return e;
    };
    if (r.get<uint32_t>() != kGgufMagic) return bad("not a GGUF file (bad magic)");
    f->version = r.get<uint32_t>();
    if (f->version < 2 || f->version > 3) return bad("unsupported GGUF version (2 and 3 are read)");
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    // every key/value and tensor info takes at least 12 bytes: a count beyond
    // the file is corrupt, not an allocation to attempt
    if (n_kv > f->size / 12 || n_tensors > f->size / 12) return bad("corrupt header counts");
    f->kv.reserve((size_t)n_kv);
    for (uint64_t i = 0; r.ok && i < n_kv; i++) {
        Kv k{};
        k.key = r.str();
        k.type = r.get<uint32_t>();
        if (k.type == 9) {
            k.array_type = r.get<uint32_t>();
            k.array_len = r.get<uint64_t>();
            if (!r.ok) break;
            k.data_off = r.pos;
            // re-read the array body by skipping it as a whole value
            r.pos -= 12;
            r.skip_value(9);
            k.data_len = r.pos - k.data_off;
        } else if (k.type == 8) {
            k.data_len = r.get<uint64_t>();
            k.data_off = r.pos;
            r.skip(k.data_len);
        } else {
            k.data_off = r.pos;
            k.data_len = scalar_size(k.type);
            r.skip_value(k.type);
        }
        f->kv.push_back(std::move(k));
    }
    if (!r.ok) return bad("truncated or corrupt metadata");
    f->tensors.reserve((size_t)n_tensors);
    for (uint64_t i = 0; r.ok && i < n_tensors; i++) {
        Tensor t{};
        t.name = r.str();
        t.n_dims = r.get<uint32_t>();
        if (t.n_dims > 4) return bad("tensor with more than 4 dimensions");
        uint64_t n = 1;
        for (uint32_t d = 0; d < 4; d++) {
            t.ne[d] = d < t.n_dims ? r.get<uint64_t>() : 1;
            if (t.ne[d] && n > UINT64_MAX / t.ne[d]) return bad("tensor element count overflows");
            n *= t.ne[d];
        }
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        uint64_t bs, ts;
        ggml_block(t.type, bs, ts);
        // ceil(n / bs) * ts (parser.c3:149-158), without wrapping
        const uint64_t blocks = n / bs + (n % bs != 0);
        if (ts && blocks > UINT64_MAX / ts) return bad("tensor byte size overflows");
        t.data_size = blocks * ts;
        f->tensors.push_back(std::move(t));
    }
    if (!r.ok) return bad("truncated tensor infos");
    f->data_base = (r.pos + kGgufAlignment - 1) & ~(kGgufAlignment - 1);
    for (const Tensor& t : f->tensors)
        if (t.offset > f->size || f->data_base > f->size - t.offset ||
            t.data_size > f->size - f->data_base - t.offset)
            return bad(("tensor data outside the file: " + t.name).c_str());
    *out = f;
    return ok();
}

int llmr_gguf_close(llmr_gguf* f) {
    if (!f) return ok();
    if (f->map) munmap(f->map, (size_t)f->size);
    delete f;
    return ok();
}

int llmr_gguf_info(const llmr_gguf* f, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv) {
    if (!f) return fail(LLMR_ERR_INVALID_ARG, "null GGUF handle");
    if (version) *version = f->version;
    if (n_tensors) *n_tensors = f->tensors.size();
    if (n_kv) *n_kv = f->kv.size();
    return ok();
}

int llmr_gguf_tensor(const llmr_gguf* f, uint64_t index, llmr_gguf_tensor_info* out) {
    if (!f || !out) return fail(LLMR_ERR_INVALID_ARG, "null GGUF handle or output");
    if (index >= f->tensors.size()) return fail(LLMR_ERR_INVALID_ARG, "tensor index %llu out of range",
                                               (unsigned long long)index);
    const Tensor& t = f->tensors[index];
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->data_size = t.data_size;
    out->data = (const uint8_t*)f->map + f->data_base + t.offset;
    return ok();
}

int llmr_gguf_find_tensor(const llmr_gguf* f, const char* name, uint64_t* index) {
    if (!f || !name || !index) return fail(LLMR_ERR_INVALID_ARG, "null argument");
    for (uint64_t i = 0; i < f->tensors.size(); i++)
        if (f->tensors[i].name == name) {
            *index = i;
            return ok();
        }
    return fail(LLMR_ERR_INVALID_ARG, "no tensor named %s", name);
}

int llmr_gguf_kv(const llmr_gguf* f, uint64_t index, llmr_gguf_kv_info* out) {
    if (!f || !out) return fail(LLMR_ERR_INVALID_ARG, "null GGUF handle or output");
    if (index >= f->kv.size()) return fail(LLMR_ERR_INVALID_ARG, "metadata index %llu out of range",
                                          (unsigned long long)index);
    const Kv& k = f->kv[index];
    out->key = k.key.c_str();
    out->type = k.type;
    out->array_type = k.array_type;
    out->array_len = k.array_len;
    out->data = (const uint8_t*)f->map + k.data_off;
    out->data_len = k.data_len;
    return ok();
}

int llmr_gguf_find_kv(const llmr_gguf* f, const char* key, uint64_t* index) {
    if (!f || !key || !index) return fail(LLMR_ERR_INVALID_ARG, "null argument");
    for (uint64_t i = 0; i < f->kv.size(); i++)
        if (f->kv[i].key == key) {
            *index = i;
            return ok();
        }
    return fail(LLMR_ERR_INVALID_ARG, "no metadata key %s", key);
}

int llmr_gguf_upload_tensor(llmr_context* ctx, const llmr_gguf* f, uint64_t index, void* dst_dev,
                            size_t dst_bytes) {
    llmr_gguf_tensor_info t;
    if (int r = llmr_gguf_tensor(f, index, &t)) return r;
    if (t.data_size == 0) return fail(LLMR_ERR_UNSUPPORTED, "tensor %s: GGML type %u has no known size", t.name,
                                      t.type);
    if (!dst_dev || dst_bytes < t.data_size)
        return fail(LLMR_ERR_INVALID_ARG, "tensor %s needs %llu device bytes", t.name,
                    (unsigned long long)t.data_size);
    return llmr_upload(ctx, dst_dev, t.data, (size_t)t.data_size);
}

int llmr_gguf_load_tensor(llmr_context* ctx, const llmr_gguf* f, uint64_t index, void** out_dev_ptr) {
    llmr_gguf_tensor_info t;
    if (!out_dev_ptr) return fail(LLMR_ERR_INVALID_ARG, "null output pointer");
    *out_dev_ptr = nullptr;
    if (int r = llmr_gguf_tensor(f, index, &t)) return r;
    if (t.data_size == 0) return fail(LLMR_ERR_UNSUPPORTED, "tensor %s: GGML type %u has no known size", t.name,
                                      t.type);
    void* p = nullptr;
    if (int r = llmr_alloc(ctx, (size_t)t.data_size, &p)) return r;
    if (int r = llmr_upload(ctx, p, t.data, (size_t)t.data_size)) {
        (void)llmr_free(ctx, p);
        return r;
    }
    *out_dev_ptr = p;
    return ok();
}

}  // extern "C"
