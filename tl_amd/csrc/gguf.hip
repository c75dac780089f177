// GGUF files: the tensor map of tl_gguf_load (crates/tl_runtime/src/gguf.rs:34-196) with the
// accessors of crates/tl_runtime/src/tensor_map.rs, and the residency path of the quantized
// weights: blocks go from the memory-mapped file straight into the device format (one
// upload, no f32 caches; the reference copies each tensor to a Vec and caches an f32 and a
// transposed f32 copy, quantized.rs:117-165).
//
// File layout read here (GGUF v2 / v3; "GGUF" little-endian, "FUGG" big-endian header):
//   magic u32, version u32, tensor_count u64, kv_count u64,
//   kv_count x (key string, value type u32, value),
//   tensor_count x (name string, n_dims u32, ne u64[n_dims], ggml type u32, offset u64),
//   padding to general.alignment (default 32), tensor data (offsets relative to its start).
// A string is a u64 length + bytes.  Shapes follow gguf.rs:129-136: trailing 1s trimmed,
// ne reversed to the row-major [.., N, K].  Types follow gguf.rs:157-168: F32, F16, Q4_0,
// Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q4_K, Q6_K are kept, other types are skipped; a tensor whose
// data runs past the end of the file is skipped (gguf.rs:177-182).  Data bytes are used as
// stored, in either byte order, as the reference does.
#include "internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace tlhip {

struct GgufTensor {
    std::string name;
    int type = 0;
    int rank = 0;
    int64_t shape[TL_HIP_MAX_RANK] = {0};  // row-major (reversed ne)
    uint64_t offset = 0;                   // absolute file offset
    uint64_t nbytes = 0;
    QWeight* q = nullptr;                  // device residency, uploaded on first request
};

struct GgufMeta {
    int vtype = 0;  // GGUF value type
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
};

struct Gguf {
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<GgufTensor> tensors;
    std::map<std::string, size_t> index;
    std::map<std::string, GgufMeta> meta;
};

// bytes per block and weights per block of the GGML types the reference maps (gguf.rs:157-168)
static bool type_geometry(int t, int* elems, int* bytes) {
    switch (t) {
        case 0: *elems = 1; *bytes = 4; return true;     // F32
        case 1: *elems = 1; *bytes = 2; return true;     // F16
        case 2: *elems = 32; *bytes = 18; return true;   // Q4_0
        case 3: *elems = 32; *bytes = 20; return true;   // Q4_1
        case 6: *elems = 32; *bytes = 22; return true;   // Q5_0
        case 7: *elems = 32; *bytes = 24; return true;   // Q5_1
        case 8: *elems = 32; *bytes = 34; return true;   // Q8_0
        case 9: *elems = 32; *bytes = 36; return true;   // Q8_1
        case 12: *elems = 256; *bytes = 144; return true;  // Q4_K
        case 14: *elems = 256; *bytes = 210; return true;  // Q6_K
        default: return false;
    }
}

namespace {
// Bounds-checked reader over the mapped header.
struct Reader {
    const uint8_t* p;
    size_t size, pos = 0;
    bool swap, ok = true;
    bool need(size_t n) {
        if (!ok || pos + n > size || pos + n < pos) ok = false;
        return ok;
    }
    uint64_t uint(int n) {
        if (!need((size_t)n)) return 0;
        uint64_t v = 0;
        for (int i = 0; i < n; i++) {
            const int b = swap ? n - 1 - i : i;  // little-endian unless the header is big-endian
            v |= (uint64_t)p[pos + b] << (8 * i);
        }
        pos += (size_t)n;
        return v;
    }
    std::string str() {
        const uint64_t n = uint(8);
        if (!need((size_t)n)) return std::string();
        std::string s(reinterpret_cast<const char*>(p + pos), (size_t)n);
        pos += (size_t)n;
        return s;
    }
};

// scalar GGUF value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
// 9 array, 10 u64, 11 i64, 12 f64
int scalar_width(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

bool read_value(Reader& r, uint32_t t, GgufMeta* m, int depth) {
    if (t == 8) {
        std::string s = r.str();
        if (m) m->s = s;
        return r.ok;
    }
    if (t == 9) {
        if (depth > 4) return false;
        const uint32_t et = (uint32_t)r.uint(4);
        const uint64_t n = r.uint(8);
        const int w = scalar_width(et);
        if (w && n <= r.size) {  // fixed-width elements: skip in one step
            if (!r.need((size_t)(n * (uint64_t)w))) return false;
            r.pos += (size_t)(n * (uint64_t)w);
            return true;
        }
        if (et != 8 && et != 9) return false;
        for (uint64_t i = 0; i < n && r.ok; i++)
            if (!read_value(r, et, nullptr, depth + 1)) return false;
        return r.ok;
    }
    const int w = scalar_width(t);
    if (!w) return false;
    const uint64_t raw = r.uint(w);
    if (m) {
        m->u = raw;
        switch (t) {
            case 1: m->i = (int8_t)raw; break;
            case 3: m->i = (int16_t)raw; break;
            case 5: m->i = (int32_t)raw; break;
            case 11: m->i = (int64_t)raw; break;
            default: m->i = (int64_t)raw; break;
        }
        if (t == 6) {
            float f;
            uint32_t b = (uint32_t)raw;
            std::memcpy(&f, &b, 4);
            m->f = f;
        } else if (t == 12) {
            std::memcpy(&m->f, &raw, 8);
        } else {
            m->f = (t == 1 || t == 3 || t == 5 || t == 11) ? (double)m->i : (double)raw;
        }
    }
    return r.ok;
}
}  // namespace

__global__ void k_gguf_f16(const __half* __restrict__ in, float* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __half2float(in[i]);
}

static Gguf* G(tl_hip_gguf* h) { return reinterpret_cast<Gguf*>(h); }
static const Gguf* G(const tl_hip_gguf* h) { return reinterpret_cast<const Gguf*>(h); }

static const GgufTensor* find(const Gguf* g, const char* name) {
    if (!name) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tensor name");
        return nullptr;
    }
    auto it = g->index.find(name);
    if (it == g->index.end()) {
        // tensor_map.rs:144-148 / 298
        set_error(TL_HIP_ERR_ARG, "ArgumentError: Weight '%s' not found in loaded file.", name);
        return nullptr;
    }
    return &g->tensors[it->second];
}

static void unmap(Gguf* g) {
    if (g->map) munmap(const_cast<uint8_t*>(g->map), g->size);
    g->map = nullptr;
}

}  // namespace tlhip

using namespace tlhip;

extern "C" {

tl_hip_gguf* tl_hip_gguf_open(const char* path) {
    if (!path) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: path");
        return nullptr;
    }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: Failed to open GGUF file %s", path);  // gguf.rs:46-52
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 4) {
        close(fd);
        set_error(TL_HIP_ERR_ARG, "ArgumentError: File too small");  // gguf.rs:62-65
        return nullptr;
    }
    void* mp = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (mp == MAP_FAILED) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: Failed to mmap GGUF file");
        return nullptr;
    }
    Gguf* g = new Gguf();
    g->map = static_cast<const uint8_t*>(mp);
    g->size = (size_t)st.st_size;
    auto fail = [&](const char* what) -> tl_hip_gguf* {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: Failed to decode GGUF: %s", what);  // gguf.rs:94-100
        unmap(g);
        delete g;
        return nullptr;
    };
    bool swap;
    if (std::memcmp(g->map, "GGUF", 4) == 0) swap = false;       // gguf.rs:66-74
    else if (std::memcmp(g->map, "FUGG", 4) == 0) swap = true;
    else return fail("invalid GGUF magic");
    Reader r{g->map, g->size, 4, swap};
    g->version = (uint32_t)r.uint(4);
    if (g->version != 2 && g->version != 3) return fail("unsupported GGUF version (2 and 3 are read)");
    const uint64_t n_tensors = r.uint(8), n_kv = r.uint(8);
    if (!r.ok || n_tensors > g->size || n_kv > g->size) return fail("truncated header");
    for (uint64_t i = 0; i < n_kv; i++) {
        const std::string key = r.str();
        const uint32_t t = (uint32_t)r.uint(4);
        GgufMeta m;
        m.vtype = (int)t;
        if (!r.ok || !read_value(r, t, &m, 0)) return fail("bad metadata value");
        g->meta[key] = m;
    }
    auto al = g->meta.find("general.alignment");  // gguf.rs:108-113 (default 32)
    if (al != g->meta.end() && al->second.vtype != 8 && al->second.vtype != 9 && al->second.u > 0)
        g->alignment = al->second.u;
    struct Raw {
        std::string name;
        uint32_t nd;
        uint64_t ne[8];
        uint32_t type;
        uint64_t off;
    };
    std::vector<Raw> raws;
    raws.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Raw t;
        t.name = r.str();
        t.nd = (uint32_t)r.uint(4);
        if (!r.ok || t.nd > 8) return fail("bad tensor info");
        for (uint32_t d = 0; d < t.nd; d++) t.ne[d] = r.uint(8);
        t.type = (uint32_t)r.uint(4);
        t.off = r.uint(8);
        if (!r.ok) return fail("truncated tensor info");
        raws.push_back(t);
    }
    const uint64_t meta_end = r.pos;  // gguf.rs:102-117
    g->data_offset = meta_end + (g->alignment - meta_end % g->alignment) % g->alignment;
    for (const Raw& t : raws) {
        int elems, bytes;
        if (!type_geometry((int)t.type, &elems, &bytes)) {
            fprintf(stderr, "[tl_hip_gguf_open] Skipping tensor '%s': unsupported type kind=%u\n", t.name.c_str(),
                    t.type);  // gguf.rs:170-176
            continue;
        }
        std::vector<int64_t> shape;
        uint64_t numel = 1;
        bool overflow = false;
        for (uint32_t d = 0; d < t.nd; d++) {
            shape.push_back((int64_t)t.ne[d]);
            if (t.ne[d] && numel > UINT64_MAX / t.ne[d]) overflow = true;
            numel *= t.ne[d];
        }
        while (shape.size() > 1 && shape.back() == 1) shape.pop_back();  // gguf.rs:129-133
        if (t.nd == 0 || overflow || shape.size() > TL_HIP_MAX_RANK || numel % (uint64_t)elems) {
            fprintf(stderr, "[tl_hip_gguf_open] Skipping tensor '%s': bad shape\n", t.name.c_str());
            continue;
        }
        GgufTensor gt;
        gt.name = t.name;
        gt.type = (int)t.type;
        gt.rank = (int)shape.size();
        for (int d = 0; d < gt.rank; d++) gt.shape[d] = shape[gt.rank - 1 - d];  // gguf.rs:134-136
        gt.nbytes = numel / (uint64_t)elems * (uint64_t)bytes;
        gt.offset = g->data_offset + t.off;
        if (gt.offset < g->data_offset || gt.offset + gt.nbytes > g->size || gt.offset + gt.nbytes < gt.offset) {
            fprintf(stderr, "Error: Tensor %s data out of bounds\n", t.name.c_str());  // gguf.rs:177-182
            continue;
        }
        g->index[gt.name] = g->tensors.size();
        g->tensors.push_back(gt);
    }
    return reinterpret_cast<tl_hip_gguf*>(g);
}

int tl_hip_gguf_close(tl_hip_gguf* h) {
    if (!h) return TL_HIP_OK;
    Gguf* g = G(h);
    for (auto& t : g->tensors)
        if (t.q) tl_hip_qtensor_release(reinterpret_cast<tl_hip_qtensor*>(t.q));
    unmap(g);
    delete g;
    return TL_HIP_OK;
}

int64_t tl_hip_gguf_tensor_count(const tl_hip_gguf* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf");
        return -1;
    }
    return (int64_t)G(h)->tensors.size();
}

const char* tl_hip_gguf_tensor_name(const tl_hip_gguf* h, int64_t i) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf");
        return nullptr;
    }
    const Gguf* g = G(h);
    if (i < 0 || i >= (int64_t)g->tensors.size()) {
        set_error(TL_HIP_ERR_INDEX, "IndexOutOfBounds: tensor %lld of %zu", (long long)i, g->tensors.size());
        return nullptr;
    }
    return g->tensors[(size_t)i].name.c_str();
}

int tl_hip_gguf_tensor_info(const tl_hip_gguf* h, const char* name, int* ggml_type, int64_t* shape, int* rank,
                            uint64_t* nbytes) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf");
        return TL_HIP_ERR_NULL;
    }
    const GgufTensor* t = find(G(h), name);
    if (!t) return TL_HIP_ERR_ARG;
    if (ggml_type) *ggml_type = t->type;
    if (rank) *rank = t->rank;
    if (shape)
        for (int d = 0; d < t->rank; d++) shape[d] = t->shape[d];
    if (nbytes) *nbytes = t->nbytes;
    return TL_HIP_OK;
}

const uint8_t* tl_hip_gguf_tensor_data(const tl_hip_gguf* h, const char* name, uint64_t* nbytes) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf");
        return nullptr;
    }
    const GgufTensor* t = find(G(h), name);
    if (!t) return nullptr;
    if (nbytes) *nbytes = t->nbytes;
    return G(h)->map + t->offset;
}

int tl_hip_gguf_meta_f64(const tl_hip_gguf* h, const char* key, double* out) {
    if (!h || !key || !out) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf, key or output");
        return TL_HIP_ERR_NULL;
    }
    auto it = G(h)->meta.find(key);
    if (it == G(h)->meta.end() || it->second.vtype == 8 || it->second.vtype == 9) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: no numeric metadata '%s'", key);
        return TL_HIP_ERR_ARG;
    }
    *out = it->second.f;
    return TL_HIP_OK;
}

const char* tl_hip_gguf_meta_str(const tl_hip_gguf* h, const char* key) {
    if (!h || !key) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf or key");
        return nullptr;
    }
    auto it = G(h)->meta.find(key);
    if (it == G(h)->meta.end() || it->second.vtype != 8) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: no string metadata '%s'", key);
        return nullptr;
    }
    return it->second.s.c_str();
}

tl_hip_qtensor* tl_hip_gguf_get_quantized(tl_hip_gguf* h, const char* name) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf");
        return nullptr;
    }
    Gguf* g = G(h);
    const GgufTensor* ct = find(g, name);
    if (!ct) return nullptr;
    GgufTensor* t = &g->tensors[g->index[ct->name]];
    if (!t->q) {
        tl_hip_qtensor* q = tl_hip_qtensor_new(t->type, g->map + t->offset, (size_t)t->nbytes, t->shape, t->rank);
        if (!q) return nullptr;
        t->q = Q(q);
    }
    t->q->refs.fetch_add(1);  // the caller's reference (Arc::clone, tensor_map.rs:293-296)
    return reinterpret_cast<tl_hip_qtensor*>(t->q);
}

tl_hip_tensor* tl_hip_gguf_get(tl_hip_gguf* h, const char* name) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: gguf");
        return nullptr;
    }
    Gguf* g = G(h);
    const GgufTensor* t = find(g, name);
    if (!t) return nullptr;
    if (t->type == TL_HIP_GGML_F32)
        return tl_hip_tensor_new(reinterpret_cast<const float*>(g->map + t->offset), t->shape, t->rank);
    if (t->type == TL_HIP_GGML_F16) {  // QTensor::dequantize_f16 (quantized.rs:167-180)
        Tensor* o = tensor_alloc(t->shape, t->rank, TL_HIP_F32);
        if (!o) return nullptr;
        hipStream_t s = cur_stream();
        __half* tmp = o->numel ? (__half*)dev_alloc((size_t)o->numel * 2) : nullptr;
        if (o->numel && !tmp) {
            tensor_drop(o);
            return nullptr;
        }
        hipError_t e = hipSuccess;
        if (o->numel) {
            e = hipMemcpyAsync(tmp, g->map + t->offset, (size_t)o->numel * 2, hipMemcpyHostToDevice, s);
            if (e == hipSuccess) {
                k_gguf_f16<<<cdiv(o->numel, 256), 256, 0, s>>>(tmp, o->f32(), o->numel);
                e = hipGetLastError();
            }
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            dev_free(tmp);
        }
        if (e != hipSuccess) {
            hip_fail(e, "f16 tensor upload");
            tensor_drop(o);
            return nullptr;
        }
        return H(o);
    }
    // quantized: QTensor::dequantize_to_tensor (tensor_map.rs:130-142) through a 2-D residency
    // of the same bytes ([numel / last, last]), then the file's shape
    const int64_t last = t->shape[t->rank - 1];
    int64_t flat[2] = {1, last};
    for (int d = 0; d < t->rank - 1; d++) flat[0] *= t->shape[d];
    tl_hip_qtensor* q;
    if (t->rank == 2) {
        q = tl_hip_gguf_get_quantized(h, name);
    } else {
        q = tl_hip_qtensor_new(t->type, g->map + t->offset, (size_t)t->nbytes, flat, 2);
    }
    if (!q) return nullptr;
    tl_hip_tensor* out = tl_hip_qtensor_dequantize(q);
    tl_hip_qtensor_release(q);
    if (out && t->rank != 2) {
        tl_hip_tensor* r = tl_hip_tensor_reshape(out, t->shape, t->rank);
        tl_hip_tensor_release(out);
        out = r;
    }
    return out;
}

}  // extern "C"
