/*
 * The model file on the device (include/q38_gguf.h): a GGUF reader with the
 * reference's checks (src/gguf/mod.rs), the streamed upload of its tensor
 * data into HBM, and the device-side checkpoint of the recurrent state
 * (src/model/ops.rs:1627-1647).
 */
#define __HIP_PLATFORM_AMD__ 1
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../../include/q38_bench.h"
#include "../../../include/q38_gguf.h"

/* the library's error slot (q38_attn.cpp) */
int q38_fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

namespace {

constexpr uint32_t kMagic = 0x46554747u; /* "GGUF" little-endian */

/* metadata value types (MetaType, mod.rs:32-46) */
enum : uint32_t { M_U8, M_I8, M_U16, M_I16, M_U32, M_I32, M_F32, M_BOOL, M_STRING, M_ARRAY, M_U64, M_I64, M_F64 };

uint64_t scalar_size(uint32_t t) {
    switch (t) {
    case M_U8: case M_I8: case M_BOOL: return 1;
    case M_U16: case M_I16: return 2;
    case M_U32: case M_I32: case M_F32: return 4;
    case M_U64: case M_I64: case M_F64: return 8;
    default: return 0;
    }
}

/* ggml types the reference knows, with (elements, bytes) per block
 * (GgmlType, mod.rs:81-179) */
bool ggml_block(uint32_t t, uint64_t &elems, uint64_t &bytes) {
    switch (t) {
    case 0: elems = 1; bytes = 4; return true;     /* F32 */
    case 1: elems = 1; bytes = 2; return true;     /* F16 */
    case 30: elems = 1; bytes = 2; return true;    /* BF16 */
    case 2: elems = 32; bytes = 18; return true;   /* Q4_0 */
    case 3: elems = 32; bytes = 20; return true;   /* Q4_1 */
    case 6: elems = 32; bytes = 22; return true;   /* Q5_0 */
    case 7: elems = 32; bytes = 24; return true;   /* Q5_1 */
    case 8: elems = 32; bytes = 34; return true;   /* Q8_0 */
    case 20: elems = 32; bytes = 18; return true;  /* IQ4_NL */
    case 10: elems = 256; bytes = 84; return true; /* Q2_K */
    case 11: elems = 256; bytes = 110; return true; /* Q3_K */
    case 12: elems = 256; bytes = 144; return true; /* Q4_K */
    case 13: elems = 256; bytes = 176; return true; /* Q5_K */
    case 14: elems = 256; bytes = 210; return true; /* Q6_K */
    case 16: elems = 256; bytes = 66; return true;  /* IQ2_XXS */
    case 17: elems = 256; bytes = 74; return true;  /* IQ2_XS */
    case 18: elems = 256; bytes = 98; return true;  /* IQ3_XXS */
    case 19: elems = 256; bytes = 50; return true;  /* IQ1_S */
    case 21: elems = 256; bytes = 110; return true; /* IQ3_S */
    case 22: elems = 256; bytes = 82; return true;  /* IQ2_S */
    case 23: elems = 256; bytes = 136; return true; /* IQ4_XS */
    case 29: elems = 256; bytes = 56; return true;  /* IQ1_M */
    default: return false;
    }
}

/* A bounds-checked little-endian cursor: a read past the end marks the
 * cursor failed and yields zero (Reader, mod.rs:219-306). */
struct Cursor {
    const uint8_t *base;
    size_t size, at = 0;
    bool failed = false;

    const uint8_t *take(uint64_t n) {
        if (failed) return nullptr;
        if (n > size - at) {
            failed = true;
            return nullptr;
        }
        const uint8_t *p = base + at;
        at += (size_t)n;
        return p;
    }
    template <typename T> T le() {
        const uint8_t *p = take(sizeof(T));
        T v = 0;
        if (p) memcpy(&v, p, sizeof(T)); /* the host is little-endian */
        return v;
    }
    bool string(const uint8_t *&data, uint64_t &len) {
        len = le<uint64_t>();
        if (failed) return false;
        data = take(len);
        return data != nullptr;
    }
    bool skip_values(uint32_t type, uint64_t count) {
        if (const uint64_t sz = scalar_size(type)) {
            if (count > UINT64_MAX / sz) return false;
            return take(count * sz) != nullptr;
        }
        if (type == M_STRING) {
            for (uint64_t i = 0; i < count; ++i) {
                const uint8_t *d;
                uint64_t n;
                if (!string(d, n)) return false;
            }
            return true;
        }
        return false;
    }
};

struct Meta {
    std::string key;
    uint32_t type, array_type;
    uint64_t count;
    const uint8_t *data;
    uint64_t len;
};

struct Tensor {
    std::string name;
    uint32_t n_dims, type;
    uint64_t shape[Q38_GGUF_MAX_DIMS];
    uint64_t offset, nbytes;
};

int invalid(const char *msg) { return q38_fail("invalid GGUF: %s", msg); }

}  // namespace

struct q38_gguf {
    void *map = nullptr;
    size_t size = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t data_offset = 0;
    std::vector<Meta> meta;
    std::vector<Tensor> tensors;

    ~q38_gguf() {
        if (map) munmap(map, size);
    }

    int parse() {
        Cursor r{static_cast<const uint8_t *>(map), size};
        const uint32_t magic = r.le<uint32_t>();
        version = r.le<uint32_t>();
        const uint64_t n_tensors = r.le<uint64_t>();
        const uint64_t n_meta = r.le<uint64_t>();
        if (magic != kMagic || version < 2 || version > 3 || n_tensors == 0)
            return invalid("unsupported or corrupt GGUF header");
        /* parse_metadata (mod.rs:347-409) */
        for (uint64_t i = 0; i < n_meta; ++i) {
            Meta m{};
            const uint8_t *kd;
            uint64_t kn;
            if (!r.string(kd, kn)) return invalid("metadata key");
            m.key.assign(reinterpret_cast<const char *>(kd), (size_t)kn);
            m.type = r.le<uint32_t>();
            if (r.failed) return invalid("metadata type");
            if (m.type > M_F64) return invalid("unknown meta type");
            m.array_type = UINT32_MAX;
            m.count = 1;
            if (m.type == M_STRING) {
                if (!r.string(m.data, m.len)) return invalid("meta string");
            } else if (m.type == M_ARRAY) {
                m.array_type = r.le<uint32_t>();
                if (m.array_type > M_F64) return invalid("unknown array type");
                if (m.array_type == M_ARRAY) return invalid("nested arrays not allowed");
                m.count = r.le<uint64_t>();
                const size_t start = r.at;
                if (!r.skip_values(m.array_type, m.count)) return invalid("array value");
                m.data = r.base + start;
                m.len = r.at - start;
            } else {
                m.len = scalar_size(m.type);
                m.data = r.take(m.len);
                if (!m.data) return invalid("scalar value");
            }
            meta.push_back(std::move(m));
        }
        /* parse_tensors (mod.rs:411-457) */
        for (uint64_t i = 0; i < n_tensors; ++i) {
            Tensor t{};
            const uint8_t *nd;
            uint64_t nn;
            if (!r.string(nd, nn)) return invalid("tensor name");
            t.name.assign(reinterpret_cast<const char *>(nd), (size_t)nn);
            t.n_dims = r.le<uint32_t>();
            if (r.failed || t.n_dims == 0 || t.n_dims > Q38_GGUF_MAX_DIMS) return invalid("tensor n_dims");
            uint64_t elements = 1;
            for (uint32_t d = 0; d < t.n_dims; ++d) {
                t.shape[d] = r.le<uint64_t>();
                if (t.shape[d] == 0 || elements > UINT64_MAX / t.shape[d]) return invalid("tensor shape overflow");
                elements *= t.shape[d];
            }
            t.type = r.le<uint32_t>();
            t.offset = r.le<uint64_t>();
            if (r.failed) return invalid("tensor trailer");
            uint64_t be, bb;
            if (!ggml_block(t.type, be, bb)) return invalid("unknown tensor type");
            if (t.shape[0] % be != 0 || elements % be != 0 || elements / be > UINT64_MAX / bb)
                return invalid("tensor bytes overflow");
            t.nbytes = elements / be * bb;
            tensors.push_back(std::move(t));
        }
        /* general.alignment (mod.rs:491-500) */
        for (const Meta &m : meta) {
            if (m.key != "general.alignment") continue;
            if (m.type == M_U32 && m.len == 4) {
                uint32_t declared;
                memcpy(&declared, m.data, 4);
                if (declared == 0 || (declared & (declared - 1)) != 0) return invalid("invalid GGUF alignment");
                alignment = declared;
            }
            break;
        }
        const uint64_t end = r.at, align = alignment;
        if (end > UINT64_MAX - (align - 1)) return invalid("data_offset overflow");
        data_offset = (end + align - 1) & ~(align - 1);
        if (data_offset > size) return invalid("tensor data begins past end of file");
        for (const Tensor &t : tensors) {
            if (t.offset > UINT64_MAX - data_offset) return invalid("tensor offset overflow");
            const uint64_t start = data_offset + t.offset;
            if (t.nbytes > UINT64_MAX - start) return invalid("tensor nbytes overflow");
            if (start + t.nbytes > size) return invalid("tensor outside GGUF file");
        }
        return 0;
    }
};

extern "C" {

int q38_gguf_open(const char *path, q38_gguf **out) {
    if (path == nullptr || out == nullptr) return q38_fail("NULL argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return q38_fail("I/O error: cannot open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        close(fd);
        return q38_fail("I/O error: %s", strerror(e));
    }
    if (st.st_size < 24) {
        close(fd);
        return invalid("file smaller than 24 bytes");
    }
    void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    const int e = errno;
    close(fd);
    if (map == MAP_FAILED) return q38_fail("I/O error: mmap: %s", strerror(e));
    q38_gguf *g = new q38_gguf;
    g->map = map;
    g->size = (size_t)st.st_size;
    if (g->parse() != 0) {
        delete g;
        return -1;
    }
    *out = g;
    return 0;
}

int q38_gguf_close(q38_gguf *g) {
    delete g;
    return 0;
}

int q38_gguf_info(const q38_gguf *g, uint32_t *version, uint32_t *alignment, uint64_t *data_offset, int *n_tensors,
                  int *n_metadata) {
    if (g == nullptr) return q38_fail("gguf is NULL");
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (n_tensors) *n_tensors = (int)g->tensors.size();
    if (n_metadata) *n_metadata = (int)g->meta.size();
    return 0;
}

int q38_gguf_find_tensor(const q38_gguf *g, const char *name, int *index) {
    if (g == nullptr || name == nullptr || index == nullptr) return q38_fail("NULL argument");
    for (size_t i = 0; i < g->tensors.size(); ++i)
        if (g->tensors[i].name == name) {
            *index = (int)i;
            return 0;
        }
    return q38_fail("tensor %s not found", name);
}

int q38_gguf_tensor(const q38_gguf *g, int index, const char **name, int *ggml_type, int *n_dims,
                    uint64_t shape[Q38_GGUF_MAX_DIMS], uint64_t *offset, uint64_t *nbytes) {
    if (g == nullptr) return q38_fail("gguf is NULL");
    if (index < 0 || (size_t)index >= g->tensors.size())
        return q38_fail("tensor index %d outside [0, %zu)", index, g->tensors.size());
    const Tensor &t = g->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = (int)t.type;
    if (n_dims) *n_dims = (int)t.n_dims;
    if (shape)
        for (int d = 0; d < Q38_GGUF_MAX_DIMS; ++d) shape[d] = d < (int)t.n_dims ? t.shape[d] : 0;
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return 0;
}

int q38_gguf_meta_u32(const q38_gguf *g, const char *key, uint32_t *value) {
    if (g == nullptr || key == nullptr || value == nullptr) return q38_fail("NULL argument");
    for (const Meta &m : g->meta) {
        if (m.key != key) continue;
        if (m.type != M_U32 || m.len != 4) return q38_fail("metadata %s is not a Uint32", key);
        memcpy(value, m.data, 4);
        return 0;
    }
    return q38_fail("metadata %s not found", key);
}

int q38_gguf_upload(q38_ctx *ctx, const q38_gguf *g, void **d_base, size_t *bytes) {
    if (ctx == nullptr || g == nullptr || d_base == nullptr) return q38_fail("NULL argument");
    uint64_t extent = 0;
    for (const Tensor &t : g->tensors) extent = std::max(extent, t.offset + t.nbytes);
    void *dst = nullptr;
    if (q38_alloc(ctx, (size_t)extent, &dst) != 0) return -1;
    /* two pinned staging buffers: while one is copied to the device, the
     * other is filled from the mapping */
    constexpr size_t kChunk = (size_t)32 << 20;
    hipStream_t stream = static_cast<hipStream_t>(q38_ctx_stream(ctx));
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = 0;
    auto cleanup = [&]() {
        (void)hipStreamSynchronize(stream);
        for (int i = 0; i < 2; ++i) {
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (stage[i]) (void)hipHostFree(stage[i]);
        }
    };
    auto check = [&](hipError_t e, const char *what) {
        if (e != hipSuccess && rc == 0) rc = q38_fail("%s: %s", what, hipGetErrorString(e));
        return e == hipSuccess;
    };
    for (int i = 0; i < 2 && rc == 0; ++i) {
        check(hipHostMalloc(&stage[i], kChunk, hipHostMallocDefault), "hipHostMalloc");
        if (rc == 0) check(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "hipEventCreate");
    }
    const uint8_t *src = static_cast<const uint8_t *>(g->map) + g->data_offset;
    for (uint64_t off = 0, k = 0; rc == 0 && off < extent; off += kChunk, ++k) {
        const int b = (int)(k & 1);
        const size_t n = (size_t)std::min<uint64_t>(kChunk, extent - off);
        if (k >= 2 && !check(hipEventSynchronize(done[b]), "hipEventSynchronize")) break;
        memcpy(stage[b], src + off, n);
        if (!check(hipMemcpyAsync(static_cast<uint8_t *>(dst) + off, stage[b], n, hipMemcpyHostToDevice, stream),
                   "hipMemcpyAsync"))
            break;
        check(hipEventRecord(done[b], stream), "hipEventRecord");
    }
    cleanup();
    if (rc != 0) {
        q38_free(ctx, dst);
        return rc;
    }
    *d_base = dst;
    if (bytes) *bytes = (size_t)extent;
    return 0;
}

static int state_copy(q38_ctx *ctx, const float *a, const float *b, size_t na, size_t nb, float *da, float *db) {
    if (ctx == nullptr || a == nullptr || b == nullptr || da == nullptr || db == nullptr)
        return q38_fail("NULL argument");
    if (na % 4 != 0 || nb % 4 != 0) return q38_fail("state lengths %zu and %zu must be multiples of 4", na, nb);
    if (((uintptr_t)a | (uintptr_t)b | (uintptr_t)da | (uintptr_t)db) % 16 != 0)
        return q38_fail("state buffers must be 16-byte aligned");
    if (q38_device_copy(ctx, da, a, na * 4) != 0) return -1;
    return q38_device_copy(ctx, db, b, nb * 4);
}

int q38_recurrent_checkpoint(q38_ctx *ctx, const float *d_conv_state, const float *d_delta_state, size_t n_conv,
                             size_t n_delta, float *d_conv_ckpt, float *d_delta_ckpt) {
    return state_copy(ctx, d_conv_state, d_delta_state, n_conv, n_delta, d_conv_ckpt, d_delta_ckpt);
}

int q38_recurrent_restore(q38_ctx *ctx, const float *d_conv_ckpt, const float *d_delta_ckpt, size_t n_conv,
                          size_t n_delta, float *d_conv_state, float *d_delta_state) {
    return state_copy(ctx, d_conv_ckpt, d_delta_ckpt, n_conv, n_delta, d_conv_state, d_delta_state);
}

}  /* extern "C" */
