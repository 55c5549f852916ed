// GGUF reader; see gguf.h.  Error texts mirror error.rs:3-49 of the
// reference so C-ABI callers see the same messages.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <stdexcept>

#include "oxb_common.h"

namespace oxb {

namespace {

struct ParseError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct Reader {
    const uint8_t *p;
    size_t n, off = 0;
    void need(uint64_t k) {
        if (k > n - off) {  // off <= n always; this form cannot wrap
            char buf[160];
            snprintf(buf, sizeof buf,
                     "GGUF parse error: Unexpected EOF at offset %zu (need %llu bytes, have %zu)",
                     off, (unsigned long long)k, n);
            throw ParseError(buf);
        }
    }
    template <class T>
    T rd() {
        need(sizeof(T));
        T v;
        memcpy(&v, p + off, sizeof(T));
        off += sizeof(T);
        return v;
    }
    std::string str() {
        uint64_t len = rd<uint64_t>();
        need(len);
        std::string s((const char *)p + off, (size_t)len);
        off += len;
        return s;
    }
};

// Smallest encoding of one value of each metadata type (a string is its u64
// length, an array its u32 type + u64 length); 0 for unknown types.
uint64_t min_value_bytes(uint32_t ty) {
    static const uint8_t kMin[13] = {1, 1, 2, 2, 4, 4, 4, 1, 8, 12, 8, 8, 8};
    return ty < 13 ? kMin[ty] : 0;
}

GgufValue read_value(Reader &r, uint32_t ty, int depth = 0) {
    GgufValue v;
    switch (ty) {
        case 0: v.kind = GgufValue::U64; v.u = r.rd<uint8_t>(); break;
        case 1: v.kind = GgufValue::I64; v.i = r.rd<int8_t>(); v.u = (uint64_t)v.i; break;
        case 2: v.kind = GgufValue::U64; v.u = r.rd<uint16_t>(); break;
        case 3: v.kind = GgufValue::I64; v.i = r.rd<int16_t>(); v.u = (uint64_t)v.i; break;
        case 4: v.kind = GgufValue::U64; v.u = r.rd<uint32_t>(); break;
        case 5: v.kind = GgufValue::I64; v.i = r.rd<int32_t>(); v.u = (uint64_t)(uint32_t)v.i; break;
        case 6: v.kind = GgufValue::F64; v.f = r.rd<float>(); break;
        case 7: v.kind = GgufValue::BOOL; v.u = r.rd<uint8_t>() != 0; break;
        case 8: v.kind = GgufValue::STR; v.s = r.str(); break;
        case 9: {
            v.kind = GgufValue::ARR;
            uint32_t et = r.rd<uint32_t>();
            uint64_t len = r.rd<uint64_t>();
            if (depth >= 4) throw ParseError("GGUF parse error: arrays nested more than 4 deep");
            const uint64_t each = min_value_bytes(et);
            if (each && len > (r.n - r.off) / each)
                throw ParseError("GGUF parse error: array length exceeds file size");
            if (each) v.arr.reserve((size_t)len);
            for (uint64_t k = 0; k < len; ++k) v.arr.push_back(read_value(r, et, depth + 1));
            break;
        }
        case 10: v.kind = GgufValue::U64; v.u = r.rd<uint64_t>(); break;
        case 11: v.kind = GgufValue::I64; v.i = r.rd<int64_t>(); v.u = (uint64_t)v.i; break;
        case 12: v.kind = GgufValue::F64; v.f = r.rd<double>(); break;
        default: {
            char buf[64];
            snprintf(buf, sizeof buf, "Unknown GGUF metadata type: %u", ty);
            throw ParseError(buf);
        }
    }
    return v;
}

}  // namespace

GgufFile::~GgufFile() {
    if (base) munmap((void *)base, size);
}

const GgufTensor *GgufFile::find(const std::string &name) const {
    for (auto &t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

const GgufValue *GgufFile::get(const std::string &key) const {
    auto it = meta.find(key);
    return it == meta.end() ? nullptr : &it->second;
}

int64_t GgufFile::payload_bytes(const GgufTensor &t) {
    const uint64_t n = t.n_elements();
    switch (t.type) {  // model/gguf.rs:38-53, model/loader.rs:110-116
        case GGML_F32: case GGML_I32: return (int64_t)(n * 4);
        case GGML_F16: case GGML_I16: case GGML_BF16: return (int64_t)(n * 2);
        case GGML_I8: return (int64_t)n;
        case GGML_I64: case GGML_F64: return (int64_t)(n * 8);
        case GGML_TQ1_0: return (int64_t)std::ceil((double)n * 54.0 / 256.0);
        case GGML_TQ2_0: return (int64_t)std::ceil((double)n * 66.0 / 256.0);
        case GGML_I2_S: return (int64_t)((n + 3) / 4 + 32);
        default: return -1;
    }
}

GgufFile *gguf_open(const char *path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_error("IO error: %s: %s", path, strerror(errno));
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        set_error("IO error: %s: %s", path, strerror(errno));
        close(fd);
        return nullptr;
    }
    size_t size = (size_t)st.st_size;
    void *m = size ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    close(fd);
    if (m == MAP_FAILED) {
        if (size == 0) {
            set_error("GGUF parse error: Unexpected EOF at offset 0 (need 4 bytes, have 0)");
        } else {
            set_error("IO error: mmap %s: %s", path, strerror(errno));
        }
        return nullptr;
    }
    auto *g = new GgufFile();
    g->base = (const uint8_t *)m;
    g->size = size;
    try {
        Reader r{g->base, size};
        uint32_t magic = r.rd<uint32_t>();
        if (magic != 0x46554747u) {
            char buf[96];
            snprintf(buf, sizeof buf, "Invalid GGUF magic: 0x%08x (expected 0x46554747)", magic);
            throw ParseError(buf);
        }
        g->version = r.rd<uint32_t>();
        if (g->version < 2 || g->version > 3) {
            char buf[64];
            snprintf(buf, sizeof buf, "Unsupported GGUF version: %u", g->version);
            throw ParseError(buf);
        }
        uint64_t n_tensors = r.rd<uint64_t>();
        uint64_t n_kv = r.rd<uint64_t>();
        for (uint64_t k = 0; k < n_kv; ++k) {
            std::string key = r.str();
            uint32_t ty = r.rd<uint32_t>();
            g->meta[key] = read_value(r, ty);
        }
        if (n_tensors > size) throw ParseError("GGUF parse error: tensor count exceeds file size");
        for (uint64_t k = 0; k < n_tensors; ++k) {
            GgufTensor t;
            t.name = r.str();
            uint32_t nd = r.rd<uint32_t>();
            if (nd > 8) throw ParseError("GGUF parse error: tensor rank > 8");
            // The element count must not wrap: every stored type takes at
            // least 54/256 byte per element, so a count above 8x the file
            // size cannot describe data inside it.
            uint64_t elems = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                t.shape.push_back(r.rd<uint64_t>());
                if (__builtin_mul_overflow(elems, t.shape.back(), &elems) || elems > 8 * (uint64_t)size)
                    throw ParseError("GGUF parse error: tensor " + t.name + " element count exceeds file size");
            }
            t.type = r.rd<uint32_t>();
            t.offset = r.rd<uint64_t>();
            g->tensors.push_back(std::move(t));
        }
        uint64_t align = 32;
        if (auto *a = g->get("general.alignment"))
            if (a->is_int() && a->u > 0) align = a->u;
        g->data_offset = (size_t)((r.off + align - 1) / align * align);
        for (auto &t : g->tensors) {
            int64_t pb = GgufFile::payload_bytes(t);
            if (pb < 0) {
                char buf[64];
                snprintf(buf, sizeof buf, "Unsupported GGML type: %u", t.type);
                throw ParseError(buf);
            }
            if (g->data_offset > size || t.offset > size - g->data_offset ||
                (uint64_t)pb > size - g->data_offset - t.offset) {
                char buf[256];
                snprintf(buf, sizeof buf,
                         "GGUF parse error: tensor %s data [%llu, +%lld) exceeds file size %zu",
                         t.name.c_str(), (unsigned long long)(g->data_offset + t.offset),
                         (long long)pb, size);
                throw ParseError(buf);
            }
        }
    } catch (const ParseError &e) {
        set_error("%s", e.what());
        delete g;
        return nullptr;
    }
    return g;
}

}  // namespace oxb
