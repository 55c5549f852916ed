// GGUF v2/v3 reader (host).  Follows the reference parser
// (model/gguf.rs:144-231): little-endian header, typed metadata key/values,
// tensor infos, data section aligned to general.alignment (default 32).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace oxb {

enum GgmlType : uint32_t {
    GGML_F32 = 0,
    GGML_F16 = 1,
    GGML_I8 = 16,
    GGML_I16 = 17,
    GGML_I32 = 18,
    GGML_I64 = 27,
    GGML_F64 = 28,
    GGML_BF16 = 30,
    GGML_TQ1_0 = 34,
    GGML_TQ2_0 = 35,
    GGML_I2_S = 36,  // ternary, 2 bits per weight + 32-byte scale trailer
};

struct GgufValue {
    enum Kind { U64, I64, F64, BOOL, STR, ARR } kind = U64;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    std::vector<GgufValue> arr;
    bool is_int() const { return kind == U64 || kind == I64 || kind == BOOL; }
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> shape;  // ne0 (innermost) first
    uint32_t type = 0;
    uint64_t offset = 0;          // relative to the data section
    uint64_t n_elements() const {
        uint64_t n = 1;
        for (auto d : shape) n *= d;
        return n;
    }
};

struct GgufFile {
    uint32_t version = 0;
    std::map<std::string, GgufValue> meta;
    std::vector<GgufTensor> tensors;
    size_t data_offset = 0;
    // mapped file
    const uint8_t *base = nullptr;
    size_t size = 0;

    ~GgufFile();
    const GgufTensor *find(const std::string &name) const;
    const GgufValue *get(const std::string &key) const;
    // Bytes of a tensor's payload (I2_S: ceil(n/4) + 32).  -1 on unsupported type.
    static int64_t payload_bytes(const GgufTensor &t);
};

// Parse `path` (memory-mapped).  Returns nullptr and sets the thread error
// with the reference's messages on failure.
GgufFile *gguf_open(const char *path);

}  // namespace oxb
