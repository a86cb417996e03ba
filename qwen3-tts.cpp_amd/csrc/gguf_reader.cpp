// gguf_reader.cpp -- see gguf_reader.h.
#include "gguf_reader.h"

#include <cstring>

namespace qwen3_tts {

namespace {

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STR = 8, T_ARR = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12,
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case T_U8: case T_I8: case T_BOOL: return 1;
        case T_U16: case T_I16: return 2;
        case T_U32: case T_I32: case T_F32: return 4;
        case T_U64: case T_I64: case T_F64: return 8;
        default: return 0;
    }
}

}  // namespace

size_t gguf_tensor_nbytes(int32_t type, const int64_t ne[4]) {
    const int64_t n = ne[0] * ne[1] * ne[2] * ne[3];
    if (type == 0) return (size_t) n * 4;
    if (type == 1) return (size_t) n * 2;
    if (type == 8) return ne[0] % 32 ? 0 : (size_t) (n / 32) * 34;
    return 0;
}

std::string gguf_type_name(int32_t type) {
    // ggml_type ids of the public GGUF specification
    static const char * const names[] = {"F32", "F16", "Q4_0", "Q4_1", "type 4", "type 5", "Q5_0", "Q5_1", "Q8_0",
                                         "Q8_1", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_K", "IQ2_XXS", "IQ2_XS",
                                         "IQ3_XXS", "IQ1_S", "IQ4_NL", "IQ3_S", "IQ2_S", "IQ4_XS", "I8", "I16", "I32",
                                         "I64", "F64", "IQ1_M", "BF16"};
    if (type >= 0 && type < (int32_t) (sizeof(names) / sizeof(names[0]))) return names[type];
    return "type " + std::to_string(type);
}

void GGUFReader::close() {
    if (f_) { std::fclose(f_); f_ = nullptr; }
    u32_.clear(); f32_.clear(); tensors_.clear();
}

bool GGUFReader::get_u32(const std::string & k, uint32_t & out) const {
    auto it = u32_.find(k);
    if (it == u32_.end()) return false;
    out = (uint32_t) it->second;
    return true;
}

bool GGUFReader::get_f32(const std::string & k, float & out) const {
    auto it = f32_.find(k);
    if (it == f32_.end()) return false;
    out = it->second;
    return true;
}

bool GGUFReader::open(const std::string & path) {
    close();
    f_ = std::fopen(path.c_str(), "rb");
    if (!f_) { err_ = "Failed to open GGUF file: " + path; return false; }
    auto rd = [&](void * p, size_t n) { return std::fread(p, 1, n, f_) == n; };
    auto rd_str = [&](std::string & s) -> bool {
        uint64_t len = 0;
        if (!rd(&len, 8) || len > (1u << 26)) return false;
        s.resize(len);
        return len == 0 || rd(&s[0], len);
    };
    auto skip = [&](uint64_t n) { return std::fseek(f_, (long) n, SEEK_CUR) == 0; };
    uint32_t magic = 0, version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!rd(&magic, 4) || std::memcmp(&magic, "GGUF", 4) != 0) { err_ = "not a GGUF file: " + path; return false; }
    if (!rd(&version, 4) || version < 2 || version > 3) { err_ = "unsupported GGUF version"; return false; }
    if (!rd(&n_tensors, 8) || !rd(&n_kv, 8)) { err_ = "truncated GGUF header"; return false; }
    uint32_t alignment = 32;
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t t = 0;
        if (!rd_str(key) || !rd(&t, 4)) { err_ = "truncated GGUF metadata"; return false; }
        if (t == T_STR) {
            std::string v;
            if (!rd_str(v)) { err_ = "truncated GGUF string"; return false; }
        } else if (t == T_ARR) {
            uint32_t et = 0;
            uint64_t cnt = 0;
            if (!rd(&et, 4) || !rd(&cnt, 8)) { err_ = "truncated GGUF array"; return false; }
            if (et == T_STR) {
                for (uint64_t j = 0; j < cnt; ++j) {
                    std::string v;
                    if (!rd_str(v)) { err_ = "truncated GGUF array"; return false; }
                }
            } else {
                const size_t es = scalar_size(et);
                if (!es || !skip(es * cnt)) { err_ = "bad GGUF array"; return false; }
            }
        } else {
            const size_t es = scalar_size(t);
            if (!es) { err_ = "bad GGUF value type"; return false; }
            uint8_t buf[8] = {0};
            if (!rd(buf, es)) { err_ = "truncated GGUF value"; return false; }
            if (t == T_F32) { float v; std::memcpy(&v, buf, 4); f32_[key] = v; }
            else if (t == T_F64) { double v; std::memcpy(&v, buf, 8); f32_[key] = (float) v; }
            else {
                uint64_t v = 0;
                std::memcpy(&v, buf, es);
                u32_[key] = v;
            }
        }
        if (key == "general.alignment" && u32_.count(key)) alignment = (uint32_t) u32_[key];
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GGUFTensorInfo ti;
        uint32_t type = 0;
        if (!rd_str(ti.name) || !rd(&ti.n_dims, 4) || ti.n_dims > 4) { err_ = "bad GGUF tensor info"; return false; }
        for (uint32_t d = 0; d < ti.n_dims; ++d) {
            uint64_t v;
            if (!rd(&v, 8)) { err_ = "truncated GGUF tensor info"; return false; }
            ti.ne[d] = (int64_t) v;
        }
        if (!rd(&type, 4) || !rd(&ti.offset, 8)) { err_ = "truncated GGUF tensor info"; return false; }
        ti.type = (int32_t) type;
        ti.nbytes = gguf_tensor_nbytes(ti.type, ti.ne);
        tensors_.push_back(ti);
    }
    const long pos = std::ftell(f_);
    data_offset_ = ((uint64_t) pos + alignment - 1) / alignment * alignment;
    return true;
}

bool GGUFReader::read_tensor(const GGUFTensorInfo & t, std::vector<uint8_t> & dst) {
    if (!f_) { err_ = "GGUF file not open"; return false; }
    if (t.nbytes == 0) { err_ = "unsupported tensor type for " + t.name; return false; }
    dst.resize(t.nbytes);
    if (std::fseek(f_, (long) (data_offset_ + t.offset), SEEK_SET) != 0) {
        err_ = "Failed to seek to tensor data: " + t.name;
        return false;
    }
    if (std::fread(dst.data(), 1, t.nbytes, f_) != t.nbytes) {
        err_ = "Failed to read tensor data: " + t.name;
        return false;
    }
    return true;
}

bool GGUFReader::read_tensor_rows(const GGUFTensorInfo & t, int64_t row0, int64_t n_rows, void * dst) {
    if (!f_) { err_ = "GGUF file not open"; return false; }
    if (t.nbytes == 0) { err_ = "unsupported tensor type for " + t.name; return false; }
    const int64_t rows = t.n_dims >= 2 ? t.ne[1] * t.ne[2] * t.ne[3] : 1;
    if (row0 < 0 || n_rows < 0 || row0 + n_rows > rows) { err_ = "row range out of bounds for " + t.name; return false; }
    const size_t row_bytes = t.nbytes / (size_t) rows, n = row_bytes * (size_t) n_rows;
    if (std::fseek(f_, (long) (data_offset_ + t.offset + row_bytes * (size_t) row0), SEEK_SET) != 0) {
        err_ = "Failed to seek to tensor data: " + t.name;
        return false;
    }
    if (std::fread(dst, 1, n, f_) != n) {
        err_ = "Failed to read tensor data: " + t.name;
        return false;
    }
    return true;
}

}  // namespace qwen3_tts
