// gguf_reader.h -- minimal GGUF v2/v3 reader (metadata key/values and tensor
// directory) for loading the talker / code-predictor weights.  The file
// format (magic "GGUF", version, tensor and KV counts, typed KV entries,
// tensor infos, aligned data section) is the public GGUF specification the
// reference reads through gguf.h (src/gguf_loader.cpp).
#pragma once

#include <cstdint>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

namespace qwen3_tts {

struct GGUFTensorInfo {
    std::string name;
    uint32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    int32_t type = 0;
    uint64_t offset = 0;      // relative to the data section
    size_t nbytes = 0;
};

class GGUFReader {
public:
    ~GGUFReader() { close(); }
    bool open(const std::string & path);
    void close();
    const std::string & error() const { return err_; }

    bool has_key(const std::string & k) const { return u32_.count(k) || f32_.count(k); }
    // numeric value of an integer-typed key (any width), false if absent
    bool get_u32(const std::string & k, uint32_t & out) const;
    bool get_f32(const std::string & k, float & out) const;

    const std::vector<GGUFTensorInfo> & tensors() const { return tensors_; }
    // reads a tensor's bytes into dst (resized)
    bool read_tensor(const GGUFTensorInfo & t, std::vector<uint8_t> & dst);
    // reads rows [row0, row0 + n_rows) of a tensor (rows along ne[1], each
    // nbytes / ne[1] bytes) into dst, which holds at least that many bytes
    bool read_tensor_rows(const GGUFTensorInfo & t, int64_t row0, int64_t n_rows, void * dst);

private:
    FILE * f_ = nullptr;
    std::string err_;
    std::map<std::string, uint64_t> u32_;
    std::map<std::string, float> f32_;
    std::vector<GGUFTensorInfo> tensors_;
    uint64_t data_offset_ = 0;
};

// ggml tensor byte size for the types the frame loop uses (F32, F16, Q8_0);
// 0 for anything else.
size_t gguf_tensor_nbytes(int32_t type, const int64_t ne[4]);
// ggml's name of a tensor type id ("F16", "Q4_K", ...; "type <id>" if unknown)
std::string gguf_type_name(int32_t type);

}  // namespace qwen3_tts
