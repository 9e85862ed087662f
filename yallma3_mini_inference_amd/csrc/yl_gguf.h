// yl_gguf.h -- GGUF v3 reader for the llama loader (host side).
//
// Follows TransformerLlamaGguf::load_model_inner
// (transformer_llama_gguf.rs:183-332): little-endian header, typed metadata
// (value types 0..12, arrays as element type + count), tensor infos, data
// section aligned to general.alignment (default 32).  Where the reference
// panics, this reader returns an error message instead.
#pragma once

#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace yl {

struct GgufValue {
    int type = -1;            // GGUF value type; -1 = absent
    uint64_t u = 0;           // unsigned integers and bool
    int64_t i = 0;            // signed integers
    double f = 0.0;           // floats
    std::string s;            // strings
    uint64_t arr_len = 0;     // arrays
    int arr_type = -1;
    std::vector<std::string> arr_str;  // string arrays (tokenizer)
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;      // relative to the data section
    uint64_t n_elements = 0;
    const uint8_t* data = nullptr;  // resolved pointer into the mapping
    uint64_t avail = 0;             // bytes from data to end of file
};

class GgufFile {
public:
    ~GgufFile();
    bool open(const std::string& path, std::string* err);
    const GgufValue* get(const std::string& key) const;
    const GgufTensor* tensor(const std::string& name) const;
    const std::map<std::string, GgufValue>& meta() const { return meta_; }

private:
    const uint8_t* map_ = nullptr;
    size_t len_ = 0;
    std::map<std::string, GgufValue> meta_;
    std::map<std::string, GgufTensor> tensors_;
};

// metadata accessors with the reference's accepted types
bool meta_u64(const GgufFile& g, const char* key, uint64_t* out);             // u64/u32 (:123-129)
bool meta_f32(const GgufFile& g, const char* key, float* out);                // f32/f64 (:131-137)

}  // namespace yl
