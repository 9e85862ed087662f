// yl_gguf.cpp -- GGUF v3 reader (transformer_llama_gguf.rs:72-107,183-332).
#include "yl_gguf.h"

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace yl {

namespace {

struct Reader {
    const uint8_t* p;
    size_t len, off = 0;
    bool bad = false;
    bool need(uint64_t k) {
        if (bad || k > len || off > len - k) { bad = true; return false; }
        return true;
    }
    uint64_t u(int n) {
        if (!need((uint64_t)n)) return 0;
        uint64_t v = 0;
        for (int i = 0; i < n; i++) v |= (uint64_t)p[off + i] << (8 * i);
        off += (size_t)n;
        return v;
    }
    std::string str() {
        const uint64_t n = u(8);
        if (!need(n)) return std::string();
        std::string s((const char*)p + off, (size_t)n);
        off += (size_t)n;
        return s;
    }
};

// read_gguf_value, transformer_llama_gguf.rs:80-107
bool read_value(Reader& r, uint32_t type, GgufValue* v, bool keep_strings, std::string* err) {
    v->type = (int)type;
    switch (type) {
    case 0: v->u = r.u(1); break;
    case 1: v->i = (int8_t)r.u(1); break;
    case 2: v->u = r.u(2); break;
    case 3: v->i = (int16_t)r.u(2); break;
    case 4: v->u = r.u(4); break;
    case 5: v->i = (int32_t)r.u(4); break;
    case 6: { const uint32_t b = (uint32_t)r.u(4); float f; memcpy(&f, &b, 4); v->f = f; break; }
    case 7: v->u = r.u(1) != 0; break;
    case 8: v->s = r.str(); break;
    case 9: {
        const uint32_t et = (uint32_t)r.u(4);
        const uint64_t n = r.u(8);
        v->arr_type = (int)et;
        v->arr_len = n;
        for (uint64_t k = 0; k < n && !r.bad; k++) {
            GgufValue e;
            if (!read_value(r, et, &e, false, err)) return false;
            if (keep_strings && et == 8) v->arr_str.push_back(std::move(e.s));
        }
        break;
    }
    case 10: v->u = r.u(8); break;
    case 11: v->i = (int64_t)r.u(8); break;
    case 12: { const uint64_t b = r.u(8); double d; memcpy(&d, &b, 8); v->f = d; break; }
    default:
        *err = "Unknown GGUF metadata value type: " + std::to_string(type);
        return false;
    }
    if (r.bad) { *err = "GGUF file truncated"; return false; }
    return true;
}

}  // namespace

GgufFile::~GgufFile() {
    if (map_) munmap((void*)map_, len_);
}

bool GgufFile::open(const std::string& path, std::string* err) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) { *err = "cannot open " + path; return false; }
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); *err = "cannot stat " + path; return false; }
    len_ = (size_t)st.st_size;
    if (len_ < 24) { ::close(fd); *err = "Not a GGUF file (too short)"; return false; }
    void* m = mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) { *err = "mmap failed for " + path; return false; }
    map_ = (const uint8_t*)m;
    Reader r{map_, len_};
    if (r.u(4) != 0x46554747u) { *err = "Not a GGUF file (bad magic)"; return false; }
    const uint32_t version = (uint32_t)r.u(4);
    if (version != 3) { *err = "Only GGUF version 3 is supported, got version " + std::to_string(version); return false; }
    const uint64_t n_tensors = r.u(8), n_kv = r.u(8);
    for (uint64_t i = 0; i < n_kv; i++) {
        const std::string key = r.str();
        const uint32_t vt = (uint32_t)r.u(4);
        if (r.bad) { *err = "GGUF file truncated"; return false; }
        GgufValue v;
        if (!read_value(r, vt, &v, key == "tokenizer.ggml.tokens" || key == "tokenizer.ggml.merges", err))
            return false;
        meta_[key] = std::move(v);
    }
    std::vector<GgufTensor> infos;
    for (uint64_t i = 0; i < n_tensors; i++) {
        GgufTensor t;
        t.name = r.str();
        const uint32_t nd = (uint32_t)r.u(4);
        t.n_elements = 1;
        for (uint32_t d = 0; d < nd && !r.bad; d++) {
            const uint64_t v = r.u(8);
            t.dims.push_back(v);
            t.n_elements *= v;
        }
        t.type = (uint32_t)r.u(4);
        t.offset = r.u(8);
        if (r.bad) { *err = "GGUF file truncated in tensor infos"; return false; }
        infos.push_back(std::move(t));
    }
    uint64_t alignment = 32;
    meta_u64(*this, "general.alignment", &alignment);
    if (alignment == 0 || (alignment & (alignment - 1))) {
        *err = "GGUF alignment must be a power of 2, got " + std::to_string(alignment);
        return false;
    }
    const uint64_t data_start = ((uint64_t)r.off + alignment - 1) / alignment * alignment;
    for (auto& t : infos) {
        const uint64_t at = data_start + t.offset;
        if (at > len_) { *err = "tensor " + t.name + " starts beyond the end of the file"; return false; }
        t.data = map_ + at;
        t.avail = len_ - at;
        tensors_[t.name] = t;
    }
    return true;
}

const GgufValue* GgufFile::get(const std::string& key) const {
    auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

const GgufTensor* GgufFile::tensor(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

bool meta_u64(const GgufFile& g, const char* key, uint64_t* out) {
    const GgufValue* v = g.get(key);
    if (!v || (v->type != 10 && v->type != 4)) return false;
    *out = v->u;
    return true;
}

bool meta_f32(const GgufFile& g, const char* key, float* out) {
    const GgufValue* v = g.get(key);
    if (!v || (v->type != 6 && v->type != 12)) return false;
    *out = (float)v->f;
    return true;
}

}  // namespace yl
