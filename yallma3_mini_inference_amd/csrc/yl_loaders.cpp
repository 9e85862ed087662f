// yl_loaders.cpp -- the reference's safetensors and lm.rs model files, read
// into a HostModel (host side).  Where the reference panics on a malformed
// file, these return an error message.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>

#include "yallma3.h"
#include "yl_host_model.h"
#include "yl_internal.h"
#include "yl_json.h"

namespace yl {
namespace {

bool read_file(const std::string& path, std::string* out, std::string* err) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) { *err = "cannot open " + path; return false; }
    out->clear();
    char buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof buf, f)) > 0) out->append(buf, k);
    fclose(f);
    return true;
}

bool file_exists(const std::string& p) {
    FILE* f = fopen(p.c_str(), "rb");
    if (f) fclose(f);
    return f != nullptr;
}

std::string parent_dir(const std::string& p) {
    const size_t s = p.rfind('/');
    return s == std::string::npos ? "." : p.substr(0, s);
}

float half_bits_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {
            int ee = -1;
            uint32_t mm = m;
            do { ee++; mm <<= 1; } while (!(mm & 0x400));
            bits = sign | ((uint32_t)(127 - 15 - ee) << 23) | ((mm & 0x3ff) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Rust `(v).round() as i32`, then clamp to i8 (util.rs:497-500)
int8_t round_clamp_i8(float v) {
    if (v != v) return 0;
    float r = roundf(v);
    if (r > 2147483647.0f) r = 2147483647.0f;
    if (r < -2147483648.0f) r = -2147483648.0f;
    long q = (long)r;
    if (q < -128) q = -128;
    if (q > 127) q = 127;
    return (int8_t)q;
}

// util::load_q8_tensor_st (util.rs:452-503): 8-bit affine groups (u8 value *
// f16 scale + f16 bias) dequantized and requantized symmetric per group.
bool load_q8_st(const uint8_t* data, size_t size, size_t rows, size_t cols, size_t gs, size_t w_off, size_t s_off,
                size_t b_off, HostMat* out, std::string* err) {
    const size_t n = rows * cols, groups = n / gs;
    if (gs > 256 || gs == 0 || cols % 4 || n % gs) { *err = "safetensors Q8: group size must divide the tensor (<= 256)"; return false; }
    if (w_off + n > size || s_off + groups * 2 > size || b_off + groups * 2 > size) {
        *err = "safetensors Q8: tensor exceeds the file";
        return false;
    }
    out->f16 = false;
    out->o = rows;
    out->n = cols;
    out->gs = (int)gs;
    out->q.assign(n, 0);
    out->s.assign(groups, 0.0f);
    float deq[256];
    for (size_t g = 0; g < groups; g++) {
        const float scale = half_bits_to_float(rd16(data + s_off + g * 2));
        const float bias = half_bits_to_float(rd16(data + b_off + g * 2));
        const size_t start = g * gs, end = std::min(start + gs, n);
        float max_abs = 0.0f;
        for (size_t i = start; i < end; i++) {
            const float prod = (float)data[w_off + i] * scale;
            const float f = prod + bias;
            deq[i - start] = f;
            const float a = fabsf(f);
            if (a > max_abs) max_abs = a;
        }
        const float sym = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        out->s[g] = sym;
        for (size_t i = start; i < end; i++) out->q[i] = round_clamp_i8(deq[i - start] / sym);
    }
    return true;
}

struct StTensor {
    std::string dtype;
    std::vector<uint64_t> shape;
    size_t offset = 0;   // absolute
};

}  // namespace

bool load_safetensors(const std::string& path, uint32_t max_ctx_len, int fmt_override, HostModel* m, std::string* err) {
    const std::string dir = parent_dir(path);
    std::string cfg_text;
    if (!read_file(dir + "/config.json", &cfg_text, err)) return false;
    json::Value cfg;
    if (!json::parse(cfg_text, &cfg, err)) { *err = "config.json: " + *err; return false; }
    auto req_u = [&](const char* k, int* out) {
        const json::Value* v = cfg.get(k);
        uint64_t u;
        if (!v || !v->as_u64(&u) || u > 0x7fffffffu) { *err = std::string("config.json: missing or non-integer ") + k; return false; }
        *out = (int)u;
        return true;
    };
    auto req_f = [&](const char* k, float* out) {
        const json::Value* v = cfg.get(k);
        double d;
        if (!v || !v->as_f64(&d)) { *err = std::string("config.json: missing or non-numeric ") + k; return false; }
        *out = (float)d;
        return true;
    };
    int max_seq = 0;
    if (!req_u("hidden_size", &m->dim) || !req_u("intermediate_size", &m->hidden) ||
        !req_u("num_attention_heads", &m->n_heads) || !req_u("num_key_value_heads", &m->n_kv) ||
        !req_u("head_dim", &m->hd) || !req_u("num_hidden_layers", &m->n_layers) || !req_u("vocab_size", &m->vocab) ||
        !req_f("rms_norm_eps", &m->eps) || !req_f("rope_theta", &m->rope_theta) ||
        !req_u("max_position_embeddings", &max_seq))
        return false;
    // format: the override, else the quantization section (transformer_llama_st.rs:60-93)
    const json::Value* q = cfg.get("quantization");
    uint64_t gsu = 32;
    bool q4 = false;
    if (q && q->get("group_size")) q->get("group_size")->as_u64(&gsu);
    if (fmt_override == YL_F16) m->f16 = true;
    else if (fmt_override == YL_Q8_0) m->f16 = false;
    else if (fmt_override == YL_Q4_0) q4 = true;
    else if (!q) m->f16 = true;
    else {
        const json::Value* qt = q->get("quant_type");
        q4 = qt && qt->as_str() && *qt->as_str() == "Q4_0";
    }
    if (q4) {
        *err = "safetensors Q4_0: the reference loads these tensors as Q8 and runs its Q4_0 kernel on them; not built";
        return false;
    }
    m->gs = m->f16 ? 32 : (int)gsu;
    m->ctx = (int)std::min<uint32_t>((uint32_t)max_seq, max_ctx_len);
    m->name = "TransformerLlamaSt";

    std::string file;
    if (!read_file(path, &file, err)) return false;
    const uint8_t* data = reinterpret_cast<const uint8_t*>(file.data());
    if (file.size() < 8) { *err = "safetensors: file too short"; return false; }
    uint64_t hlen;
    memcpy(&hlen, data, 8);
    if (hlen > file.size() - 8) { *err = "safetensors: header exceeds the file"; return false; }
    json::Value hdr;
    if (!json::parse(file.substr(8, hlen), &hdr, err) || hdr.kind != json::Value::kObj) {
        *err = "safetensors header: " + *err;
        return false;
    }
    std::map<std::string, StTensor> ts;
    const size_t data_start = 8 + hlen;
    for (const auto& kv : hdr.obj) {
        if (kv.first == "__metadata__") continue;
        StTensor t;
        const json::Value* dt = kv.second.get("dtype");
        const json::Value* sh = kv.second.get("shape");
        const json::Value* of = kv.second.get("data_offsets");
        uint64_t a = 0;
        if (!dt || !dt->as_str() || !sh || sh->kind != json::Value::kArr || !of || of->kind != json::Value::kArr ||
            of->arr.empty() || !of->arr[0].as_u64(&a)) {
            *err = "safetensors header: bad entry " + kv.first;
            return false;
        }
        t.dtype = *dt->as_str();
        for (const auto& d : sh->arr) {
            uint64_t u;
            if (!d.as_u64(&u)) { *err = "safetensors header: bad shape of " + kv.first; return false; }
            t.shape.push_back(u);
        }
        t.offset = data_start + a;
        ts[kv.first] = t;
    }
    auto find = [&](const std::string& nm) -> const StTensor* {
        auto it = ts.find(nm);
        if (it == ts.end()) { *err = "safetensors: missing tensor " + nm; return nullptr; }
        return &it->second;
    };
    auto f16_vec = [&](const StTensor* t, size_t n, std::vector<float>* out) {
        if (t->offset + n * 2 > file.size()) { *err = "safetensors: tensor exceeds the file"; return false; }
        out->resize(n);
        for (size_t i = 0; i < n; i++) (*out)[i] = half_bits_to_float(rd16(data + t->offset + 2 * i));
        return true;
    };
    const size_t dim = m->dim;
    const StTensor* nw = find("model.norm.weight");
    if (!nw) return false;
    if (nw->dtype != "F16" || nw->shape.empty() || nw->shape[0] != dim) {
        *err = "model.norm.weight must be F16 of hidden_size";   // transformer_llama_st.rs:168-169
        return false;
    }
    if (!f16_vec(nw, dim, &m->rms_final)) return false;
    m->rms_att.resize(m->n_layers);
    m->rms_ffn.resize(m->n_layers);
    for (int l = 0; l < m->n_layers; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        const StTensor* a = find(p + "input_layernorm.weight");
        const StTensor* b = a ? find(p + "post_attention_layernorm.weight") : nullptr;
        if (!a || !b || !f16_vec(a, dim, &m->rms_att[l]) || !f16_vec(b, dim, &m->rms_ffn[l])) return false;
    }
    // token embedding
    const size_t V = m->vocab;
    if (m->f16) {
        const StTensor* e = find("model.embed_tokens.weight");
        if (!e) return false;
        if (e->dtype != "F16" || e->shape.size() != 2) { *err = "Expected F16 token embedding"; return false; }
        const size_t n = e->shape[0] * e->shape[1];
        if (n < V * dim || e->offset + n * 2 > file.size()) { *err = "token embedding smaller than vocab_size x hidden_size"; return false; }
        m->emb_f16.resize(V * dim);
        for (size_t i = 0; i < V * dim; i++) m->emb_f16[i] = rd16(data + e->offset + 2 * i);
    } else {
        const StTensor* w = find("model.embed_tokens.weight");
        const StTensor* s = w ? find("model.embed_tokens.scales") : nullptr;
        const StTensor* b = s ? find("model.embed_tokens.biases") : nullptr;
        if (!b) return false;
        if (dim % (size_t)m->gs) { *err = "token embedding: hidden_size must be a multiple of the group size"; return false; }
        if (!load_q8_st(data, file.size(), V, dim, m->gs, w->offset, s->offset, b->offset, &m->emb_q8, err)) return false;
    }
    // projections
    const size_t qr = (size_t)m->n_heads * m->hd, kr = (size_t)m->n_kv * m->hd, H = m->hidden;
    const char* names[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                            "mlp.gate_proj", "mlp.down_proj", "mlp.up_proj"};
    const size_t rows[7] = {qr, kr, kr, dim, H, dim, H};
    const size_t cols[7] = {dim, dim, dim, qr, dim, H, dim};
    m->layers.resize(m->n_layers);
    for (int l = 0; l < m->n_layers; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        for (int k = 0; k < 7; k++) {
            HostMat& h = m->layers[l][k];
            const std::string base = p + names[k];
            if (m->f16) {
                const StTensor* t = find(base + ".weight");
                if (!t) return false;
                if (t->dtype != "F16") { *err = "Expected F16 tensor, got " + t->dtype; return false; }
                size_t n = 1;
                for (uint64_t d : t->shape) n *= d;
                if (n != rows[k] * cols[k] || t->offset + n * 2 > file.size()) { *err = base + ": unexpected size"; return false; }
                h.f16 = true;
                h.o = rows[k];
                h.n = cols[k];
                h.h.resize(n);
                for (size_t i = 0; i < n; i++) h.h[i] = rd16(data + t->offset + 2 * i);
            } else {
                const StTensor* w = find(base + ".weight");
                const StTensor* s = w ? find(base + ".scales") : nullptr;
                const StTensor* b = s ? find(base + ".biases") : nullptr;
                if (!b) return false;
                if (!load_q8_st(data, file.size(), rows[k], cols[k], m->gs, w->offset, s->offset, b->offset, &h, err)) {
                    *err = base + ": " + *err;
                    return false;
                }
            }
        }
    }
    // tokenizer.json beside the model, else tokenizer.bin (transformer_llama_st.rs:287-292)
    const std::string tj = dir + "/tokenizer.json";
    m->tok = file_exists(tj) ? tokenizer_from_hf_json(tj, err) : tokenizer_from_llama2c(dir + "/tokenizer.bin", err);
    return m->tok != nullptr;
}

bool load_lmrs(const std::string& path, uint32_t max_ctx_len, int fmt_override, HostModel* m, std::string* err) {
    (void)fmt_override;   // lm.rs files are Q8_0; the reference ignores other overrides (:95-103)
    const std::string dir = parent_dir(path);
    m->tok = tokenizer_from_llama2c(dir + "/tokenizer.bin", err);
    if (!m->tok) return false;
    std::string file;
    if (!read_file(path, &file, err)) return false;
    const uint8_t* d = reinterpret_cast<const uint8_t*>(file.data());
    if (file.size() < 256 || memcmp(d, "lmrs", 4) != 0) { *err = "Model not in lm.rs format."; return false; }
    auto u32 = [&](size_t o) { uint32_t v; memcpy(&v, d + o, 4); return v; };
    auto f32 = [&](size_t o) { float v; memcpy(&v, d + o, 4); return v; };
    // TransformerArgs, packed, at bytes 8..55 (transformer_llama_lmrs.rs:31-47)
    const uint32_t dim = u32(8), hidden = u32(12), n_layers = u32(16), n_heads = u32(20), head_size = u32(24),
                   n_kv = u32(28), vocab = u32(32), seq_len = u32(36);
    m->eps = f32(40);
    m->rope_theta = f32(44);
    const uint32_t gs = u32(50);
    if (!dim || !hidden || !n_heads || !n_layers) { *err = "Invalid model configuration: critical dimensions cannot be zero"; return false; }
    if (!seq_len || !vocab) { *err = "Invalid model configuration: sequence length and vocab size must be positive"; return false; }
    if (!gs || gs % 32 || gs > (1u << 20)) { *err = "lm.rs: group size must be a multiple of 32"; return false; }
    m->dim = (int)dim; m->hidden = (int)hidden; m->n_layers = (int)n_layers; m->n_heads = (int)n_heads;
    m->hd = (int)head_size; m->n_kv = (int)n_kv; m->vocab = (int)vocab;
    m->ctx = (int)std::min(seq_len, max_ctx_len);
    m->f16 = false;
    m->gs = (int)gs;
    m->name = "TransformerLlamaLmrs";
    size_t off = 256;
    auto take_q8 = [&](size_t o, size_t n, HostMat* h) {
        const size_t count = o * n, groups = count / gs;
        if (count % gs) { *err = "lm.rs: tensor size not a multiple of the group size"; return false; }
        if (off + count + groups * 4 > file.size()) { *err = "lm.rs: tensor exceeds the file"; return false; }
        h->f16 = false;
        h->o = o;
        h->n = n;
        h->gs = (int)gs;
        h->q.assign(reinterpret_cast<const int8_t*>(d + off), reinterpret_cast<const int8_t*>(d + off) + count);
        off += count;
        h->s.resize(groups);
        memcpy(h->s.data(), d + off, groups * 4);
        off += groups * 4;
        return true;
    };
    auto take_f32 = [&](size_t n, std::vector<float>* v) {
        if (off + n * 4 > file.size()) { *err = "lm.rs: tensor exceeds the file"; return false; }
        v->resize(n);
        memcpy(v->data(), d + off, n * 4);
        off += n * 4;
        return true;
    };
    if (dim % gs) { *err = "lm.rs: dim must be a multiple of the group size"; return false; }
    if (!take_q8(vocab, dim, &m->emb_q8)) return false;
    m->rms_att.resize(n_layers);
    m->rms_ffn.resize(n_layers);
    m->layers.resize(n_layers);
    const size_t att = (size_t)n_heads * head_size, kv = (size_t)n_kv * head_size;
    for (uint32_t l = 0; l < n_layers; l++) if (!take_f32(dim, &m->rms_att[l])) return false;
    // projections by kind, each over all layers (wq, wk, wv, wo; norms; w1, w2, w3)
    const size_t shapes[7][2] = {{att, dim}, {kv, dim}, {kv, dim}, {dim, att}, {hidden, dim}, {dim, hidden}, {hidden, dim}};
    for (int k : {0, 1, 2, 3})
        for (uint32_t l = 0; l < n_layers; l++)
            if (!take_q8(shapes[k][0], shapes[k][1], &m->layers[l][k])) return false;
    for (uint32_t l = 0; l < n_layers; l++) if (!take_f32(dim, &m->rms_ffn[l])) return false;
    for (int k : {4, 5, 6})
        for (uint32_t l = 0; l < n_layers; l++)
            if (!take_q8(shapes[k][0], shapes[k][1], &m->layers[l][k])) return false;
    return take_f32(dim, &m->rms_final);
}

}  // namespace yl
