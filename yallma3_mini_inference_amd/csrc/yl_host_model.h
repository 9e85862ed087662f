// yl_host_model.h -- a model read from a safetensors or lm.rs file, on the
// host, before it is laid out on the device (the GGUF loader builds its
// device layout directly).
#pragma once

#include <stdint.h>

#include <array>
#include <string>
#include <vector>

#include "yl_tokenizer.h"

namespace yl {

struct HostMat {                  // one projection [o][n]
    bool f16 = false;             // F16 values (h) or Q8 values (q) with f32 scales (s) per gs group
    size_t o = 0, n = 0;
    int gs = 32;
    std::vector<int8_t> q;
    std::vector<float> s;
    std::vector<uint16_t> h;
};

struct HostModel {
    std::string name;             // "TransformerLlamaSt" / "TransformerLlamaLmrs"
    int dim = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv = 0, hd = 0, vocab = 0, ctx = 0;
    float eps = 0.0f, rope_theta = 0.0f;
    bool f16 = false;             // WeightFormat::F16, else Q8_0 with f32 scales
    int gs = 32;
    HostMat emb_q8;               // Q8 models: token embedding [vocab][dim] int8 + f32 scales per gs group;
                                  // the reference's f32 table is exactly q * scale (transformer_llama_lmrs.rs:176-181)
    std::vector<uint16_t> emb_f16;   // F16 models: the table's values as binary16
    std::vector<std::vector<float>> rms_att, rms_ffn;
    std::vector<float> rms_final;
    // per layer: attn q, k, v, output, ffn gate, down, up
    std::vector<std::array<HostMat, 7>> layers;
    yl_tokenizer* tok = nullptr;  // owned by the HostModel until moved into a model
    ~HostModel() { delete tok; }
};

// transformer_llama_st.rs:36-300 (config.json + model weights + tokenizer)
bool load_safetensors(const std::string& path, uint32_t max_ctx_len, int fmt_override, HostModel* m, std::string* err);
// transformer_llama_lmrs.rs:60-434 (lm.rs file + tokenizer.bin beside it)
bool load_lmrs(const std::string& path, uint32_t max_ctx_len, int fmt_override, HostModel* m, std::string* err);
// Tokenizer::from_json (tokenizer.rs:139-224) and Tokenizer::new (tokenizer.rs:226-268)
yl_tokenizer* tokenizer_from_hf_json(const std::string& path, std::string* err);
yl_tokenizer* tokenizer_from_llama2c(const std::string& path, std::string* err);

}  // namespace yl
