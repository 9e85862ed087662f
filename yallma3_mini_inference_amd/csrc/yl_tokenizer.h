// yl_tokenizer.h -- the GGUF tokenizer and the sampler (host side).
//
// Tokenizer follows tokenizer.rs: from_gguf_parts (:77-137), encode
// (:325-380) with the GPT-2 pre-split for `pre` = "gpt2"/"smollm" and plain
// byte-level BPE otherwise, the score-driven merge loop (:296-323), decode
// (:545-568), encode_wrap_n_header (:243-286), the chat-template path
// (:382-456) and apply_system_template / apply_turn_template (:458-543).
// Sampler follows sampler.rs:40-180 (temperature, softmax, top-p, argmax,
// and the xorshift draw whose state never advances).
#pragma once

#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace yl {

struct TokenizerSpec {
    std::vector<std::string> vocab;
    std::vector<std::string> merges;
    bool byte_level = true;         // GPT-2 byte characters (GGUF, tokenizer.json); false: llama2.c tokenizer.bin
    bool has_scores = false;        // scores given (tokenizer.bin) instead of derived from merges
    std::vector<float> scores;
    uint32_t bos = 0, eos = 0;
    std::string pre = "default";
    bool add_bos_token = true, add_space_prefix = false;
    bool has_template = false;
    std::string chat_template;
};

class Tokenizer {
public:
    static constexpr uint32_t kBeginOfText = 128000, kStartHeader = 128006, kEndHeader = 128007, kEot = 128009,
                              kHeaderSep = 271;

    explicit Tokenizer(TokenizerSpec spec);

    // Each returns false with *err set where the reference panics.
    bool encode(const std::string& text, bool bos, bool eos, std::vector<uint32_t>* out, std::string* err) const;
    std::string decode(const std::vector<uint32_t>& ids) const;
    bool encode_wrap_n_header(const std::string& text, const std::string& header, bool bot_wrap,
                              std::vector<uint32_t>* out, std::string* err) const;
    bool apply_system_template(const std::string& system, std::vector<uint32_t>* out, std::string* err) const;
    bool apply_turn_template(const std::string& user, bool add_empty_assistant, std::vector<uint32_t>* out,
                             std::string* err) const;
    bool render_chat_template(const std::vector<std::pair<std::string, std::string>>& messages,
                              bool add_generation_prompt, std::vector<uint32_t>* out, std::string* err) const;

    uint32_t bos() const { return bos_; }
    uint32_t eos() const { return eos_; }
    bool add_bos_token() const { return add_bos_token_; }
    bool has_chat_template() const { return has_template_; }
    size_t vocab_size() const { return vocab_.size(); }

private:
    std::vector<std::string> vocab_;
    std::vector<float> scores_;
    std::unordered_map<std::string, uint32_t> index_;   // text -> id (the last id of equal texts)
    uint32_t bos_, eos_;
    std::string pre_;
    bool add_bos_token_, add_space_prefix_;
    bool has_template_;
    std::string template_;
    bool byte_level_ = true;
    uint32_t byte_to_token_[256];
    std::vector<int> token_to_byte_;                    // -1: none
    std::unordered_map<uint32_t, uint8_t> char_to_byte_;   // GPT-2 byte table, code point -> byte

    bool has_llama_tokens() const { return vocab_.size() > 128009; }
    void bpe_merge(std::vector<uint32_t>* tokens) const;
    bool encode_template_output(const std::string& text, std::vector<uint32_t>* out, std::string* err) const;
};

// Sampler::new(vocab_size, temperature, top_p, seed) and Sampler::sample.
class Sampler {
public:
    Sampler(size_t vocab, float temperature, float top_p, uint64_t seed);
    // Samples from `logits` (vocab floats), which it rescales and normalizes
    // in place as the reference does.  Returns false where the reference
    // panics (no candidate above the top-p cutoff).
    bool sample(float* logits, uint32_t* out);

private:
    struct ProbIndex {
        float prob;
        uint32_t index;
    };
    size_t vocab_;
    std::vector<ProbIndex> idx_;   // persists between calls, as in the reference
    float temperature_, top_p_;
    uint64_t seed_;
};

// The GPT-2 pre-tokenizer split (tokenizer.rs:29-31) of UTF-8 text into
// byte ranges; exposed for tests.
std::vector<std::pair<size_t, size_t>> gpt2_split(const std::string& text);
// Rust String::from_utf8_lossy
std::string utf8_lossy(const std::string& bytes);
// Rust str::trim
std::string trim_unicode(const std::string& s);
// whether p is well-formed UTF-8
bool valid_utf8(const char* p);

class GgufFile;

}  // namespace yl

// C ABI handles (include/yallma3.h)
struct yl_tokenizer {
    yl::Tokenizer t;
};
struct yl_sampler {
    yl::Sampler s;
};

namespace yl {
// Tokenizer::from_gguf_parts + set_chat_template from a GGUF's metadata
// (transformer_llama_gguf.rs:584-641); null with *err on malformed keys.
yl_tokenizer* tokenizer_from_gguf(const GgufFile& g, std::string* err);
inline Sampler& sampler_of(yl_sampler* s) { return s->s; }
}  // namespace yl
