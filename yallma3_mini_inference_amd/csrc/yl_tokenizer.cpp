// yl_tokenizer.cpp -- GGUF tokenizer (tokenizer.rs) and sampler (sampler.rs).
#include "yl_tokenizer.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "yallma3.h"
#include "yl_gguf.h"
#include "yl_internal.h"
#include "yl_host_model.h"
#include "yl_jinja.h"
#include "yl_json.h"
#include "yl_unicode_tables.h"

namespace yl {
namespace {

template <size_t N>
bool in_ranges(const uint32_t (&r)[N][2], uint32_t cp) {
    size_t lo = 0, hi = N;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (cp < r[mid][0]) hi = mid;
        else if (cp > r[mid][1]) lo = mid + 1;
        else return true;
    }
    return false;
}
bool is_letter(uint32_t cp) { return in_ranges(kUniLetter, cp); }
bool is_number(uint32_t cp) { return in_ranges(kUniNumber, cp); }
bool is_space(uint32_t cp) { return in_ranges(kUniSpace, cp); }
bool is_other(uint32_t cp) { return !is_space(cp) && !is_letter(cp) && !is_number(cp); }

// Decodes valid UTF-8 into (code point, byte offset) pairs.
void decode_utf8(const std::string& s, std::vector<uint32_t>* cps, std::vector<size_t>* offs) {
    for (size_t p = 0; p < s.size();) {
        const unsigned char c = (unsigned char)s[p];
        uint32_t cp;
        size_t len;
        if (c < 0x80) { cp = c; len = 1; }
        else if ((c >> 5) == 6) { cp = c & 0x1F; len = 2; }
        else if ((c >> 4) == 14) { cp = c & 0x0F; len = 3; }
        else { cp = c & 0x07; len = 4; }
        if (p + len > s.size()) len = s.size() - p;
        for (size_t k = 1; k < len; k++) cp = (cp << 6) | ((unsigned char)s[p + k] & 0x3F);
        cps->push_back(cp);
        offs->push_back(p);
        p += len;
    }
    offs->push_back(s.size());
}

std::string utf8_of(uint32_t cp) {
    std::string o;
    if (cp < 0x80) o += (char)cp;
    else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
    else if (cp < 0x10000) { o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
    else {
        o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F));
        o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F));
    }
    return o;
}

// Tokenizer::build_gpt2_byte_table (tokenizer.rs:56-75): printable bytes map
// to themselves, the rest to 256, 257, ... in byte order.
void gpt2_byte_table(uint32_t table[256]) {
    bool direct[256] = {};
    for (int b = '!'; b <= '~'; b++) direct[b] = true;
    for (int b = 0xA1; b <= 0xAC; b++) direct[b] = true;
    for (int b = 0xAE; b <= 0xFF; b++) direct[b] = true;
    uint32_t n = 0;
    for (int b = 0; b < 256; b++) table[b] = direct[b] ? (uint32_t)b : 256 + n++;
}

}  // namespace

// ------------------------------------------------------------------ split
// Leftmost-first matches of
//   '(?:[sdmt]|ll|ve|re)| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+
// at each position; every character starts some alternative, so the matches
// tile the text.
std::vector<std::pair<size_t, size_t>> gpt2_split(const std::string& text) {
    std::vector<uint32_t> cp;
    std::vector<size_t> off;
    decode_utf8(text, &cp, &off);
    const size_t n = cp.size();
    std::vector<std::pair<size_t, size_t>> out;
    size_t i = 0;
    auto run = [&](size_t j, bool (*cls)(uint32_t)) {
        while (j < n && cls(cp[j])) j++;
        return j;
    };
    while (i < n) {
        size_t e = 0;
        if (cp[i] == '\'' && i + 1 < n) {
            const uint32_t a = cp[i + 1];
            if (a == 's' || a == 'd' || a == 'm' || a == 't') e = i + 2;
            else if (i + 2 < n) {
                const uint32_t b = cp[i + 2];
                if ((a == 'l' && b == 'l') || (a == 'v' && b == 'e') || (a == 'r' && b == 'e')) e = i + 3;
            }
        }
        const size_t j = cp[i] == ' ' ? i + 1 : i;   // the optional leading space
        if (!e && j < n && is_letter(cp[j])) e = run(j, is_letter);
        if (!e && j < n && is_number(cp[j])) e = run(j, is_number);
        if (!e && j < n && is_other(cp[j])) e = run(j, is_other);
        if (!e && is_space(cp[i])) e = run(i, is_space);
        if (!e) e = i + 1;   // unreachable: every character is in one class
        out.push_back({off[i], off[e]});
        i = e;
    }
    return out;
}

// Rust String::from_utf8_lossy: each maximal invalid subpart becomes U+FFFD.
std::string utf8_lossy(const std::string& s) {
    static const char kRepl[] = "\xEF\xBF\xBD";
    std::string o;
    const size_t n = s.size();
    size_t i = 0;
    while (i < n) {
        const unsigned char b = (unsigned char)s[i];
        if (b < 0x80) { o += (char)b; i++; continue; }
        const int width = (b >= 0xC2 && b <= 0xDF) ? 2 : (b >= 0xE0 && b <= 0xEF) ? 3 : (b >= 0xF0 && b <= 0xF4) ? 4 : 0;
        if (!width) { o += kRepl; i++; continue; }
        bool ok = true;
        for (int j = 1; j < width; j++) {
            if (i + j >= n) { o += kRepl; i = n; ok = false; break; }
            const unsigned char c = (unsigned char)s[i + j];
            unsigned char lo = 0x80, hi = 0xBF;
            if (j == 1) {
                if (b == 0xE0) lo = 0xA0;
                else if (b == 0xED) hi = 0x9F;
                else if (b == 0xF0) lo = 0x90;
                else if (b == 0xF4) hi = 0x8F;
            }
            if (c < lo || c > hi) { o += kRepl; i += j; ok = false; break; }
        }
        if (ok) { o.append(s, i, width); i += width; }
    }
    return o;
}

std::string trim_unicode(const std::string& s) {
    std::vector<uint32_t> cp;
    std::vector<size_t> off;
    decode_utf8(s, &cp, &off);
    size_t b = 0, e = cp.size();
    while (b < e && is_space(cp[b])) b++;
    while (e > b && is_space(cp[e - 1])) e--;
    return s.substr(off[b], off[e] - off[b]);
}

// -------------------------------------------------------------- tokenizer
Tokenizer::Tokenizer(TokenizerSpec spec)
    : vocab_(std::move(spec.vocab)), bos_(spec.bos), eos_(spec.eos), pre_(std::move(spec.pre)),
      add_bos_token_(spec.add_bos_token), add_space_prefix_(spec.add_space_prefix), has_template_(spec.has_template),
      template_(std::move(spec.chat_template)), byte_level_(spec.byte_level) {
    const size_t V = vocab_.size();
    index_.reserve(V * 2);
    for (size_t i = 0; i < V; i++) index_[vocab_[i]] = (uint32_t)i;   // equal texts: the last id
    if (spec.has_scores) {
        scores_ = spec.scores;
        scores_.resize(V, 0.0f);
    } else {
        // merge rank -> score of the merged token (from_gguf_parts, tokenizer.rs:80-90)
        scores_.assign(V, 0.0f);
        const size_t M = spec.merges.size();
        for (size_t i = 0; i < M; i++) {
            const std::string& mg = spec.merges[i];
            const size_t sp = mg.find(' ');
            if (sp == std::string::npos) continue;
            const std::string merged = mg.substr(0, sp) + mg.substr(sp + 1);
            auto it = index_.find(merged);
            if (it != index_.end()) scores_[it->second] = (float)(M - i);
        }
    }
    if (!byte_level_) {   // Tokenizer::new: bytes map to ids 3..258, no byte characters
        for (int b = 0; b < 256; b++) byte_to_token_[b] = (uint32_t)b + 3;
        return;
    }
    uint32_t table[256];
    gpt2_byte_table(table);
    token_to_byte_.assign(std::max<size_t>(V, 256), -1);
    for (int b = 0; b < 256; b++) {
        char_to_byte_[table[b]] = (uint8_t)b;
        auto it = index_.find(utf8_of(table[b]));
        byte_to_token_[b] = it != index_.end() ? it->second : 0;
        if (it != index_.end()) token_to_byte_[it->second] = b;
    }
}

void Tokenizer::bpe_merge(std::vector<uint32_t>* tokens) const {
    std::vector<uint32_t>& t = *tokens;
    std::string cat;
    for (;;) {
        float best = -1e10f;
        uint32_t best_id = 0;
        long best_idx = -1;
        for (size_t idx = 0; idx + 1 < t.size(); idx++) {
            cat.assign(vocab_[t[idx]]);
            cat += vocab_[t[idx + 1]];
            auto it = index_.find(cat);
            if (it != index_.end() && scores_[it->second] > best) {
                best = scores_[it->second];
                best_id = it->second;
                best_idx = (long)idx;
            }
        }
        if (best_idx < 0) break;
        t[best_idx] = best_id;
        t.erase(t.begin() + best_idx + 1);
    }
}

bool Tokenizer::encode(const std::string& text, bool bos, bool eos, std::vector<uint32_t>* out, std::string* err) const {
    if (text.empty()) { *err = "Text to encode should not be empty"; return false; }
    std::vector<uint32_t> tokens;
    if (bos) tokens.push_back(bos_);
    if (pre_ == "gpt2" || pre_ == "smollm") {
        std::string s = text;
        if (add_space_prefix_ && text[0] != ' ') s = " " + text;
        std::vector<uint32_t> seg;
        for (const auto& r : gpt2_split(s)) {
            seg.clear();
            for (size_t k = r.first; k < r.second; k++) seg.push_back(byte_to_token_[(unsigned char)s[k]]);
            bpe_merge(&seg);
            tokens.insert(tokens.end(), seg.begin(), seg.end());
        }
    } else if (byte_level_) {
        for (unsigned char c : text) tokens.push_back(byte_to_token_[c]);
        for (uint32_t id : tokens)
            if (id >= vocab_.size()) { *err = "token id " + std::to_string(id) + " outside the vocabulary"; return false; }
        bpe_merge(&tokens);   // the BOS token takes part in the merges (tokenizer.rs:372)
    } else {
        // each character by its vocabulary entry, else its UTF-8 bytes as ids b + 3 (tokenizer.rs:356-370)
        std::vector<uint32_t> cp;
        std::vector<size_t> off;
        decode_utf8(text, &cp, &off);
        for (size_t k = 0; k < cp.size(); k++) {
            const std::string ch = text.substr(off[k], off[k + 1] - off[k]);
            auto it = index_.find(ch);
            if (it != index_.end()) tokens.push_back(it->second);
            else
                for (unsigned char b : ch) tokens.push_back((uint32_t)b + 3);
        }
        for (uint32_t id : tokens)
            if (id >= vocab_.size()) { *err = "token id " + std::to_string(id) + " outside the vocabulary"; return false; }
        bpe_merge(&tokens);
    }
    if (eos) tokens.push_back(eos_);
    out->insert(out->end(), tokens.begin(), tokens.end());
    return true;
}

std::string Tokenizer::decode(const std::vector<uint32_t>& ids) const {
    if (!byte_level_) {   // the vocabulary texts concatenated (tokenizer.rs:560-566)
        std::string text;
        for (uint32_t tid : ids)
            if (tid < vocab_.size()) text += vocab_[tid];
        return text;
    }
    std::string bytes;
    for (uint32_t tid : ids) {
        if (tid < token_to_byte_.size() && token_to_byte_[tid] >= 0) {
            bytes += (char)token_to_byte_[tid];
        } else if (tid < vocab_.size()) {
            std::vector<uint32_t> cp;
            std::vector<size_t> off;
            decode_utf8(vocab_[tid], &cp, &off);
            for (size_t k = 0; k < cp.size(); k++) {
                auto it = char_to_byte_.find(cp[k]);
                if (it != char_to_byte_.end()) bytes += (char)it->second;
                else bytes.append(vocab_[tid], off[k], off[k + 1] - off[k]);
            }
        }
    }
    return utf8_lossy(bytes);
}

bool Tokenizer::encode_wrap_n_header(const std::string& text, const std::string& header, bool bot_wrap,
                                     std::vector<uint32_t>* out, std::string* err) const {
    if (!has_llama_tokens()) {
        if (bot_wrap && add_bos_token_) out->push_back(bos_);
        if (!text.empty() && !encode(text, false, false, out, err)) return false;
        return true;
    }
    if (bot_wrap) out->push_back(kBeginOfText);
    if (!header.empty()) {
        out->push_back(kStartHeader);
        if (!encode(header, false, false, out, err)) return false;
        out->push_back(kEndHeader);
        out->push_back(kHeaderSep);
    }
    if (!text.empty() && !encode(text, false, false, out, err)) return false;
    if (bot_wrap) {
        out->push_back(kHeaderSep);
        out->push_back(kEot);
    }
    return true;
}

bool Tokenizer::render_chat_template(const std::vector<std::pair<std::string, std::string>>& messages,
                                     bool add_generation_prompt, std::vector<uint32_t>* out, std::string* err) const {
    if (!has_template_) return true;
    jinja::List msgs;
    for (const auto& m : messages)
        msgs.push_back(jinja::Value::map({{"role", jinja::Value::str(m.first)}, {"content", jinja::Value::str(m.second)}}));
    const jinja::Value ctx = jinja::Value::map(
        {{"messages", jinja::Value::list(msgs)}, {"add_generation_prompt", jinja::Value::boolean(add_generation_prompt)}});
    std::string rendered;
    if (!jinja::render(template_, ctx, &rendered, err)) return false;
    if (rendered.empty()) return true;
    return encode_template_output(rendered, out, err);
}

// tokenizer.rs:458-494: special tokens (vocabulary texts containing '<')
// by longest match at each '<', ordinary encoding of the text between.
bool Tokenizer::encode_template_output(const std::string& text, std::vector<uint32_t>* out, std::string* err) const {
    std::unordered_map<std::string, uint32_t> specials;
    size_t longest = 0;
    for (size_t tid = 0; tid < vocab_.size(); tid++)
        if (vocab_[tid].find('<') != std::string::npos) {
            specials[vocab_[tid]] = (uint32_t)tid;
            longest = std::max(longest, vocab_[tid].size());
        }
    size_t pos = 0;
    const size_t n = text.size();
    while (pos < n) {
        if (text[pos] == '<') {
            size_t best_len = 0;
            uint32_t best_id = 0;
            for (size_t len = std::min(longest, n - pos); len > best_len; len--) {
                auto it = specials.find(text.substr(pos, len));
                if (it != specials.end()) {
                    best_len = len;
                    best_id = it->second;
                }
            }
            if (best_len) {
                out->push_back(best_id);
                pos += best_len;
                continue;
            }
        }
        const size_t start = pos;
        pos++;
        while (pos < n && text[pos] != '<') pos++;
        if (!encode(text.substr(start, pos - start), false, false, out, err)) return false;
    }
    return true;
}

bool Tokenizer::apply_system_template(const std::string& system, std::vector<uint32_t>* out, std::string* err) const {
    if (has_template_) return render_chat_template({{"system", system}}, false, out, err);
    if (has_llama_tokens()) return encode_wrap_n_header(system, "system", true, out, err);
    if (!system.empty()) return encode(system, false, false, out, err);
    return true;
}

bool Tokenizer::apply_turn_template(const std::string& user, bool add_empty_assistant, std::vector<uint32_t>* out,
                                    std::string* err) const {
    if (has_template_) {
        std::vector<std::pair<std::string, std::string>> msgs{{"user", user}};
        if (add_empty_assistant) msgs.push_back({"assistant", ""});
        std::vector<uint32_t> r;
        if (!render_chat_template(msgs, add_empty_assistant, &r, err)) return false;
        if (add_empty_assistant && !r.empty() && r.back() == kEot) r.pop_back();
        out->insert(out->end(), r.begin(), r.end());
        return true;
    }
    if (has_llama_tokens()) {
        std::vector<uint32_t> user_id, assistant_id;
        if (!encode("user", false, false, &user_id, err) || !encode("assistant", false, false, &assistant_id, err))
            return false;
        if (user_id.size() != 1 || assistant_id.size() != 1) {
            *err = "expected 'user' and 'assistant' to be single tokens";
            return false;
        }
        out->push_back(kStartHeader);
        out->push_back(user_id[0]);
        out->push_back(kEndHeader);
        out->push_back(kHeaderSep);
        if (!encode_wrap_n_header(user, "", false, out, err)) return false;
        out->push_back(kEot);
        if (add_empty_assistant) {
            out->push_back(kStartHeader);
            out->push_back(assistant_id[0]);
            out->push_back(kEndHeader);
            out->push_back(kHeaderSep);
        }
        return true;
    }
    if (add_bos_token_) out->push_back(bos_);
    return encode(user, false, false, out, err);
}

// ---------------------------------------------------------------- sampler
Sampler::Sampler(size_t vocab, float temperature, float top_p, uint64_t seed)
    : vocab_(vocab), idx_(vocab, ProbIndex{0.0f, 0}), temperature_(temperature), top_p_(top_p), seed_(seed) {}

bool Sampler::sample(float* logits, uint32_t* out) {
    const size_t n = vocab_;
    if (n == 0) return false;
    if (temperature_ == 0.0f) {   // sample_argmax (sampler.rs:67-79)
        uint32_t mi = 0;
        float mp = logits[0];
        for (size_t i = 1; i < n; i++)
            if (logits[i] > mp) { mi = (uint32_t)i; mp = logits[i]; }
        *out = mi;
        return true;
    }
    for (size_t q = 0; q < n; q++) logits[q] /= temperature_;
    // softmax (sampler.rs:21-31): f32::max fold from -inf, exp, sequential sum, divide
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, logits[i]);
    float sum = -0.0f;
    for (size_t i = 0; i < n; i++) {
        logits[i] = expf(logits[i] - mx);
        sum += logits[i];
    }
    for (size_t i = 0; i < n; i++) logits[i] /= sum;
    // random_f32(seed): the xorshift state is the constant seed (sampler.rs:81-91,170)
    uint64_t st = seed_;
    st ^= st >> 12;
    st ^= st << 25;
    st ^= st >> 27;
    const uint32_t r32 = (uint32_t)((st * 0x2545F4914F6CDD1Dull) >> 32);
    const float rand = (float)(r32 >> 8) / 16777216.0f;
    if (top_p_ <= 0.0f || top_p_ >= 1.0f) {   // sample_mult
        float cdf = 0.0f;
        for (size_t i = 0; i < n; i++) {
            cdf += logits[i];
            if (rand < cdf) { *out = (uint32_t)i; return true; }
        }
        *out = (uint32_t)(n - 1);
        return true;
    }
    // sample_topp (sampler.rs:106-156): candidates at or above the cutoff
    // overwrite the front of the persistent array, then the whole array is
    // stably sorted by descending probability
    const float cutoff = (1.0f - top_p_) / (float)(n - 1);
    size_t n0 = 0;
    for (size_t i = 0; i < n; i++)
        if (logits[i] >= cutoff) idx_[n0++] = ProbIndex{logits[i], (uint32_t)i};
    std::stable_sort(idx_.begin(), idx_.end(), [](const ProbIndex& a, const ProbIndex& b) { return a.prob > b.prob; });
    if (n0 == 0) return false;
    float cum = 0.0f;
    size_t last = n0 - 1;
    for (size_t i = 0; i < n0; i++) {
        cum += idx_[i].prob;
        if (cum > top_p_) { last = i; break; }
    }
    const float r = rand * cum;
    float cdf = 0.0f;
    for (size_t i = 0; i <= last; i++) {
        cdf += idx_[i].prob;
        if (r < cdf) { *out = idx_[i].index; return true; }
    }
    *out = idx_[last].index;
    return true;
}

}  // namespace yl

namespace yl {

bool valid_utf8(const char* p) {
    const std::string t(p);
    return utf8_lossy(t) == t;
}

yl_tokenizer* tokenizer_from_gguf(const GgufFile& g, std::string* err) {
    TokenizerSpec ts;
    const GgufValue* toks = g.get("tokenizer.ggml.tokens");
    if (!toks) { *err = "tokenizer.ggml.tokens metadata key not found"; return nullptr; }
    if (toks->type != 9 || toks->arr_type != 8) { *err = "tokenizer.ggml.tokens must be an array of strings"; return nullptr; }
    ts.vocab = toks->arr_str;
    if (const GgufValue* mg = g.get("tokenizer.ggml.merges"); mg && mg->type == 9) {
        if (mg->arr_type != 8) { *err = "tokenizer.ggml.merges element not a string"; return nullptr; }
        ts.merges = mg->arr_str;
    }
    // token ids: u32/i32/u64/i64 values, else the Llama-3 defaults (:614-628)
    auto token_id = [&](const char* key, uint32_t dflt) {
        const GgufValue* v = g.get(key);
        if (!v) return dflt;
        if (v->type == 4 || v->type == 10) return (uint32_t)v->u;
        if (v->type == 5 || v->type == 11) return (uint32_t)(uint64_t)v->i;
        return dflt;
    };
    ts.bos = token_id("tokenizer.ggml.bos_token_id", 128000u);
    ts.eos = token_id("tokenizer.ggml.eos_token_id", 128009u);
    if (const GgufValue* pr = g.get("tokenizer.ggml.pre"); pr && pr->type == 8) ts.pre = pr->s;
    auto opt_bool = [&](const char* key, bool dflt) {   // get_metadata_optional_bool (:147-155)
        const GgufValue* v = g.get(key);
        if (!v) return dflt;
        if (v->type == 7 || v->type == 0 || v->type == 4 || v->type == 10) return v->u != 0;
        return dflt;
    };
    ts.add_bos_token = opt_bool("tokenizer.ggml.add_bos_token", true);
    ts.add_space_prefix = opt_bool("tokenizer.ggml.add_space_prefix", false);
    if (const GgufValue* ct = g.get("tokenizer.chat_template"); ct && ct->type == 8) {
        ts.has_template = true;
        ts.chat_template = ct->s;
    }
    return new yl_tokenizer{Tokenizer(std::move(ts))};
}

yl_tokenizer* tokenizer_from_hf_json(const std::string& path, std::string* err) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) { *err = "cannot open " + path; return nullptr; }
    std::string text;
    char buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, k);
    fclose(f);
    json::Value root;
    if (!json::parse(text, &root, err)) return nullptr;
    const json::Value* model = root.get("model");
    const json::Value* vocab = model ? model->get("vocab") : nullptr;
    const json::Value* added = root.get("added_tokens");
    const json::Value* merges = model ? model->get("merges") : nullptr;
    if (!vocab || vocab->kind != json::Value::kObj || !added || added->kind != json::Value::kArr || !merges ||
        merges->kind != json::Value::kArr) {
        *err = "tokenizer.json: model.vocab, model.merges and added_tokens are required";
        return nullptr;
    }
    uint64_t max_id = 0, id = 0;
    for (const auto& kv : vocab->obj) {
        if (!kv.second.as_u64(&id)) { *err = "tokenizer.json: vocabulary ids must be integers"; return nullptr; }
        max_id = std::max(max_id, id);
    }
    for (const auto& t : added->arr) {
        const json::Value* v = t.get("id");
        if (!v || !v->as_u64(&id) || !t.get("content") || !t.get("content")->as_str()) {
            *err = "tokenizer.json: added_tokens need id and content";
            return nullptr;
        }
        max_id = std::max(max_id, id);
    }
    if (max_id > 10000000) { *err = "tokenizer.json: vocabulary id out of range"; return nullptr; }
    TokenizerSpec ts;
    ts.vocab.assign(max_id + 1, std::string());
    for (const auto& kv : vocab->obj) {
        kv.second.as_u64(&id);
        ts.vocab[id] = kv.first;
    }
    for (const auto& t : added->arr) {
        t.get("id")->as_u64(&id);
        ts.vocab[id] = *t.get("content")->as_str();
    }
    for (const auto& m : merges->arr) {
        if (!m.as_str()) { *err = "tokenizer.json: merges must be strings"; return nullptr; }
        ts.merges.push_back(*m.as_str());
    }
    ts.bos = 128000u;
    ts.eos = 128009u;
    for (const auto& t : added->arr) {
        const std::string& c = *t.get("content")->as_str();
        t.get("id")->as_u64(&id);
        if (c == "<|begin_of_text|>") ts.bos = (uint32_t)id;
        if (c == "<|end_of_text|>" || c == "<|eot_id|>") ts.eos = (uint32_t)id;
    }
    return new yl_tokenizer{Tokenizer(std::move(ts))};
}

yl_tokenizer* tokenizer_from_llama2c(const std::string& path, std::string* err) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) { *err = "cannot open " + path; return nullptr; }
    std::string d;
    char buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof buf, f)) > 0) d.append(buf, k);
    fclose(f);
    auto u32 = [&](size_t o) { uint32_t v; memcpy(&v, d.data() + o, 4); return v; };
    if (d.size() < 16) { *err = "tokenizer.bin: too short"; return nullptr; }
    TokenizerSpec ts;
    const uint32_t n = u32(0);
    ts.bos = u32(8);
    ts.eos = u32(12);
    ts.byte_level = false;
    ts.has_scores = true;
    size_t o = 16;
    for (uint32_t i = 0; i < n; i++) {
        if (o + 8 > d.size()) { *err = "tokenizer.bin: truncated"; return nullptr; }
        float sc;
        memcpy(&sc, d.data() + o, 4);
        const uint32_t len = u32(o + 4);
        o += 8;
        if (o + len > d.size()) { *err = "tokenizer.bin: truncated"; return nullptr; }
        std::string t = d.substr(o, len);
        if (!valid_utf8(t.c_str()) || t.find('\0') != std::string::npos) {
            *err = "tokenizer.bin: a token is not UTF-8";
            return nullptr;
        }
        ts.vocab.push_back(std::move(t));
        ts.scores.push_back(sc);
        o += len;
    }
    return new yl_tokenizer{Tokenizer(std::move(ts))};
}

}  // namespace yl

using namespace yl;

namespace {

yl_status put_ids(const std::vector<uint32_t>& ids, uint32_t* out, size_t cap, size_t* n) {
    if (n) *n = ids.size();
    if (ids.size() > cap) {
        set_error("output holds " + std::to_string(cap) + " ids, the result has " + std::to_string(ids.size()));
        return YL_ERR_RANGE;
    }
    if (out && !ids.empty()) memcpy(out, ids.data(), ids.size() * 4);
    return YL_OK;
}

}  // namespace

extern "C" {

yl_tokenizer* yl_tokenizer_load(const char* path) {
    if (!path) { set_error("tokenizer_load: null path"); return nullptr; }
    const std::string p = path;
    auto ends = [&](const char* x) {
        const size_t n = strlen(x);
        return p.size() >= n && p.compare(p.size() - n, n, x) == 0;
    };
    std::string err;
    yl_tokenizer* t = nullptr;
    if (ends(".json")) t = tokenizer_from_hf_json(p, &err);
    else if (ends(".bin")) t = tokenizer_from_llama2c(p, &err);
    else {
        GgufFile g;
        if (!g.open(path, &err)) { set_error(err); return nullptr; }
        t = tokenizer_from_gguf(g, &err);
    }
    if (!t) set_error(err);
    return t;
}

void yl_tokenizer_free(yl_tokenizer* t) { delete t; }

size_t yl_tokenizer_vocab_size(const yl_tokenizer* t) { return t ? t->t.vocab_size() : 0; }

yl_status yl_tokenize(const yl_tokenizer* t, const char* text, int32_t bos, int32_t eos, uint32_t* out, size_t cap,
                      size_t* n) {
    if (!t || !text) { set_error("tokenize: null argument"); return YL_ERR_ARG; }
    if (!valid_utf8(text)) { set_error("tokenize: text is not UTF-8"); return YL_ERR_ARG; }
    std::vector<uint32_t> ids;
    std::string err;
    if (!t->t.encode(text, bos != 0, eos != 0, &ids, &err)) { set_error(err); return YL_ERR_ARG; }
    return put_ids(ids, out, cap, n);
}

yl_status yl_detokenize(const yl_tokenizer* t, const uint32_t* ids, size_t n, char* out, size_t cap, size_t* len) {
    if (!t || (!ids && n)) { set_error("detokenize: null argument"); return YL_ERR_ARG; }
    const std::string s = t->t.decode(std::vector<uint32_t>(ids, ids + n));
    if (len) *len = s.size();
    if (s.size() + 1 > cap) { set_error("detokenize: output buffer too small"); return YL_ERR_RANGE; }
    if (out) memcpy(out, s.c_str(), s.size() + 1);
    return YL_OK;
}

yl_status yl_chat_template(const yl_tokenizer* t, int32_t which, const char* text, int32_t flag, uint32_t* out,
                           size_t cap, size_t* n) {
    if (!t || !text || which < 0 || which > 2) { set_error("chat_template: bad arguments"); return YL_ERR_ARG; }
    if (!valid_utf8(text)) { set_error("chat_template: text is not UTF-8"); return YL_ERR_ARG; }
    std::vector<uint32_t> ids;
    std::string err;
    const bool ok = which == 0   ? t->t.apply_system_template(text, &ids, &err)
                    : which == 1 ? t->t.apply_turn_template(text, flag != 0, &ids, &err)
                                 : t->t.encode_wrap_n_header(text, "", flag != 0, &ids, &err);
    if (!ok) { set_error(err); return YL_ERR_ARG; }
    return put_ids(ids, out, cap, n);
}

yl_status yl_chat_prompt(const yl_tokenizer* t, const char* user, uint32_t* out, size_t cap, size_t* n) {
    if (!t || !user) { set_error("chat_prompt: null argument"); return YL_ERR_ARG; }
    if (!valid_utf8(user)) { set_error("chat_prompt: text is not UTF-8"); return YL_ERR_ARG; }
    const std::string u = trim_unicode(user);
    if (u.empty()) { set_error("chat_prompt: empty prompt"); return YL_ERR_ARG; }
    std::vector<uint32_t> ids;
    std::string err;
    bool ok = true;
    if (!t->t.has_chat_template()) ok = t->t.apply_system_template("", &ids, &err);
    else if (t->t.add_bos_token()) ids.push_back(t->t.bos());
    if (!ok || !t->t.apply_turn_template(u, true, &ids, &err)) { set_error(err); return YL_ERR_ARG; }
    return put_ids(ids, out, cap, n);
}

yl_status yl_pretokenize(const char* text, uint32_t* bounds, size_t cap, size_t* n) {
    if (!text) { set_error("pretokenize: null text"); return YL_ERR_ARG; }
    if (!valid_utf8(text)) { set_error("pretokenize: text is not UTF-8"); return YL_ERR_ARG; }
    std::vector<uint32_t> b;
    for (const auto& r : gpt2_split(text)) {
        b.push_back((uint32_t)r.first);
        b.push_back((uint32_t)r.second);
    }
    return put_ids(b, bounds, cap, n);
}

yl_sampler* yl_sampler_new(size_t vocab, float temperature, float top_p, uint64_t seed) {
    if (vocab == 0) { set_error("sampler: empty vocabulary"); return nullptr; }
    return new yl_sampler{Sampler(vocab, temperature, top_p, seed)};
}

yl_status yl_sampler_sample(yl_sampler* s, float* logits, uint32_t* token) {
    if (!s || !logits || !token) { set_error("sampler: null argument"); return YL_ERR_ARG; }
    if (!s->s.sample(logits, token)) { set_error("sampler: no token above the top-p cutoff"); return YL_ERR_ARG; }
    return YL_OK;
}

void yl_sampler_free(yl_sampler* s) { delete s; }

}  // extern "C"
