// yl_json.h -- a small JSON reader for the safetensors header, config.json
// and tokenizer.json (RFC 8259 values; numbers kept as double plus, for
// integers, an exact int64/uint64).  Object members keep file order.
#pragma once

#include <stdint.h>
#include <stdlib.h>

#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace yl {
namespace json {

struct Value {
    enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
    bool b = false;
    double num = 0.0;
    bool is_int = false;     // the literal had no fraction or exponent
    bool neg = false;
    uint64_t mag = 0;        // |integer| when is_int (saturating)
    std::string s;
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;

    const Value* get(const std::string& k) const {
        if (kind != kObj) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    // serde_json's as_u64: a non-negative integer literal
    bool as_u64(uint64_t* out) const {
        if (kind != kNum || !is_int || neg) return false;
        *out = mag;
        return true;
    }
    // serde_json's as_f64: any number
    bool as_f64(double* out) const {
        if (kind != kNum) return false;
        *out = num;
        return true;
    }
    const std::string* as_str() const { return kind == kStr ? &s : nullptr; }
};

class Parser {
public:
    Parser(const char* p, size_t n) : p_(p), e_(p + n) {}

    bool parse(Value* v, std::string* err) {
        ws();
        if (!value(v, 0)) { *err = "JSON: " + err_ + " at byte " + std::to_string(pos()); return false; }
        ws();
        if (p_ != e_) { *err = "JSON: trailing characters at byte " + std::to_string(pos()); return false; }
        return true;
    }

private:
    const char* p_;
    const char* e_;
    const char* b_ = p_;
    std::string err_;

    size_t pos() const { return (size_t)(p_ - b_); }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool fail(const char* m) { err_ = m; return false; }
    bool lit(const char* s) {
        size_t n = 0;
        while (s[n]) n++;
        if ((size_t)(e_ - p_) < n) return false;
        for (size_t k = 0; k < n; k++)
            if (p_[k] != s[k]) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) { o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
        else {
            o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F));
            o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t* out) {
        if (e_ - p_ < 4) return false;
        uint32_t v = 0;
        for (int k = 0; k < 4; k++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        *out = v;
        return true;
    }
    bool string(std::string* o) {
        p_++;   // opening quote
        while (p_ < e_) {
            const char c = *p_++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return fail("control character in a string");
            if (c != '\\') { *o += c; continue; }
            if (p_ >= e_) break;
            const char x = *p_++;
            switch (x) {
            case '"': *o += '"'; break;
            case '\\': *o += '\\'; break;
            case '/': *o += '/'; break;
            case 'b': *o += '\b'; break;
            case 'f': *o += '\f'; break;
            case 'n': *o += '\n'; break;
            case 'r': *o += '\r'; break;
            case 't': *o += '\t'; break;
            case 'u': {
                uint32_t cp;
                if (!hex4(&cp)) return fail("bad \\u escape");
                if (cp >= 0xD800 && cp <= 0xDBFF) {   // surrogate pair
                    uint32_t lo;
                    if (e_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
                    p_ += 2;
                    if (!hex4(&lo) || lo < 0xDC00 || lo > 0xDFFF) return fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
                    return fail("lone surrogate");
                }
                put_utf8(*o, cp);
                break;
            }
            default: return fail("bad escape");
            }
        }
        return fail("unterminated string");
    }
    bool number(Value* v) {
        const char* s = p_;
        if (p_ < e_ && *p_ == '-') { v->neg = true; p_++; }
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return fail("bad number");
        uint64_t mag = 0;
        bool sat = false;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_++ - '0');
            if (mag > (UINT64_MAX - d) / 10) sat = true;
            else mag = mag * 10 + d;
        }
        bool frac = false;
        if (p_ < e_ && *p_ == '.') {
            frac = true;
            p_++;
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') p_++;
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            p_++;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) p_++;
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') p_++;
        }
        v->kind = Value::kNum;
        v->num = strtod(std::string(s, p_).c_str(), nullptr);
        v->is_int = !frac && !sat;
        v->mag = mag;
        return true;
    }
    bool value(Value* v, int depth) {
        if (depth > 256) return fail("nesting too deep");
        if (p_ >= e_) return fail("unexpected end");
        const char c = *p_;
        if (c == '{') {
            p_++;
            v->kind = Value::kObj;
            ws();
            if (p_ < e_ && *p_ == '}') { p_++; return true; }
            for (;;) {
                ws();
                if (p_ >= e_ || *p_ != '"') return fail("expected a key");
                std::string k;
                if (!string(&k)) return false;
                ws();
                if (p_ >= e_ || *p_ != ':') return fail("expected ':'");
                p_++;
                ws();
                v->obj.emplace_back(std::move(k), Value());
                if (!value(&v->obj.back().second, depth + 1)) return false;
                ws();
                if (p_ < e_ && *p_ == ',') { p_++; continue; }
                if (p_ < e_ && *p_ == '}') { p_++; return true; }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            p_++;
            v->kind = Value::kArr;
            ws();
            if (p_ < e_ && *p_ == ']') { p_++; return true; }
            for (;;) {
                ws();
                v->arr.emplace_back();
                if (!value(&v->arr.back(), depth + 1)) return false;
                ws();
                if (p_ < e_ && *p_ == ',') { p_++; continue; }
                if (p_ < e_ && *p_ == ']') { p_++; return true; }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') { v->kind = Value::kStr; return string(&v->s); }
        if (lit("true")) { v->kind = Value::kBool; v->b = true; return true; }
        if (lit("false")) { v->kind = Value::kBool; v->b = false; return true; }
        if (lit("null")) { v->kind = Value::kNull; return true; }
        return number(v);
    }
};

inline bool parse(const std::string& text, Value* v, std::string* err) {
    Parser p(text.data(), text.size());
    return p.parse(v, err);
}

}  // namespace json
}  // namespace yl
