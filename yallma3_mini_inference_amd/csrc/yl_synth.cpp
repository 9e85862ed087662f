// yl_synth.cpp -- deterministic synthetic GGUF v3 llama models.
//
// The reference only runs models from files (transformer_llama_gguf.rs:183),
// so benchmarks and parity tests need model files of the published shapes
// with seeded random weights.  Values depend only on (seed, tensor stream,
// element index): any thread count, any machine, same bytes.  No libm call
// is involved (log/sin/cos below are plain binary64 arithmetic; build with
// -ffp-contract=off), so the files are identical wherever they are written.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <thread>
#include <vector>

#include "yallma3.h"
#include "yl_internal.h"

namespace {

inline uint64_t mix64(uint64_t z) {  // splitmix64 output function
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// ln(u) for u in (0, 1]: u = m*2^e with m in [sqrt(1/2), sqrt(2)),
// ln m = 2*atanh(s), s = (m-1)/(m+1), series to s^21.
double det_log(double u) {
    uint64_t bits;
    memcpy(&bits, &u, 8);
    int e = (int)((bits >> 52) & 0x7ff) - 1023;
    bits = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull;  // m in [1,2)
    double m;
    memcpy(&m, &bits, 8);
    if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double p = 1.0 / 21.0;
    for (int k = 19; k >= 1; k -= 2) p = p * s2 + 1.0 / (double)k;
    return 2.0 * s * p + (double)e * 0x1.62e42fefa39efp-1;
}

// sin and cos of t in [0, pi/2] by Taylor series (degree 21/22).
void det_sincos_q(double t, double* s_out, double* c_out) {
    const double t2 = t * t;
    double s = 0.0, c = 0.0, ts = t, tc = 1.0;
    for (int k = 0; k < 11; k++) {
        const double sign = (k & 1) ? -1.0 : 1.0;
        s = s + sign * ts;
        c = c + sign * tc;
        ts = ts * t2 / (double)((2 * k + 2) * (2 * k + 3));
        tc = tc * t2 / (double)((2 * k + 1) * (2 * k + 2));
    }
    *s_out = s;
    *c_out = c;
}

// Box-Muller normal for element i of a stream: pair i/2 uses counters 2p, 2p+1.
inline float normal_at(uint64_t base, uint64_t i, float std_dev) {
    const uint64_t p = i >> 1;
    const uint64_t a = mix64(base + (2 * p) * 0x9E3779B97F4A7C15ull);
    const uint64_t b = mix64(base + (2 * p + 1) * 0x9E3779B97F4A7C15ull);
    const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;   // (0, 1]
    const double u2 = (double)(b >> 11) * 0x1.0p-53;         // [0, 1)
    const double r = sqrt(-2.0 * det_log(u1));
    const double q4 = u2 * 4.0;
    const int quad = (int)q4;
    const double th = (q4 - (double)quad) * 0x1.921fb54442d18p+0;  // * pi/2
    double s, c;
    det_sincos_q(th, &s, &c);
    double cs, sn;  // cos/sin of 2*pi*u2
    switch (quad) {
    case 0: cs = c; sn = s; break;
    case 1: cs = -s; sn = c; break;
    case 2: cs = -c; sn = -s; break;
    default: cs = s; sn = -c; break;
    }
    const double z = (i & 1) ? r * sn : r * cs;
    return (float)(z * (double)std_dev);
}

inline uint64_t stream_base(uint64_t seed, uint64_t stream) {
    return mix64(seed ^ mix64(stream + 0x632BE59BD9B4E019ull));
}

// binary32 -> binary16, round to nearest even (overflow -> inf).
uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) {                                   // f16 subnormal or zero
        if (ax < 0x33000000u) return (uint16_t)sign;          // < 2^-25 -> 0
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)e;                       // 14..24
        uint32_t v = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (v & 1u))) v++;
        return (uint16_t)(sign | v);
    }
    uint32_t v = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) v++;
    return (uint16_t)(sign | v);
}

template <class F>
void parallel_for(size_t n, F&& fn) {
    unsigned nt = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
    if (n < 4096) nt = 1;
    std::vector<std::thread> th;
    const size_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        const size_t b = t * chunk, e = std::min(n, b + chunk);
        if (b >= e) break;
        th.emplace_back([=, &fn] { for (size_t i = b; i < e; i++) fn(i); });
    }
    for (auto& x : th) x.join();
}

// ggml quantize_row_q8_0: d = amax/127, q = round(x * (1/d)), 34-byte blocks.
void quant_q8_0(const float* x, size_t blocks, uint8_t* out) {
    parallel_for(blocks, [&](size_t b) {
        const float* v = x + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = std::max(amax, fabsf(v[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t* blk = out + b * 34;
        const uint16_t h = f32_to_f16(d);
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) blk[2 + j] = (uint8_t)(int8_t)lroundf(v[j] * id);
    });
}

// ggml quantize_row_q4_0: d = max/-8 (max = the signed value of largest |x|),
// q = min(15, (int8)(x*(1/d) + 8.5)), element j -> low nibble of byte j,
// element j+16 -> high nibble.  18-byte blocks.
void quant_q4_0(const float* x, size_t blocks, uint8_t* out) {
    parallel_for(blocks, [&](size_t b) {
        const float* v = x + b * 32;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; j++)
            if (amax < fabsf(v[j])) { amax = fabsf(v[j]); mx = v[j]; }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t* blk = out + b * 18;
        const uint16_t h = f32_to_f16(d);
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 16; j++) {
            const int a = std::min(15, (int)(int8_t)(v[j] * id + 8.5f));
            const int c = std::min(15, (int)(int8_t)(v[16 + j] * id + 8.5f));
            blk[2 + j] = (uint8_t)(a | (c << 4));
        }
    });
}

struct Writer {
    FILE* f = nullptr;
    bool ok = true;
    void bytes(const void* p, size_t n) { if (ok && fwrite(p, 1, n, f) != n) ok = false; }
    void u32(uint32_t v) { bytes(&v, 4); }
    void u64(uint64_t v) { bytes(&v, 8); }
    void f32(float v) { bytes(&v, 4); }
    void str(const std::string& s) { u64(s.size()); bytes(s.data(), s.size()); }
    void kv_str(const char* k, const std::string& v) { str(k); u32(8); str(v); }
    void kv_u32(const char* k, uint32_t v) { str(k); u32(4); u32(v); }
    void kv_f32(const char* k, float v) { str(k); u32(6); f32(v); }
};

struct TensorSpec {
    std::string name;
    uint64_t ne0, ne1;   // ne0 = row length n, ne1 = rows (1 for vectors)
    uint32_t type;       // GGML type id
    uint64_t offset;
    uint64_t bytes;
};

constexpr uint32_t kGgmlF32 = 0, kGgmlF16 = 1, kGgmlQ4_0 = 2, kGgmlQ8_0 = 8;

uint32_t ggml_type_of(int fmt) {
    return fmt == YL_Q4_0 ? kGgmlQ4_0 : (fmt == YL_F16 ? kGgmlF16 : kGgmlQ8_0);
}

uint64_t tensor_bytes(uint32_t type, uint64_t n) {
    switch (type) {
    case kGgmlF32: return n * 4;
    case kGgmlF16: return n * 2;
    case kGgmlQ4_0: return n / 32 * 18;
    default: return n / 32 * 34;
    }
}

}  // namespace

extern "C" yl_status yl_synthetic_normal(uint64_t seed, uint64_t stream, uint64_t first, size_t count,
                                         float std_dev, float* out) {
    if (!out && count) return YL_ERR_ARG;
    const uint64_t base = stream_base(seed, stream);
    parallel_for(count, [&](size_t i) { out[i] = normal_at(base, first + i, std_dev); });
    return YL_OK;
}

static yl_status write_gguf(const char* path, const yl_synth_config* c, const yl_synth_tokenizer* tk);

extern "C" yl_status yl_write_synthetic_gguf(const char* path, const yl_synth_config* c) {
    return write_gguf(path, c, nullptr);
}

extern "C" yl_status yl_write_synthetic_gguf_tok(const char* path, const yl_synth_config* c,
                                                 const yl_synth_tokenizer* tk) {
    if (!tk || !tk->tokens || (tk->n_merges && !tk->merges)) {
        yl::set_error("yl_write_synthetic_gguf_tok: null tokenizer arrays");
        return YL_ERR_ARG;
    }
    if (!c || tk->n_tokens != c->vocab) {
        yl::set_error("yl_write_synthetic_gguf_tok: the token list must hold cfg->vocab strings");
        return YL_ERR_ARG;
    }
    return write_gguf(path, c, tk);
}

static yl_status write_gguf(const char* path, const yl_synth_config* c, const yl_synth_tokenizer* tk) {
    if (!path || !c || !c->dim || !c->n_heads || c->dim % c->n_heads || !c->n_layers || !c->vocab ||
        c->dim % 32 || c->hidden % 32 || !c->n_kv_heads || c->n_heads % c->n_kv_heads) {
        yl::set_error("yl_write_synthetic_gguf: invalid config");
        return YL_ERR_ARG;
    }
    const uint32_t hd = c->dim / c->n_heads;
    const uint64_t att = c->dim, kv = (uint64_t)c->n_kv_heads * hd;
    if (kv % 32) { yl::set_error("yl_write_synthetic_gguf: kv_dim must be a multiple of 32"); return YL_ERR_ARG; }
    std::vector<TensorSpec> ts;
    auto add = [&](const std::string& nm, uint64_t ne0, uint64_t ne1, uint32_t type) {
        ts.push_back({nm, ne0, ne1, type, 0, tensor_bytes(type, ne0 * ne1)});
    };
    const uint32_t ta = ggml_type_of(c->attn_format), tf = ggml_type_of(c->ffn_format);
    add("token_embd.weight", c->dim, c->vocab, ggml_type_of(c->embd_format));
    add("output_norm.weight", c->dim, 1, kGgmlF32);
    for (uint32_t l = 0; l < c->n_layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        add(p + "attn_norm.weight", c->dim, 1, kGgmlF32);
        add(p + "attn_q.weight", c->dim, att, ta);
        add(p + "attn_k.weight", c->dim, kv, ta);
        add(p + "attn_v.weight", c->dim, kv, ta);
        add(p + "attn_output.weight", att, c->dim, ta);
        add(p + "ffn_norm.weight", c->dim, 1, kGgmlF32);
        add(p + "ffn_gate.weight", c->dim, c->hidden, tf);
        add(p + "ffn_up.weight", c->dim, c->hidden, tf);
        add(p + "ffn_down.weight", c->hidden, c->dim, tf);
    }
    const uint64_t align = 32;
    uint64_t off = 0;
    for (auto& t : ts) {
        t.offset = off;
        off = (off + t.bytes + align - 1) / align * align;
    }

    Writer w;
    w.f = fopen(path, "wb");
    if (!w.f) { yl::set_error(std::string("cannot create ") + path); return YL_ERR_IO; }
    const uint32_t n_kv = 15 + (c->rope_scaling ? 4 : 0) + (c->attention_scale != 0.0f ? 1 : 0) +
                          (tk ? (tk->n_merges ? 1 : 0) + (tk->pre ? 1 : 0) + (tk->chat_template ? 1 : 0) +
                                    (tk->add_bos_token >= 0 ? 1 : 0) + (tk->add_space_prefix >= 0 ? 1 : 0)
                              : 0);
    w.u32(0x46554747u);
    w.u32(3);
    w.u64(ts.size());
    w.u64(n_kv);
    w.kv_str("general.architecture", "llama");
    w.kv_str("general.name", "yallma3-synthetic");
    w.kv_u32("general.alignment", (uint32_t)align);
    w.kv_u32("general.file_type", (uint32_t)c->file_type);
    w.kv_u32("llama.context_length", c->ctx_len);
    w.kv_u32("llama.embedding_length", c->dim);
    w.kv_u32("llama.feed_forward_length", c->hidden);
    w.kv_u32("llama.block_count", c->n_layers);
    w.kv_u32("llama.attention.head_count", c->n_heads);
    w.kv_u32("llama.attention.head_count_kv", c->n_kv_heads);
    w.kv_f32("llama.attention.layer_norm_rms_epsilon", c->rms_eps);
    w.kv_f32("llama.rope.freq_base", c->rope_theta);
    if (c->rope_scaling) {
        // the YaRN keys rope_gguf reads (transformer_llama_gguf.rs:242-248)
        w.kv_f32("llama.rope.scaling.factor", c->rope_scaling_factor);
        w.kv_f32("llama.rope.scaling.ext_factor", c->rope_ext_factor);
        w.kv_f32("llama.rope.scaling.attn_factor", c->rope_attn_factor);
        w.kv_u32("llama.rope.scaling.original_context_length", c->rope_original_ctx);
    }
    if (c->attention_scale != 0.0f) w.kv_f32("llama.attention.scale", c->attention_scale);
    w.kv_u32("tokenizer.ggml.bos_token_id", tk ? tk->bos : 1);
    w.kv_u32("tokenizer.ggml.eos_token_id", tk ? tk->eos : 2);
    w.str("tokenizer.ggml.tokens");
    w.u32(9);
    w.u32(8);
    w.u64(c->vocab);
    for (uint32_t i = 0; i < c->vocab; i++) w.str(tk ? std::string(tk->tokens[i]) : "<t" + std::to_string(i) + ">");
    if (tk) {
        if (tk->n_merges) {
            w.str("tokenizer.ggml.merges");
            w.u32(9);
            w.u32(8);
            w.u64(tk->n_merges);
            for (size_t i = 0; i < tk->n_merges; i++) w.str(tk->merges[i]);
        }
        if (tk->pre) w.kv_str("tokenizer.ggml.pre", tk->pre);
        if (tk->chat_template) w.kv_str("tokenizer.chat_template", tk->chat_template);
        auto kv_bool = [&](const char* k, int v) { w.str(k); w.u32(7); const uint8_t b = v ? 1 : 0; w.bytes(&b, 1); };
        if (tk->add_bos_token >= 0) kv_bool("tokenizer.ggml.add_bos_token", tk->add_bos_token);
        if (tk->add_space_prefix >= 0) kv_bool("tokenizer.ggml.add_space_prefix", tk->add_space_prefix);
    }
    for (const auto& t : ts) {
        w.str(t.name);
        const bool vec = t.ne1 == 1;
        w.u32(vec ? 1 : 2);
        w.u64(t.ne0);
        if (!vec) w.u64(t.ne1);
        w.u32(t.type);
        w.u64(t.offset);
    }
    long pos = ftell(w.f);
    std::vector<uint8_t> pad(align, 0);
    const uint64_t data_start = ((uint64_t)pos + align - 1) / align * align;
    w.bytes(pad.data(), data_start - (uint64_t)pos);

    std::vector<float> vals;
    std::vector<uint8_t> blob;
    uint64_t written = 0;
    for (size_t ti = 0; ti < ts.size(); ti++) {
        const auto& t = ts[ti];
        const uint64_t n = t.ne0 * t.ne1;
        if (t.offset > written) { w.bytes(pad.data(), t.offset - written); written = t.offset; }
        blob.assign(t.bytes, 0);
        if (t.type == kGgmlF32) {
            for (uint64_t i = 0; i < n; i++) { const float one = 1.0f; memcpy(blob.data() + 4 * i, &one, 4); }
        } else {
            vals.resize(n);
            const uint64_t base = stream_base(c->seed, ti);
            const float sd = c->weight_std;
            parallel_for(n, [&](size_t i) { vals[i] = normal_at(base, i, sd); });
            if (t.type == kGgmlQ8_0) quant_q8_0(vals.data(), n / 32, blob.data());
            else if (t.type == kGgmlQ4_0) quant_q4_0(vals.data(), n / 32, blob.data());
            else
                for (uint64_t i = 0; i < n; i++) {
                    const uint16_t h = f32_to_f16(vals[i]);
                    memcpy(blob.data() + 2 * i, &h, 2);
                }
        }
        w.bytes(blob.data(), blob.size());
        written += blob.size();
    }
    const bool ok = w.ok;
    if (fclose(w.f) != 0 || !ok) {
        yl::set_error(std::string("write failed: ") + path);
        return YL_ERR_IO;
    }
    return YL_OK;
}
