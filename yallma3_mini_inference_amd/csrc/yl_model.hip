// yl_model.hip -- model loading, device repack, sessions, the forward driver
// (eager for prompts, one HIP graph per decode step) and the C ABI.
//
// Mirrors the reference's Transformer trait (transformer.rs:19-69) and
// llama_forward_x (forward.rs:120-297): per layer
//   RMSNorm -> quantize -> Q,K,V matmuls (K/V += into the cache) -> RoPE ->
//   attention -> quantize -> WO -> residual -> RMSNorm -> quantize ->
//   W1,W3 -> SwiGLU -> quantize -> W2 -> residual,
// then the final RMSNorm and the tied-embedding logits of the last token.
// Kernel fusion (same arithmetic, fewer launches), per layer:
//   (layer 0: token embedding +) RMSNorm + quantize + Q/K/V matmul
//     + K/V cache accumulate + RoPE                   k_gemv<..., kEpiQkvRope>
//   attention + quantize                              k_attn_decode (one token),
//                                                     k_attention (prompt batch)
//   WO matmul + residual                              k_gemv<..., kEpiResid>
//   RMSNorm + quantize + W1/W3 matmul + SwiGLU
//     + quantize                                      k_gemv<..., kEpiSwiglu>
//   W2 matmul + residual                              k_gemv<..., kEpiResid>
// then final RMSNorm + logits + argmax (k_logits) and the step bookkeeping
// (k_finalize).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "yallma3.h"
#include "yl_gguf.h"
#include "yl_host_model.h"
#include "yl_tokenizer.h"
#include "yl_internal.h"

namespace yl {

thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }

constexpr uint32_t kGgmlF32 = 0, kGgmlF16 = 1, kGgmlQ4_0 = 2, kGgmlQ8_0 = 8;

static float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// binary32 -> binary16 when exact; false otherwise.
static bool float_to_half_exact(float f, uint16_t* out) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    uint16_t h;
    if (ax == 0) {
        h = (uint16_t)sign;
    } else if (ax >= 0x7f800000u) {
        h = (uint16_t)(sign | 0x7c00u | ((ax & 0x7fffffu) ? 0x200u : 0u));
    } else if (ax >= 0x38800000u && ax < 0x47800000u) {
        if (ax & 0x1fffu) return false;
        h = (uint16_t)(sign | ((ax >> 13) - (112u << 10)));
    } else if (ax < 0x38800000u) {
        const int e = (int)(ax >> 23);
        const uint32_t m = (ax & 0x7fffffu) | (e ? 0x800000u : 0u);
        const int shift = 126 - e;
        if (e == 0 || shift > 24 || (m & ((1u << shift) - 1u))) return false;
        h = (uint16_t)(sign | (m >> shift));
    } else {
        return false;
    }
    *out = h;
    return half_to_float(h) == f || (f != f);
}

// Host staging of one device matrix in the repacked layout.
struct HostQMat {
    int fmt = kQ8;
    size_t o = 0, n = 0, nb = 0;
    std::vector<uint8_t> qs;
    std::vector<uint16_t> d;
    size_t row_bytes() const { return fmt == kQ4 ? n / 2 : fmt == kF16 ? n * 2 : n; }
};

// F16 gate and up rows in the pairs the one-token F16 GEMV's SwiGLU epilogue
// reads: blocks of 64 rows, 32 gate rows then the same 32 up rows.
static void f16_pair_rows(const uint16_t* gate, const uint16_t* up, size_t o, size_t n, HostQMat* out) {
    out->fmt = kF16;
    out->o = 2 * o;
    out->n = n;
    out->qs.resize(2 * o * n * 2);
    uint16_t* dst = reinterpret_cast<uint16_t*>(out->qs.data());
    for (size_t r0 = 0; r0 < o; r0 += kF16PairRows)
        for (int k = 0; k < 2; k++) {
            const uint16_t* src = (k == 0 ? gate : up) + r0 * n;
            memcpy(dst, src, kF16PairRows * n * 2);
            dst += kF16PairRows * n;
        }
}

// GGUF blocks -> repacked planes (transformer_llama_gguf.rs:345-410).
static bool host_from_gguf(uint32_t type, const uint8_t* src, uint64_t avail, size_t o, size_t n,
                           HostQMat* h, std::string* err) {
    if (n % 32) { *err = "row length must be a multiple of 32"; return false; }
    h->o = o; h->n = n; h->nb = n / 32;
    const size_t blocks = o * h->nb;
    if (type == kGgmlQ8_0) {
        if (blocks * 34 > avail) { *err = "Q8_0 tensor exceeds the file"; return false; }
        h->fmt = kQ8;
        h->qs.resize(o * n);
        h->d.resize(blocks);
        for (size_t b = 0; b < blocks; b++) {
            const uint8_t* blk = src + b * 34;
            h->d[b] = (uint16_t)(blk[0] | (blk[1] << 8));
            memcpy(&h->qs[b * 32], blk + 2, 32);
        }
        return true;
    }
    if (type == kGgmlQ4_0) {
        if (blocks * 18 > avail) { *err = "Q4_0 tensor exceeds the file"; return false; }
        h->fmt = kQ4;
        h->qs.resize(o * n / 2);
        h->d.resize(blocks);
        for (size_t b = 0; b < blocks; b++) {
            const uint8_t* blk = src + b * 18;
            h->d[b] = (uint16_t)(blk[0] | (blk[1] << 8));
            memcpy(&h->qs[b * 16], blk + 2, 16);
        }
        return true;
    }
    if (type == kGgmlF16) {   // load_f16_tensor (transformer_llama_gguf.rs:412-421): kept as f16 bits
        if (o * n * 2 > avail) { *err = "F16 tensor exceeds the file"; return false; }
        h->fmt = kF16;
        h->nb = 0;
        h->qs.assign(src, src + o * n * 2);
        return true;
    }
    *err = "unsupported tensor type " + std::to_string(type) + " (Q8_0, Q4_0 and F16 are built)";
    return false;
}

static bool host_concat_rows(const std::vector<const HostQMat*>& parts, HostQMat* out, std::string* err) {
    out->fmt = parts[0]->fmt; out->n = parts[0]->n; out->nb = parts[0]->nb; out->o = 0;
    for (auto p : parts) {
        if (p->fmt != out->fmt || p->n != out->n) {
            *err = "attn_q/attn_k/attn_v must share one format and row length";
            return false;
        }
        out->o += p->o;
    }
    for (auto p : parts) {
        out->qs.insert(out->qs.end(), p->qs.begin(), p->qs.end());
        out->d.insert(out->d.end(), p->d.begin(), p->d.end());
    }
    return true;
}

// [w1 rows 32g..32g+31 | w3 rows 32g..32g+31] for every 32-row group g, so
// one workgroup of the fused kernel sees gate and up of the same outputs.
static bool host_interleave_gate_up(const HostQMat& w1, const HostQMat& w3, HostQMat* out, std::string* err) {
    if (w1.fmt != w3.fmt || w1.n != w3.n || w1.o != w3.o || w1.o % 32) {
        *err = "ffn_gate/ffn_up must share format and shape (rows a multiple of 32)";
        return false;
    }
    out->fmt = w1.fmt; out->n = w1.n; out->nb = w1.nb; out->o = 2 * w1.o;
    const size_t rb = w1.row_bytes();
    out->qs.resize(out->o * rb);
    out->d.resize(out->o * out->nb);
    for (size_t g = 0; g < w1.o / 32; g++) {
        for (int half = 0; half < 2; half++) {
            const HostQMat& src = half ? w3 : w1;
            const size_t dst_row = g * 64 + half * 32;
            memcpy(&out->qs[dst_row * rb], &src.qs[g * 32 * rb], 32 * rb);
            memcpy(&out->d[dst_row * out->nb], &src.d[g * 32 * src.nb], 32 * src.nb * 2);
        }
    }
    return true;
}

static bool upload_qmat(const HostQMat& h, QMat* m, std::string* err) {
    m->fmt = h.fmt; m->o = (int)h.o; m->n = (int)h.n; m->nb = (int)h.nb;
    if (hipMalloc(&m->qs, h.qs.size() + 256) != hipSuccess || hipMalloc(&m->d, h.d.size() * 2 + 256) != hipSuccess) {
        *err = "hipMalloc failed for a weight matrix";
        return false;
    }
    if (hipMemcpy(m->qs, h.qs.data(), h.qs.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->d, h.d.data(), h.d.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
        *err = "hipMemcpy failed for a weight matrix";
        return false;
    }
    return true;
}

static void free_qmat(QMat* m) {
    if (m->qs) hipFree(m->qs);
    if (m->d) hipFree(m->d);
    if (m->sf) hipFree(m->sf);
    m->qs = nullptr; m->d = nullptr; m->sf = nullptr;
}

static float* upload_f32(const float* src, size_t n, std::string* err) {
    float* p = nullptr;
    if (hipMalloc(&p, n * 4 + 256) != hipSuccess || hipMemcpy(p, src, n * 4, hipMemcpyHostToDevice) != hipSuccess) {
        *err = "upload of f32 vector failed";
        return nullptr;
    }
    return p;
}

// The (cos, sin) per pair and position of rope_gguf (util.rs:653-718), with
// the C library's powf/cosf/sinf/logf as Rust's std calls them.
// util::rope (util.rs:589-635): per pair j of a head, freq = theta^(-2j/hd)
// with the llama3 frequency scaling (factor 32, low 1, high 4, the model's
// ctx_len standing for the original context), angle = pos * freq; f32 steps
// and the C library's powf/cosf/sinf as Rust's std calls them.
static void rope_table_hf(float rope_theta, int head_size, uint32_t ctx_len, uint32_t count, float* cos_t, float* sin_t) {
    const float rope_factor = 32.0f, low_freq_factor = 1.0f, high_freq_factor = 4.0f;
    const float old_context_len = (float)ctx_len;
    const float low_freq_wavelen = old_context_len / low_freq_factor;
    const float high_freq_wavelen = old_context_len / high_freq_factor;
    const int half = head_size / 2;
    std::vector<float> freqs(half);
    for (int j = 0; j < half; j++) {
        const int head_dim = j * 2;
        float freq = powf(rope_theta, -(float)head_dim / (float)head_size);
        const float wavelen = (2.0f * 3.14159265358979323846f) / freq;
        if (wavelen > low_freq_wavelen) {
            freq = freq / rope_factor;
        } else if (wavelen <= low_freq_wavelen && wavelen >= high_freq_wavelen) {
            const float smooth = (old_context_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
            freq = (1.0f - smooth) * freq / rope_factor + smooth * freq;
        }
        freqs[j] = freq;
    }
    for (uint32_t pos = 0; pos < count; pos++)
        for (int j = 0; j < half; j++) {
            const float val = (float)pos * freqs[j];
            cos_t[(size_t)pos * half + j] = cosf(val);
            sin_t[(size_t)pos * half + j] = sinf(val);
        }
}

static void rope_table(const yl_rope_params& p, uint32_t pos_begin, uint32_t count, float* cos_t, float* sin_t) {
    const float beta_fast = 32.0f, beta_slow = 1.0f;
    const float two_pi = 2.0f * 3.14159265358979323846f;
    const uint32_t n_pairs = p.head_size / 2;
    const float theta_scale = powf(p.rope_theta, -2.0f / (float)p.head_size);
    const float n_ctx_orig = (float)p.original_ctx_len;
    float corr_start = fmaf(logf(n_ctx_orig / (beta_fast * two_pi)), (float)p.head_size, 0.0f) /
                       (2.0f * logf(p.rope_theta));
    corr_start = fmaxf(floorf(corr_start), 0.0f);   // Rust's f32::max: NaN gives the other operand
    const float corr_end = fmaf(logf(n_ctx_orig / (beta_slow * two_pi)), (float)p.head_size, 0.0f) /
                           (2.0f * logf(p.rope_theta));
    const float corr_dims_1 =
        fminf(corr_start, corr_end) + fminf(corr_end, (float)n_pairs) - fmaxf(corr_start, 0.0f);
    for (uint32_t r = 0; r < count; r++) {
        float theta = (float)(pos_begin + r);
        for (uint32_t k = 0; k < n_pairs; k++) {
            const float theta_interp = p.freq_scale * theta / 1.0f;
            float t = theta_interp;
            if (p.ext_factor != 0.0f) {
                // rope_yarn_ramp(corr_start, corr_dims_1, 2k) (util.rs:720-724)
                const float y = ((float)(k * 2) * 0.5f - corr_start) / fmaxf(corr_dims_1 - corr_start, 0.001f);
                const float ramp_mix = (1.0f - fminf(1.0f, fmaxf(y, 0.0f))) * p.ext_factor;
                t = theta_interp * (1.0f - ramp_mix) + theta / 1.0f * ramp_mix;
            }
            cos_t[(size_t)r * n_pairs + k] = cosf(t) * p.attn_factor;
            sin_t[(size_t)r * n_pairs + k] = sinf(t) * p.attn_factor;
            theta = theta * theta_scale;
        }
    }
}

}  // namespace yl

using namespace yl;

struct yl_weight {
    QMat m;
};

struct Layer {
    QMat qkv, wo, w13, w2;
    QMat w1, w3;                // F16 and f32-scaled Q8 models: gate and up apart (w13 unused)
    QMat wq, wk, wv;            // f32-scaled Q8 models: q, k, v apart (qkv unused)
    float* rms_att = nullptr;
    float* rms_ffn = nullptr;
};

struct yl_model {
    yl_shape shape{};
    int dim = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv = 0, hd = 0, vocab = 0, ctx = 0;
    int kv_ld = 0;   // cache positions: ctx rounded up to a multiple of 4 (key row stride)
    int att = 0, kv = 0;
    float eps = 0.0f, attn_scale = 0.0f;
    yl_rope_params rope{};
    std::vector<Layer> layers;
    float* rms_final = nullptr;
    EmbQ8 emb;
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    bool f16 = false;           // WeightFormat::F16: matmul_f32 on f16 weights (no activation quantization)
    bool q8g = false;           // Q8 with f32 scales and group size gs (lm.rs, safetensors)
    int gs = 32;
    int hf_rope = 0;            // 1: util::rope pairs (j, j + head/2); 0: rope_gguf pairs (2j, 2j + 1)
    int pair_rows = 16;         // q8g: gate/up rows per interleaved block of w13 (16, or 32 with q8_gemv)
    bool q8_gemv = false;       // q8g with group size 32, 64 or 128: one-token steps on the GGUF path's GEMVs
    uint32_t bos = 128000, eos = 128009;
    std::string name = "TransformerLlamaGguf";
    std::vector<std::string> vocab_str;
    std::unique_ptr<yl_tokenizer> tok;   // tokenizer.ggml.* and tokenizer.chat_template
    size_t weight_bytes = 0, emb_bytes = 0;
    int device = 0;
};

struct yl_session {
    const yl_model* m = nullptr;
    hipStream_t stream = nullptr;
    float* kc = nullptr;
    float* vc = nullptr;
    size_t kv_floats = 0;
    StepState* st = nullptr;        // device
    StepState* st_host = nullptr;   // pinned
    int cap_b = 0;
    float *x = nullptr, *sq = nullptr, *logits = nullptr;
    int8_t *aq = nullptr, *hq = nullptr, *nq = nullptr;   // nq/ns: normalized, quantized rows (prompt)
    float *as_ = nullptr, *hs = nullptr, *ns = nullptr;
    // F16 models: normalized rows, raw QKV outputs, attention output, gate/up/h (f32)
    float *xn = nullptr, *qkv_raw = nullptr, *attf = nullptr, *gate = nullptr, *up = nullptr, *hf = nullptr;
    int8_t* gq = nullptr;                // f32-scaled Q8 models: quantized activation row and its scales
    float* gsc = nullptr;
    float* sc = nullptr;                 // attention scores of long contexts [n_heads][ctx]
    float* psc = nullptr;                // prompt attention scratch (batches of 64+ tokens)
    size_t psc_bytes = 0;
    int pseq = 0;                        // seq_len of the prompt call being enqueued
    uint32_t* tokens = nullptr;
    uint32_t* ring = nullptr;
    uint32_t ring_cap = 0;
    // decode-step graphs, one per context bucket: decode attention is sized
    // for the bucket's longest context (see decode_bucket)
    struct DecodeGraph {
        int max_seq;
        hipGraphExec_t exec;
    };
    std::vector<DecodeGraph> graphs;
    int dec_seq = 0;                     // bucket of the decode step being enqueued
    int attn_mode = YL_ATTN_EXACT;       // decode attention: exact order, or split over the context
    float* split = nullptr;              // partials + counts of the split decode attention
    uint64_t prof_seq = 0;               // seq_len of the step yl_profile_kernel times
    uint32_t pos = 0;
};

namespace {

void model_release(yl_model* m) {
    if (!m) return;
    for (auto& L : m->layers) {
        free_qmat(&L.qkv); free_qmat(&L.wo); free_qmat(&L.w13); free_qmat(&L.w2); free_qmat(&L.w1); free_qmat(&L.w3);
        free_qmat(&L.wq); free_qmat(&L.wk); free_qmat(&L.wv);
        if (L.rms_att) hipFree(L.rms_att);
        if (L.rms_ffn) hipFree(L.rms_ffn);
    }
    if (m->rms_final) hipFree(m->rms_final);
    if (m->emb.q) hipFree(m->emb.q);
    if (m->emb.d) hipFree(m->emb.d);
    if (m->emb.d32) hipFree(m->emb.d32);
    if (m->rope_cos) hipFree(m->rope_cos);
    if (m->rope_sin) hipFree(m->rope_sin);
    delete m;
}

// token_embd (Q8_0 or Q4_0 blocks) -> interleaved Q8_0 planes.  A Q4_0 row
// element is the unsigned nibble times the f16 scale (gguf.rs:394-405,474-486),
// which the Q8_0 plane holds exactly as q = nibble.
bool upload_embedding(const GgufTensor* t, int dim, int vocab, EmbQ8* e, std::string* err) {
    if ((uint64_t)dim * vocab > t->n_elements) { *err = "token_embd.weight smaller than vocab*dim"; return false; }
    if (dim % 32) { *err = "embedding length must be a multiple of 32"; return false; }
    const int tiles = (vocab + 63) / 64;
    const int nbE = dim / 32, dimp = (dim + 63) & ~63;
    // padding blocks (dim..dimp) keep scale 0: their values are exact zeros
    std::vector<int8_t> q((size_t)tiles * 64 * dimp, 0);
    std::vector<uint16_t> d((size_t)tiles * 64 * (dimp / 32), 0);
    const size_t blocks = (size_t)vocab * nbE;
    if (t->type == kGgmlF16) {
        // f16 values in the same chunk-major order (16 per chunk, 32 bytes);
        // the padding columns are +0
        if ((uint64_t)vocab * dim * 2 > t->avail) { *err = "token_embd exceeds the file"; return false; }
        std::vector<uint16_t> h((size_t)tiles * 64 * dimp, 0);
        for (int v = 0; v < vocab; v++)
            for (int i = 0; i < dim; i++)
                h[emb_q_off(tiles, v / 64, i >> 4, v % 64) + (i & 15)] =
                    (uint16_t)(t->data[((size_t)v * dim + i) * 2] | (t->data[((size_t)v * dim + i) * 2 + 1] << 8));
        e->vocab = vocab; e->dim = dim; e->tiles = tiles; e->dimp = dimp; e->fmt = 1;
        if (hipMalloc(&e->q, h.size() * 2 + 256) != hipSuccess || hipMalloc(&e->d, 256) != hipSuccess ||
            hipMemcpy(e->q, h.data(), h.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
            *err = "upload of the token embedding failed";
            return false;
        }
        return true;
    }
    if (t->type == kGgmlQ8_0) {
        if (blocks * 34 > t->avail) { *err = "token_embd exceeds the file"; return false; }
    } else if (t->type == kGgmlQ4_0) {
        if (blocks * 18 > t->avail) { *err = "token_embd exceeds the file"; return false; }
    } else {
        *err = "token_embd.weight type " + std::to_string(t->type) + " is not built (Q8_0, Q4_0 and F16 are)";
        return false;
    }
    for (int v = 0; v < vocab; v++) {
        const size_t tile = v / 64, lane = v % 64;
        for (int b = 0; b < nbE; b++) {
            int8_t vals[32];
            uint16_t sc;
            if (t->type == kGgmlQ8_0) {
                const uint8_t* blk = t->data + ((size_t)v * nbE + b) * 34;
                sc = (uint16_t)(blk[0] | (blk[1] << 8));
                memcpy(vals, blk + 2, 32);
            } else {
                const uint8_t* blk = t->data + ((size_t)v * nbE + b) * 18;
                sc = (uint16_t)(blk[0] | (blk[1] << 8));
                for (int j = 0; j < 16; j++) {
                    vals[2 * j] = (int8_t)(blk[2 + j] & 0x0f);
                    vals[2 * j + 1] = (int8_t)((blk[2 + j] >> 4) & 0x0f);
                }
            }
            d[emb_d_idx(tiles, tile, b, (int)lane)] = sc;
            for (int h = 0; h < 2; h++) {
                int8_t* dst = &q[emb_q_off(tiles, tile, 2 * b + h, (int)lane)];
                for (int j = 0; j < 16; j++) dst[j] = (int8_t)((uint8_t)vals[16 * h + j] ^ 0x80u);  // u = q + 128
            }
        }
    }
    e->vocab = vocab; e->dim = dim; e->tiles = tiles; e->dimp = dimp;
    if (hipMalloc(&e->q, q.size() + 256) != hipSuccess || hipMalloc(&e->d, d.size() * 2 + 256) != hipSuccess ||
        hipMemcpy(e->q, q.data(), q.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(e->d, d.data(), d.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
        *err = "upload of the token embedding failed";
        return false;
    }
    return true;
}

yl_model* load_model(const char* path, uint32_t max_ctx_len, int32_t fmt_override, yl_status* st) {
    std::string err;
    *st = YL_ERR_GGUF;
    GgufFile g;
    if (!g.open(path, &err)) {
        set_error(err);
        *st = (err.rfind("cannot", 0) == 0) ? YL_ERR_IO : YL_ERR_GGUF;
        return nullptr;
    }
    const GgufValue* arch = g.get("general.architecture");
    if (!arch || arch->type != 8) { set_error("Missing or wrong type for metadata key: general.architecture"); return nullptr; }
    if (arch->s != "llama") { set_error("Unsupported GGUF architecture: " + arch->s); return nullptr; }
    std::unique_ptr<yl_model, void (*)(yl_model*)> m(new yl_model(), model_release);
    uint64_t u = 0;
    float f = 0.0f;
    auto req_u = [&](const char* k, int* dst) {
        if (!meta_u64(g, k, &u)) { set_error(std::string("Missing or wrong type for metadata key: ") + k); return false; }
        *dst = (int)u;
        return true;
    };
    if (!req_u("llama.embedding_length", &m->dim) || !req_u("llama.feed_forward_length", &m->hidden) ||
        !req_u("llama.block_count", &m->n_layers) || !req_u("llama.attention.head_count", &m->n_heads))
        return nullptr;
    m->n_kv = meta_u64(g, "llama.attention.head_count_kv", &u) ? (int)u : m->n_heads;
    if (!meta_f32(g, "llama.attention.layer_norm_rms_epsilon", &m->eps)) {
        set_error("Missing or wrong type for metadata key: llama.attention.layer_norm_rms_epsilon");
        return nullptr;
    }
    const uint64_t file_type = meta_u64(g, "general.file_type", &u) ? u : 7;
    const float rope_theta = meta_f32(g, "llama.rope.freq_base", &f) ? f : 10000.0f;
    int seq_len = 0;
    if (!req_u("llama.context_length", &seq_len)) return nullptr;
    if (m->n_heads <= 0 || m->dim % m->n_heads) { set_error("dim must be divisible by n_heads"); return nullptr; }
    m->hd = m->dim / m->n_heads;
    m->ctx = (int)((uint32_t)seq_len < max_ctx_len ? (uint32_t)seq_len : max_ctx_len);
    m->kv_ld = (m->ctx + 3) & ~3;
    const GgufValue* toks = g.get("tokenizer.ggml.tokens");
    if (!toks) { set_error("tokenizer.ggml.tokens metadata key not found"); return nullptr; }
    if (toks->type != 9) { set_error("tokenizer.ggml.tokens must be an array of strings"); return nullptr; }
    m->vocab = (int)toks->arr_len;
    m->vocab_str = toks->arr_str;
    const float raw = meta_f32(g, "llama.rope.scaling.factor", &f) ? f : 1.0f;
    m->rope.freq_scale = raw != 0.0f ? 1.0f / raw : 1.0f;
    m->rope.ext_factor = meta_f32(g, "llama.rope.scaling.ext_factor", &f) ? f : 0.0f;
    m->rope.attn_factor = meta_f32(g, "llama.rope.scaling.attn_factor", &f) ? f : 1.0f;
    m->rope.original_ctx_len = meta_u64(g, "llama.rope.scaling.original_context_length", &u) ? (uint32_t)u : (uint32_t)seq_len;
    const float att_scale_meta = meta_f32(g, "llama.attention.scale", &f) ? f : 0.0f;
    m->rope.rope_theta = rope_theta;
    m->rope.head_size = (uint32_t)m->hd;
    m->rope.n_heads = (uint32_t)m->n_heads;
    m->rope.n_kv_heads = (uint32_t)m->n_kv;
    int wfmt;
    if (fmt_override >= 0) {
        if (fmt_override > 2) { set_error("invalid format override"); *st = YL_ERR_ARG; return nullptr; }
        wfmt = fmt_override;
    } else if (file_type == 1) wfmt = YL_F16;
    else if (file_type == 2) wfmt = YL_Q4_0;
    else if (file_type == 7) wfmt = YL_Q8_0;
    else { set_error("Unsupported GGUF file_type: " + std::to_string(file_type) + " -- supported: F16=1, Q4_0=2, Q8_0=7"); return nullptr; }
    {
        std::string terr;
        m->tok.reset(tokenizer_from_gguf(g, &terr));
        if (!m->tok) { set_error(terr); return nullptr; }
        m->bos = m->tok->t.bos();
        m->eos = m->tok->t.eos();
    }

    m->att = m->n_heads * m->hd;
    m->kv = m->n_kv * m->hd;
    m->attn_scale = att_scale_meta != 0.0f ? att_scale_meta : 1.0f / sqrtf((float)m->hd);
    if (m->n_kv <= 0 || m->n_heads % m->n_kv) { set_error("n_heads must be a multiple of n_kv_heads"); return nullptr; }
    if (m->dim % 32 || m->hidden % 32 || m->kv % 32 || (m->hd != 32 && m->hd != 64 && m->hd != 128) ||
        m->dim > 4096 || m->ctx <= 0) {
        // dim <= 4096: one wavefront normalizes the residual row inside the
        // QKV and gate/up matmuls
        set_error("unsupported shape: dim, hidden and kv_dim must be multiples of 32, head_size 32/64/128, "
                  "dim <= 4096");
        *st = YL_ERR_UNSUPPORTED;
        return nullptr;
    }
    // kernels address one layer's value cache (kv_ld x kv_dim floats) with
    // 32-bit byte offsets
    if ((uint64_t)m->kv_ld * (uint64_t)m->kv * 4 >= (1ull << 31)) {
        set_error("context_length " + std::to_string(m->ctx) + " too long: one layer's KV cache must stay below "
                  "2 GiB (cap it with max_ctx_len)");
        *st = YL_ERR_UNSUPPORTED;
        return nullptr;
    }
    hipGetDevice(&m->device);

    const GgufTensor* te = g.tensor("token_embd.weight");
    if (!te) { set_error("token_embd.weight not found"); return nullptr; }
    if (!upload_embedding(te, m->dim, m->vocab, &m->emb, &err)) { set_error(err); *st = YL_ERR_UNSUPPORTED; return nullptr; }
    m->emb_bytes = m->emb.fmt == 1 ? (size_t)m->vocab * m->dim * 2
                                   : (size_t)m->vocab * m->dim + (size_t)m->vocab * (m->dim / 32) * 2;

    auto load_f32 = [&](const std::string& nm, size_t n, float** dst) {
        const GgufTensor* t = g.tensor(nm);
        if (!t) { set_error("Missing tensor: " + nm); return false; }
        if (t->type != kGgmlF32) { set_error("Expected F32 tensor: " + nm); return false; }
        if (t->n_elements < n || t->avail < n * 4) { set_error("tensor too small: " + nm); return false; }
        std::vector<float> v(n);
        memcpy(v.data(), t->data, n * 4);
        *dst = upload_f32(v.data(), n, &err);
        if (!*dst) { set_error(err); return false; }
        return true;
    };
    if (!load_f32("output_norm.weight", m->dim, &m->rms_final)) return nullptr;
    m->layers.resize(m->n_layers);
    for (int l = 0; l < m->n_layers; l++) {
        Layer& L = m->layers[l];
        const std::string p = "blk." + std::to_string(l) + ".";
        if (!load_f32(p + "attn_norm.weight", m->dim, &L.rms_att) || !load_f32(p + "ffn_norm.weight", m->dim, &L.rms_ffn))
            return nullptr;
        const char* names[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_down", "ffn_up"};
        const size_t rows[7] = {(size_t)m->att, (size_t)m->kv, (size_t)m->kv, (size_t)m->dim,
                                (size_t)m->hidden, (size_t)m->dim, (size_t)m->hidden};
        const size_t cols[7] = {(size_t)m->dim, (size_t)m->dim, (size_t)m->dim, (size_t)m->att,
                                (size_t)m->dim, (size_t)m->hidden, (size_t)m->dim};
        HostQMat h[7];
        for (int k = 0; k < 7; k++) {
            const GgufTensor* t = g.tensor(p + names[k] + ".weight");
            if (!t) { set_error("Missing tensor: " + p + names[k] + ".weight"); return nullptr; }
            if (t->n_elements != rows[k] * cols[k]) { set_error("unexpected element count for " + t->name); return nullptr; }
            if (!host_from_gguf(t->type, t->data, t->avail, rows[k], cols[k], &h[k], &err)) {
                set_error(t->name + ": " + err);
                *st = YL_ERR_UNSUPPORTED;
                return nullptr;
            }
        }
        int n_f16 = 0;
        for (int k = 0; k < 7; k++) n_f16 += h[k].fmt == kF16;
        if (n_f16 != 0 && n_f16 != 7) {
            set_error(p + "*: F16 projections beside quantized ones are not built (the F16 path needs all seven)");
            *st = YL_ERR_UNSUPPORTED;
            return nullptr;
        }
        if (l == 0) m->f16 = n_f16 == 7;
        else if (m->f16 != (n_f16 == 7)) { set_error("layers mix F16 and quantized weights"); *st = YL_ERR_UNSUPPORTED; return nullptr; }
        HostQMat qkv, w13;
        bool ok = host_concat_rows({&h[0], &h[1], &h[2]}, &qkv, &err) && upload_qmat(qkv, &L.qkv, &err) &&
                  upload_qmat(h[3], &L.wo, &err) && upload_qmat(h[5], &L.w2, &err);
        if (ok && m->f16) {
            f16_pair_rows(reinterpret_cast<const uint16_t*>(h[4].qs.data()),
                          reinterpret_cast<const uint16_t*>(h[6].qs.data()), h[4].o, h[4].n, &w13);
            ok = upload_qmat(w13, &L.w13, &err);
        } else if (ok) {
            ok = host_interleave_gate_up(h[4], h[6], &w13, &err) && upload_qmat(w13, &L.w13, &err);
        }
        if (!ok) {
            set_error(p + err);
            return nullptr;
        }
        m->weight_bytes += L.qkv.bytes() + L.wo.bytes() + L.w13.bytes() + L.w2.bytes() + L.w1.bytes() + L.w3.bytes();
    }
    // RoPE angle table for every position of the context
    {
        const size_t half = m->hd / 2;
        std::vector<float> c((size_t)m->ctx * half), s((size_t)m->ctx * half);
        rope_table(m->rope, 0, (uint32_t)m->ctx, c.data(), s.data());
        m->rope_cos = upload_f32(c.data(), c.size(), &err);
        m->rope_sin = upload_f32(s.data(), s.size(), &err);
        if (!m->rope_cos || !m->rope_sin) { set_error(err); return nullptr; }
    }
    yl_shape& S = m->shape;
    S.dimension = m->dim; S.hidden_dimension = m->hidden; S.n_heads = m->n_heads; S.head_size = m->hd;
    S.n_kv_heads = m->n_kv; S.vocab_size = m->vocab; S.n_layers = m->n_layers; S.ctx_len = m->ctx;
    S.rms_norm_eps = m->eps; S.rope_theta = rope_theta; S.group_size = 32;
    S.rope_freq_scale = m->rope.freq_scale; S.rope_ext_factor = m->rope.ext_factor;
    S.rope_attn_factor = m->rope.attn_factor; S.rope_original_ctx_len = m->rope.original_ctx_len;
    S.attention_scale = att_scale_meta; S.weight_format = wfmt;
    *st = YL_OK;
    return m.release();
}

// A safetensors or lm.rs model (HostModel) onto the device.
static bool upload_embedding_table(const HostModel& h, EmbQ8* e, std::string* err) {
    const int dim = h.dim, vocab = h.vocab;
    const int tiles = (vocab + 63) / 64, dimp = (dim + 63) & ~63;
    e->vocab = vocab; e->dim = dim; e->tiles = tiles; e->dimp = dimp;
    if (h.emb_f16.empty()) {
        // int8 values chunk-major as the Q8_0 table's bytes, f32 group scales
        // [group][tile][lane]; the padding columns hold value 0, scale 0
        const HostMat& q = h.emb_q8;
        const int gs = q.gs, ngs = (dimp + gs - 1) / gs, G = dim / gs;
        std::vector<int8_t> vb((size_t)tiles * 64 * dimp, 0);
        std::vector<float> sb((size_t)ngs * tiles * 64, 0.0f);
        for (int v = 0; v < vocab; v++) {
            for (int i = 0; i < dim; i++) vb[emb_q_off(tiles, v / 64, i >> 4, v % 64) + (i & 15)] = q.q[(size_t)v * dim + i];
            for (int g = 0; g < G; g++) sb[((size_t)g * tiles + v / 64) * 64 + v % 64] = q.s[(size_t)v * G + g];
        }
        e->fmt = 3;
        e->gs = gs;
        if (hipMalloc(&e->q, vb.size() + 256) != hipSuccess || hipMalloc(&e->d32, sb.size() * 4 + 256) != hipSuccess ||
            hipMalloc(&e->d, 256) != hipSuccess || hipMemcpy(e->q, vb.data(), vb.size(), hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(e->d32, sb.data(), sb.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            *err = "upload of the token embedding failed";
            return false;
        }
        return true;
    }
    std::vector<uint16_t> buf((size_t)tiles * 64 * dimp, 0);
    for (int v = 0; v < vocab; v++)
        for (int i = 0; i < dim; i++) buf[emb_q_off(tiles, v / 64, i >> 4, v % 64) + (i & 15)] = h.emb_f16[(size_t)v * dim + i];
    e->fmt = 1;
    if (hipMalloc(&e->q, buf.size() * 2 + 256) != hipSuccess || hipMalloc(&e->d, 256) != hipSuccess ||
        hipMemcpy(e->q, buf.data(), buf.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
        *err = "upload of the token embedding failed";
        return false;
    }
    return true;
}

static bool upload_hostmat(const HostMat& h, QMat* m, std::string* err) {
    m->o = (int)h.o; m->n = (int)h.n;
    if (h.f16) {
        m->fmt = kF16; m->nb = 0;
        if (hipMalloc(&m->qs, h.h.size() * 2 + 256) != hipSuccess ||
            hipMemcpy(m->qs, h.h.data(), h.h.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
            *err = "weight upload failed";
            return false;
        }
        return true;
    }
    m->fmt = kQ8; m->nb = (int)(h.n / 32); m->gs = h.gs;   // nb: 32-blocks (scales: n / gs per row)
    if (hipMalloc(&m->qs, h.q.size() + 256) != hipSuccess || hipMalloc(&m->sf, h.s.size() * 4 + 256) != hipSuccess ||
        hipMemcpy(m->qs, h.q.data(), h.q.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->sf, h.s.data(), h.s.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        *err = "weight upload failed";
        return false;
    }
    return true;
}

yl_model* model_from_host(HostModel& h, yl_status* st) {
    *st = YL_ERR_UNSUPPORTED;
    std::unique_ptr<yl_model, void (*)(yl_model*)> m(new yl_model(), model_release);
    m->name = h.name;
    m->dim = h.dim; m->hidden = h.hidden; m->n_layers = h.n_layers; m->n_heads = h.n_heads; m->n_kv = h.n_kv;
    m->hd = h.hd; m->vocab = h.vocab; m->ctx = h.ctx; m->eps = h.eps;
    m->kv_ld = (m->ctx + 3) & ~3;
    m->att = m->n_heads * m->hd;
    m->kv = m->n_kv * m->hd;
    m->attn_scale = 1.0f / sqrtf((float)m->hd);
    m->hf_rope = 1;
    m->f16 = h.f16;
    m->q8g = !h.f16;
    m->gs = h.gs;
    // group size 32, 64 or 128 (rows up to the GEMV's limits): one-token
    // steps run the 32-block GEMV (kQ8S / kQ8S64 / kQ8S128), whose SwiGLU
    // tiles are 32 gate + 32 up rows
    m->q8_gemv = m->q8g && m->dim <= 4096 &&
                 ((m->gs == 32 && m->att <= 16384 && m->hidden <= 16384) ||
                  ((m->gs == 64 || m->gs == 128) && m->att <= 8192 && m->hidden <= 8192));
    m->pair_rows = m->q8_gemv ? 32 : 16;
    if (m->n_kv <= 0 || m->n_heads % m->n_kv || (m->hd != 32 && m->hd != 64 && m->hd != 128) || m->dim % 32 ||
        m->hidden % 32 || m->att % 32 || m->kv % 32 || m->ctx <= 0 || m->dim > 8192 ||
        (m->q8g && (m->dim % m->gs || m->att % m->gs || m->hidden % m->gs || m->hidden % m->pair_rows))) {
        set_error("unsupported shape: head_size 32/64/128, dimensions multiples of 32 (and of the group size)");
        return nullptr;
    }
    if ((uint64_t)m->kv_ld * (uint64_t)m->kv * 4 >= (1ull << 31)) {
        set_error("context_length " + std::to_string(m->ctx) + " too long: cap it with max_ctx_len");
        return nullptr;
    }
    hipGetDevice(&m->device);
    std::string err;
    if (!upload_embedding_table(h, &m->emb, &err)) { set_error(err); return nullptr; }
    m->emb_bytes = m->emb.fmt == 1 ? (size_t)m->vocab * m->dim * 2
                                    : (size_t)m->vocab * m->dim + (size_t)m->vocab * (m->dim / m->emb.gs) * 4;
    m->rms_final = upload_f32(h.rms_final.data(), m->dim, &err);
    if (!m->rms_final) { set_error(err); return nullptr; }
    m->layers.resize(m->n_layers);
    for (int l = 0; l < m->n_layers; l++) {
        Layer& L = m->layers[l];
        const auto& H = h.layers[l];
        L.rms_att = upload_f32(h.rms_att[l].data(), m->dim, &err);
        L.rms_ffn = upload_f32(h.rms_ffn[l].data(), m->dim, &err);
        if (!L.rms_att || !L.rms_ffn) { set_error(err); return nullptr; }
        bool ok;
        if (m->f16) {
            // q, k and v rows in one matrix, q and k in util::rope's pair
            // order as below (the QKV GEMV rotates adjacent rows)
            HostQMat qkv;
            qkv.fmt = kF16; qkv.n = H[0].n; qkv.o = H[0].o + H[1].o + H[2].o;
            for (int k = 0; k < 3; k++)
                for (size_t p = 0; p < H[k].o; p++) {
                    const size_t r = k < 2 ? (size_t)qk_column((int)p, m->hd, 1) : p;
                    const uint8_t* src = (const uint8_t*)(H[k].h.data() + r * H[k].n);
                    qkv.qs.insert(qkv.qs.end(), src, src + H[k].n * 2);
                }
            HostQMat w13;
            f16_pair_rows(H[4].h.data(), H[6].h.data(), H[4].o, H[4].n, &w13);
            ok = upload_qmat(qkv, &L.qkv, &err) && upload_hostmat(H[3], &L.wo, &err) && upload_qmat(w13, &L.w13, &err) &&
                 upload_hostmat(H[5], &L.w2, &err);
        } else {
            // q, k and v rows in one matrix, the q and k rows of each head in
            // util::rope's pair order (stored row p holds qk_column(p), so a
            // rotated pair is two adjacent rows); gate and up rows interleaved
            // in blocks of m->pair_rows (the SwiGLU tiles of the GEMVs)
            HostMat qkv, w13;
            qkv.o = H[0].o + H[1].o + H[2].o; qkv.n = H[0].n; qkv.gs = H[0].gs;
            for (int k = 0; k < 3; k++) {
                const size_t G = H[k].n / H[k].gs;
                for (size_t p = 0; p < H[k].o; p++) {
                    const size_t r = k < 2 ? (size_t)qk_column((int)p, m->hd, 1) : p;
                    qkv.q.insert(qkv.q.end(), H[k].q.begin() + r * H[k].n, H[k].q.begin() + (r + 1) * H[k].n);
                    qkv.s.insert(qkv.s.end(), H[k].s.begin() + r * G, H[k].s.begin() + (r + 1) * G);
                }
            }
            w13.o = 2 * H[4].o; w13.n = H[4].n; w13.gs = H[4].gs;
            const size_t G = H[4].n / H[4].gs, P = (size_t)m->pair_rows;
            for (size_t r0 = 0; r0 < H[4].o; r0 += P)
                for (int k : {4, 6}) {
                    w13.q.insert(w13.q.end(), H[k].q.begin() + r0 * H[k].n, H[k].q.begin() + (r0 + P) * H[k].n);
                    w13.s.insert(w13.s.end(), H[k].s.begin() + r0 * G, H[k].s.begin() + (r0 + P) * G);
                }
            ok = upload_hostmat(qkv, &L.qkv, &err) && upload_hostmat(H[3], &L.wo, &err) &&
                 upload_hostmat(w13, &L.w13, &err) && upload_hostmat(H[5], &L.w2, &err);
        }
        if (!ok) { set_error(err); return nullptr; }
        m->weight_bytes += L.qkv.bytes() + L.wo.bytes() + L.w13.bytes() + L.w1.bytes() + L.w2.bytes() + L.w3.bytes();
    }
    {
        const size_t half = m->hd / 2;
        std::vector<float> c((size_t)m->ctx * half), sn((size_t)m->ctx * half);
        rope_table_hf(h.rope_theta, m->hd, (uint32_t)m->ctx, (uint32_t)m->ctx, c.data(), sn.data());
        m->rope_cos = upload_f32(c.data(), c.size(), &err);
        m->rope_sin = upload_f32(sn.data(), sn.size(), &err);
        if (!m->rope_cos || !m->rope_sin) { set_error(err); return nullptr; }
    }
    m->tok.reset(h.tok);
    h.tok = nullptr;
    m->bos = m->tok->t.bos();
    m->eos = m->tok->t.eos();
    m->vocab_str.clear();
    yl_shape& S = m->shape;
    S.dimension = m->dim; S.hidden_dimension = m->hidden; S.n_heads = m->n_heads; S.head_size = m->hd;
    S.n_kv_heads = m->n_kv; S.vocab_size = m->vocab; S.n_layers = m->n_layers; S.ctx_len = m->ctx;
    S.rms_norm_eps = m->eps; S.rope_theta = h.rope_theta; S.group_size = m->gs;
    S.rope_freq_scale = 1.0f; S.rope_ext_factor = 0.0f; S.rope_attn_factor = 1.0f;
    S.rope_original_ctx_len = (uint32_t)m->ctx; S.attention_scale = 0.0f; S.weight_format = m->f16 ? YL_F16 : YL_Q8_0;
    *st = YL_OK;
    return m.release();
}

// The prompt attention scratch for `batch` tokens from `start_pos` (kept at
// the largest size used; prompts below 64 tokens need none).
bool prompt_scratch(yl_session* s, int batch, uint32_t start_pos) {
    s->pseq = (int)start_pos + batch;
    if (!prompt_attn_applies(batch, s->pseq, s->m->hd)) return true;
    const size_t need = prompt_attn_bytes(s->m->n_heads, s->pseq, batch);
    if (need <= s->psc_bytes) return true;
    hipStreamSynchronize(s->stream);
    if (s->psc) hipFree(s->psc);
    s->psc = nullptr;
    s->psc_bytes = 0;
    if (hipMalloc(&s->psc, need + 256) != hipSuccess) {
        s->psc = nullptr;
        set_error("hipMalloc failed for the prompt attention scratch");
        return false;
    }
    s->psc_bytes = need;
    return true;
}

bool session_grow(yl_session* s, int batch) {
    if (batch <= s->cap_b) return true;
    const yl_model* m = s->m;
    // the decode graphs hold the old buffer addresses: drop them, they are
    // captured again on the next decode steps
    hipStreamSynchronize(s->stream);
    for (auto& g : s->graphs) hipGraphExecDestroy(g.exec);
    s->graphs.clear();
    auto rel = [](auto*& p) { if (p) hipFree(p); p = nullptr; };
    rel(s->x); rel(s->sq); rel(s->aq); rel(s->hq); rel(s->as_); rel(s->hs); rel(s->tokens); rel(s->nq); rel(s->ns);
    rel(s->xn); rel(s->qkv_raw); rel(s->attf); rel(s->gate); rel(s->up); rel(s->hf); rel(s->gq); rel(s->gsc);
    const size_t B = (size_t)batch;
    if (m->q8g) {
        const size_t mx = std::max({(size_t)m->dim, (size_t)m->att, (size_t)m->hidden});
        if (hipMalloc(&s->gq, B * mx + 256) != hipSuccess || hipMalloc(&s->gsc, B * mx / m->gs * 4 + 256) != hipSuccess) {
            set_error("hipMalloc failed for session buffers");
            s->cap_b = 0;
            return false;
        }
    }
    if (m->f16 || m->q8g) {
        const bool okf = hipMalloc(&s->xn, B * m->dim * 4 + 256) == hipSuccess &&
                         hipMalloc(&s->qkv_raw, B * (m->att + 2 * m->kv) * 4 + 256) == hipSuccess &&
                         hipMalloc(&s->attf, B * m->att * 4 + 256) == hipSuccess &&
                         hipMalloc(&s->gate, B * 2 * m->hidden * 4 + 256) == hipSuccess &&
                         hipMalloc(&s->up, B * m->hidden * 4 + 256) == hipSuccess &&
                         hipMalloc(&s->hf, B * m->hidden * 4 + 256) == hipSuccess;
        if (!okf) { set_error("hipMalloc failed for session buffers"); s->cap_b = 0; return false; }
    }
    bool ok = hipMalloc(&s->x, B * m->dim * 4 + 256) == hipSuccess &&
              hipMalloc(&s->sq, B * m->att * 4 + 256) == hipSuccess &&
              hipMalloc(&s->aq, B * m->att + 256) == hipSuccess &&
              hipMalloc(&s->hq, B * m->hidden + 256) == hipSuccess &&
              hipMalloc(&s->as_, B * m->att / 8 + 256) == hipSuccess &&
              hipMalloc(&s->hs, B * m->hidden / 8 + 256) == hipSuccess &&
              hipMalloc(&s->tokens, B * 4 + 256) == hipSuccess &&
              hipMalloc(&s->nq, B * m->dim + 256) == hipSuccess &&
              hipMalloc(&s->ns, B * m->dim / 8 + 256) == hipSuccess;
    if (!ok) { set_error("hipMalloc failed for session buffers"); s->cap_b = 0; return false; }
    s->cap_b = batch;
    return true;
}

// The GEMV weight format of a matrix: its own, or kQ8S / kQ8S64 / kQ8S128
// for Q8 rows with f32 scales (which reach the GEMV with group size 32, 64
// or 128 only: yl_model::q8_gemv).
static int gemv_fmt(const QMat& w) {
    if (!w.sf) return w.fmt;
    return w.gs == 128 ? kQ8S128 : (w.gs == 64 ? kQ8S64 : kQ8S);
}

uint64_t gemv_bytes(const QMat& w, int out_elems, int batch) {
    return (uint64_t)w.bytes() + (uint64_t)batch * ((uint64_t)w.n + (uint64_t)w.nb * 4 + (uint64_t)out_elems * 4);
}

// Kernel classes of a forward pass, in step order (also the profiling
// classes of yl_profile_kernel).
enum OpClass : int { kOpQkv = 0, kOpAttn = 1, kOpWo = 2, kOpW13 = 3, kOpW2 = 4, kOpLogits = 5 };

// Prompt batches from this many tokens run the projections on the int8
// MFMA GEMM (activations normalized and quantized once per row first).
constexpr int kGemmMinTokens = 16;

// The projections of op `cls` of layer l over `batch` tokens on the GEMM
// (prologue: the row normalization the QKV and gate/up GEMMs read first);
// hipErrorNotSupported when a shape needs the GEMV instead.
hipError_t enqueue_op_gemm(const yl_model* m, yl_session* s, int cls, int l, int batch, const uint32_t* tok,
                           float* kc, float* vc, uint64_t* bytes, bool prologue) {
    hipStream_t st = s->stream;
    const Layer& L = m->layers[l];
    GemvArgs a{};
    const QMat* w = nullptr;
    int epi = 0;
    switch (cls) {
    case kOpQkv:
        w = &L.qkv; epi = kEpiQkvRope;
        a.xq = s->nq; a.xs = s->ns;
        a.q_out = s->sq; a.k_cache = kc; a.v_cache = vc;
        a.att_dim = m->att; a.kv_dim = m->kv; a.head_size = m->hd; a.kv_ld = m->kv_ld;
        a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin; a.state = s->st;
        break;
    case kOpWo:
        w = &L.wo; epi = kEpiResid;
        a.xq = s->aq; a.xs = s->as_; a.x = s->x;
        break;
    case kOpW13:
        w = &L.w13; epi = kEpiSwiglu;
        a.xq = s->nq; a.xs = s->ns;
        a.hq = s->hq; a.hs = s->hs; a.h_f32 = nullptr; a.hidden = m->hidden; a.h_fmt = L.w2.fmt;
        break;
    case kOpW2:
        w = &L.w2; epi = kEpiResid;
        a.xq = s->hq; a.xs = s->hs; a.x = s->x;
        break;
    default:
        return hipErrorNotSupported;
    }
    a.qs = w->qs; a.d = w->d; a.n = w->n; a.o = w->o; a.nb = w->nb;
    if (!gemm_supported(a, w->fmt, epi, batch)) return hipErrorNotSupported;
    hipError_t e = hipSuccess;
    if (prologue && (cls == kOpQkv || cls == kOpW13)) {
        // RMSNorm (+ the layer-0 embedding lookup) and quantization of every row
        if (cls == kOpQkv && l == 0) e = launch_embed(m->emb, tok, batch, s->x, st);
        if (e == hipSuccess)
            e = launch_rmsnorm(w->fmt, s->x, cls == kOpQkv ? L.rms_att : L.rms_ffn, m->dim, m->eps, batch, nullptr,
                               s->nq, s->ns, st);
        if (e != hipSuccess) return e;
    }
    if (bytes) *bytes = gemv_bytes(*w, w->o, batch);
    return launch_gemm(a, w->fmt, epi, batch, st);
}

// Enqueues op `cls` of layer l for `batch` tokens whose ids are at `tok`
// (device) and whose first position is st->pos (device), on s->stream.
// `bytes` (nullable) receives the algorithmic bytes the launch reads and
// writes.
static hipError_t enqueue_attn_f32(const yl_model* m, yl_session* s, int batch, float* kc, float* vc);

hipError_t enqueue_op(const yl_model* m, yl_session* s, int cls, int l, int batch, const uint32_t* tok, int advance,
                      uint64_t* bytes, bool prologue = true) {
    hipStream_t st = s->stream;
    const size_t lay_kv = (size_t)m->kv_ld * m->kv;
    if (cls == kOpLogits) {
        // final RMSNorm + logits of the last token + argmax + step bookkeeping
        if (bytes) *bytes = (uint64_t)m->emb_bytes + (uint64_t)m->dim * 8 + (uint64_t)m->vocab * 4;
        return launch_logits(m->emb, s->x + (size_t)(batch - 1) * m->dim, m->rms_final, m->eps, s->logits,
                             s->st, s->ring, s->ring_cap, advance, st);
    }
    const Layer& L = m->layers[l];
    float* kc = s->kc + (size_t)l * lay_kv;
    float* vc = s->vc + (size_t)l * lay_kv;
    // f32-scaled Q8 with 64- or 128-groups: attention and SwiGLU hand over
    // f32 rows, which the Wo and down GEMVs quantize (such a group spans
    // several of the producers' 32-wide workgroups)
    const bool f32_act = m->q8g && m->gs > 32;
    if (batch >= kGemmMinTokens && cls != kOpAttn) {
        hipError_t e = enqueue_op_gemm(m, s, cls, l, batch, tok, kc, vc, bytes, prologue);
        if (e != hipErrorNotSupported) return e;
    }
    GemvArgs a{};
    switch (cls) {
    case kOpQkv:
        // RMSNorm + quantize (prologue) -> Q,K,V -> K/V += into the cache -> RoPE
        a.qs = L.qkv.qs; a.d = L.qkv.d; a.sf = L.qkv.sf; a.n = L.qkv.n; a.o = L.qkv.o; a.nb = L.qkv.nb;
        a.x = s->x; a.norm_w = L.rms_att; a.eps = m->eps;
        a.hf_rows = m->hf_rope;
        if (l == 0 && m->emb.fmt == 0) { a.emb = m->emb; a.tokens = tok; }
        if (l == 0 && m->emb.fmt != 0) {   // an f16 table: the lookup runs first
            const hipError_t e = launch_embed(m->emb, tok, batch, s->x, st);
            if (e != hipSuccess) return e;
        }
        a.q_out = s->sq; a.k_cache = kc; a.v_cache = vc;
        a.att_dim = m->att; a.kv_dim = m->kv; a.head_size = m->hd; a.kv_ld = m->kv_ld;
        a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin; a.state = s->st;
        if (bytes) *bytes = gemv_bytes(L.qkv, L.qkv.o, batch);
        return launch_gemv(a, gemv_fmt(L.qkv), kEpiQkvRope, batch, st);
    case kOpAttn:
        // attention (+ quantize of its output).  Algorithmic bytes: the keys
        // and values of every position, the queries, the quantized output.
        if (bytes)
            *bytes = 2ull * s->prof_seq * (uint64_t)m->kv * 4 +
                     (uint64_t)batch * ((uint64_t)m->att * 4 + (uint64_t)m->att + (uint64_t)m->att / 8);
        if (f32_act && batch == 1)   // f32 output: the Wo GEMV quantizes it in 64-groups
            return enqueue_attn_f32(m, s, batch, kc, vc);
        if (batch == 1 && s->attn_mode == YL_ATTN_SPLIT)
            return launch_attn_split(s->sq, kc, vc, s->st, m->kv_ld, m->n_heads, m->n_kv, m->hd, m->attn_scale,
                                     L.wo.fmt, s->aq, s->as_, nullptr, s->split, st);
        if (batch == 1)
            return launch_attn_decode(s->sq, kc, vc, s->st, s->dec_seq, m->kv_ld, m->n_heads, m->n_kv, m->hd,
                                      m->attn_scale, L.wo.fmt, s->aq, s->as_, nullptr, s->sc, st);
        if (prompt_attn_applies(batch, s->pseq, m->hd))
            return launch_prompt_attention(s->sq, kc, vc, s->st, batch, s->pseq, m->kv_ld, m->n_heads, m->n_kv, m->hd,
                                           m->attn_scale, L.wo.fmt, s->aq, s->as_, nullptr, s->psc, st);
        return launch_attention(s->sq, kc, vc, s->st, batch, s->pseq, m->kv_ld, m->n_heads, m->n_kv, m->hd,
                                m->attn_scale, L.wo.fmt, s->aq, s->as_, nullptr, st);
    case kOpWo:
        // WO -> residual add
        a.qs = L.wo.qs; a.d = L.wo.d; a.sf = L.wo.sf; a.n = L.wo.n; a.o = L.wo.o; a.nb = L.wo.nb;
        a.xq = s->aq; a.xs = s->as_; a.x = s->x;
        if (bytes) *bytes = gemv_bytes(L.wo, L.wo.o, batch);
        if (f32_act) {
            a.xf = s->attf;
            return launch_gemv(a, gemv_fmt(L.wo), kEpiResidQ, batch, st);
        }
        return launch_gemv(a, gemv_fmt(L.wo), kEpiResid, batch, st);
    case kOpW13:
        // RMSNorm + quantize (prologue) -> W1, W3 -> SwiGLU -> quantize
        a.qs = L.w13.qs; a.d = L.w13.d; a.sf = L.w13.sf; a.n = L.w13.n; a.o = L.w13.o; a.nb = L.w13.nb;
        a.x = s->x; a.norm_w = L.rms_ffn; a.eps = m->eps;
        a.hq = s->hq; a.hs = s->hs; a.h_f32 = nullptr; a.hidden = m->hidden; a.h_fmt = L.w2.fmt;
        if (f32_act) {   // f32 h: the down GEMV quantizes it in 64-groups
            a.hq = nullptr; a.hs = nullptr; a.h_f32 = s->hf;
        }
        if (bytes) *bytes = gemv_bytes(L.w13, m->hidden / 4 + m->hidden / 32, batch);
        return launch_gemv(a, gemv_fmt(L.w13), kEpiSwiglu, batch, st);
    case kOpW2:
        // W2 -> residual add
        a.qs = L.w2.qs; a.d = L.w2.d; a.sf = L.w2.sf; a.n = L.w2.n; a.o = L.w2.o; a.nb = L.w2.nb;
        a.xq = s->hq; a.xs = s->hs; a.x = s->x;
        if (bytes) *bytes = gemv_bytes(L.w2, L.w2.o, batch);
        if (f32_act) {
            a.xf = s->hf;
            return launch_gemv(a, gemv_fmt(L.w2), kEpiResidQ, batch, st);
        }
        return launch_gemv(a, gemv_fmt(L.w2), kEpiResid, batch, st);
    default:
        return hipErrorInvalidValue;
    }
}

// Attention of layer l into s->attf (f32), for the F16 and f32-scaled Q8
// models (the same kernels as the GGUF path, with an f32 output).
static hipError_t enqueue_attn_f32(const yl_model* m, yl_session* s, int batch, float* kc, float* vc) {
    hipStream_t st = s->stream;
    if (batch == 1 && s->attn_mode == YL_ATTN_SPLIT)
        return launch_attn_split(s->sq, kc, vc, s->st, m->kv_ld, m->n_heads, m->n_kv, m->hd, m->attn_scale, -1,
                                 nullptr, nullptr, s->attf, s->split, st);
    if (batch == 1)
        return launch_attn_decode(s->sq, kc, vc, s->st, s->dec_seq, m->kv_ld, m->n_heads, m->n_kv, m->hd,
                                  m->attn_scale, -1, nullptr, nullptr, s->attf, s->sc, st);
    if (prompt_attn_applies(batch, s->pseq, m->hd))
        return launch_prompt_attention(s->sq, kc, vc, s->st, batch, s->pseq, m->kv_ld, m->n_heads, m->n_kv, m->hd,
                                       m->attn_scale, -1, nullptr, nullptr, s->attf, s->psc, st);
    return launch_attention(s->sq, kc, vc, s->st, batch, s->pseq, m->kv_ld, m->n_heads, m->n_kv, m->hd,
                            m->attn_scale, -1, nullptr, nullptr, s->attf, st);
}

static uint64_t attn_bytes(const yl_model* m, const yl_session* s, int batch) {
    return 2ull * s->prof_seq * (uint64_t)m->kv * 4 + (uint64_t)batch * (uint64_t)m->att * 8;
}

// One op class of layer l of an F16 model's forward pass (forward.rs:120-297
// with F16Kernel: activations stay f32, every matmul is matmul_f32 and
// assigns its columns, so K and V overwrite their cache entries).  `bytes`
// (nullable): the algorithmic bytes of the class -- f16 weights, f32
// activations read, f32 outputs written.
hipError_t enqueue_op_f16(const yl_model* m, yl_session* s, int cls, int l, int batch, const uint32_t* tok,
                          int advance, uint64_t* bytes) {
    hipStream_t st = s->stream;
    const uint64_t B = (uint64_t)batch;
    if (cls == kOpLogits) {
        if (bytes) *bytes = (uint64_t)m->emb_bytes + (uint64_t)m->dim * 8 + (uint64_t)m->vocab * 4;
        return launch_logits(m->emb, s->x + (size_t)(batch - 1) * m->dim, m->rms_final, m->eps, s->logits, s->st,
                             s->ring, s->ring_cap, advance, st);
    }
    const size_t lay_kv = (size_t)m->kv_ld * m->kv;
    const Layer& L = m->layers[l];
    float* kc = s->kc + (size_t)l * lay_kv;
    float* vc = s->vc + (size_t)l * lay_kv;
    hipError_t e = hipSuccess;
    const bool one = batch == 1;
    switch (cls) {
    case kOpQkv: {
        const int qkv_n = m->att + 2 * m->kv;
        if (bytes) *bytes = (uint64_t)qkv_n * m->dim * 2 + B * ((uint64_t)m->dim * 4 + (uint64_t)qkv_n * 4);
        if (l == 0) e = launch_embed(m->emb, tok, batch, s->x, st);
        if (one) {   // RMSNorm, RoPE and the cache writes inside the GEMV
            F16Qkv qa;
            qa.q_out = s->sq; qa.k_cache = kc; qa.v_cache = vc;
            qa.rope_cos = m->rope_cos; qa.rope_sin = m->rope_sin; qa.st = s->st;
            qa.att = m->att; qa.kv = m->kv; qa.hd = m->hd; qa.kv_ld = m->kv_ld; qa.hf = m->hf_rope;
            if (e == hipSuccess)
                e = launch_f16_gemv((const uint16_t*)L.qkv.qs, m->dim, qkv_n, s->x, L.rms_att, m->eps, 3, nullptr,
                                    st, &qa);
            return e;
        } else {
            if (e == hipSuccess)
                e = launch_rmsnorm(-1, s->x, L.rms_att, m->dim, m->eps, batch, s->xn, nullptr, nullptr, st);
            if (e == hipSuccess)
                e = launch_matmul_f16((const uint16_t*)L.qkv.qs, m->dim, qkv_n, s->xn, batch, s->qkv_raw, qkv_n, 0, st);
        }
        if (e == hipSuccess)
            e = launch_qkv_f16(s->qkv_raw, m->rope_cos, m->rope_sin, s->st, batch, s->sq, kc, vc, m->att, m->kv, m->hd,
                               m->kv_ld, m->hf_rope ? 2 : 0, st);
        return e;
    }
    case kOpAttn:
        if (bytes) *bytes = attn_bytes(m, s, batch);
        return enqueue_attn_f32(m, s, batch, kc, vc);
    case kOpWo:
        if (bytes) *bytes = (uint64_t)m->att * m->dim * 2 + B * ((uint64_t)m->att * 4 + (uint64_t)m->dim * 8);
        return launch_matmul_f16((const uint16_t*)L.wo.qs, m->att, m->dim, s->attf, batch, s->x, m->dim, 1, st);
    case kOpW13:
        // gate and up rows in pairs (32 + 32 per 64-row block), SwiGLU after
        if (bytes) *bytes = 2ull * m->hidden * m->dim * 2 + B * ((uint64_t)m->dim * 4 + (uint64_t)m->hidden * 4);
        if (one)
            return launch_f16_gemv((const uint16_t*)L.w13.qs, m->dim, 2 * m->hidden, s->x, L.rms_ffn, m->eps, 2, s->hf,
                                   st);
        e = launch_rmsnorm(-1, s->x, L.rms_ffn, m->dim, m->eps, batch, s->xn, nullptr, nullptr, st);
        if (e == hipSuccess)
            e = launch_matmul_f16((const uint16_t*)L.w13.qs, m->dim, 2 * m->hidden, s->xn, batch, s->gate,
                                  2 * m->hidden, 0, st);
        if (e == hipSuccess) e = launch_swiglu_pairs(s->gate, m->hidden, batch, s->hf, st);
        return e;
    case kOpW2:
        if (bytes) *bytes = (uint64_t)m->hidden * m->dim * 2 + B * ((uint64_t)m->hidden * 4 + (uint64_t)m->dim * 8);
        return launch_matmul_f16((const uint16_t*)L.w2.qs, m->hidden, m->dim, s->hf, batch, s->x, m->dim, 1, st);
    default:
        return hipErrorInvalidValue;
    }
}

// One op class of layer l of a Q8 model with f32 scales and group size gs
// (forward.rs:120-297 with Q8Kernel; lm.rs and safetensors models): every
// activation row quantized in gs groups, q/gate/up/FFN outputs from zero, K
// and V accumulated onto the cache entries (`+=`), RoPE in place afterwards.
// One token: RMSNorm and quantization run inside the GEMV workgroups, and
// SwiGLU in the gate/up GEMV's epilogue (five kernels per layer and RoPE).
// Prompts: the rows are normalized and quantized once by their own kernels
// first.  `bytes`: int8 weights + f32 scales, the activations read, the
// outputs written.
// The projections of op `cls` of layer l of an f32-scaled Q8 model over
// `batch` tokens on the int8 MFMA GEMM (group sizes 32, 64, 128: the GEMM's
// kQ8S / kQ8S64 / kQ8S128): every input row normalized (QKV, gate/up) and
// quantized in groups of gs by its own kernels first; SwiGLU hands over f32
// h.  hipErrorNotSupported when a shape needs the tile kernel instead.
static hipError_t enqueue_op_gemm_q8g(const yl_model* m, yl_session* s, int cls, int l, int batch,
                                      const uint32_t* tok, float* kc, float* vc, uint64_t* bytes) {
    hipStream_t st = s->stream;
    const Layer& L = m->layers[l];
    const int gs = m->gs;
    GemvArgs a{};
    const QMat* w = nullptr;
    int epi = 0, n = 0;
    const float* in = nullptr;        // the f32 rows quantized for the GEMM
    const float* norm_w = nullptr;    // RMSNorm of the residual stream first
    switch (cls) {
    case kOpQkv:
        w = &L.qkv; epi = kEpiQkvRope; n = m->dim; norm_w = L.rms_att;
        a.q_out = s->sq; a.k_cache = kc; a.v_cache = vc;
        a.att_dim = m->att; a.kv_dim = m->kv; a.head_size = m->hd; a.kv_ld = m->kv_ld;
        a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin; a.state = s->st; a.hf_rows = m->hf_rope;
        break;
    case kOpWo:
        w = &L.wo; epi = kEpiResid; n = m->att; in = s->attf; a.x = s->x;
        break;
    case kOpW13:
        w = &L.w13; epi = kEpiSwiglu; n = m->dim; norm_w = L.rms_ffn;
        a.hq = nullptr; a.hs = nullptr; a.h_f32 = s->hf; a.hidden = m->hidden;
        break;
    case kOpW2:
        w = &L.w2; epi = kEpiResid; n = m->hidden; in = s->hf; a.x = s->x;
        break;
    default:
        return hipErrorNotSupported;
    }
    a.qs = w->qs; a.sf = w->sf; a.n = w->n; a.o = w->o; a.nb = w->nb;
    a.xq = s->gq; a.xs = s->gsc;
    const int wf = gemv_fmt(*w);
    if (!gemm_supported(a, wf, epi, batch)) return hipErrorNotSupported;
    hipError_t e = hipSuccess;
    if (norm_w) {
        if (cls == kOpQkv && l == 0) e = launch_embed(m->emb, tok, batch, s->x, st);
        if (e == hipSuccess) e = launch_rmsnorm(-1, s->x, norm_w, m->dim, m->eps, batch, s->xn, nullptr, nullptr, st);
        in = s->xn;
    }
    if (e == hipSuccess) e = launch_quantize_gs(in, s->gq, s->gsc, gs, (size_t)batch * n, st);
    if (e != hipSuccess) return e;
    if (bytes) *bytes = gemv_bytes(*w, w->o, batch);
    return launch_gemm(a, wf, epi, batch, st);
}

hipError_t enqueue_op_q8g(const yl_model* m, yl_session* s, int cls, int l, int batch, const uint32_t* tok,
                          int advance, uint64_t* bytes) {
    hipStream_t st = s->stream;
    const uint64_t B = (uint64_t)batch;
    const int gs = m->gs;
    if (cls == kOpLogits) {
        if (bytes) *bytes = (uint64_t)m->emb_bytes + (uint64_t)m->dim * 8 + (uint64_t)m->vocab * 4;
        return launch_logits(m->emb, s->x + (size_t)(batch - 1) * m->dim, m->rms_final, m->eps, s->logits, s->st,
                             s->ring, s->ring_cap, advance, st);
    }
    const size_t lay_kv = (size_t)m->kv_ld * m->kv;
    const Layer& L = m->layers[l];
    float* kc = s->kc + (size_t)l * lay_kv;
    float* vc = s->vc + (size_t)l * lay_kv;
    if (m->q8_gemv && batch >= kGemmMinTokens && cls != kOpAttn) {
        const hipError_t e = enqueue_op_gemm_q8g(m, s, cls, l, batch, tok, kc, vc, bytes);
        if (e != hipErrorNotSupported) return e;
    }
    const bool one = batch == 1;
    auto args = [&](const QMat& w, int epi) {
        Q8gArgs a;
        a.w = (const int8_t*)w.qs; a.wsc = w.sf; a.n = w.n; a.o = w.o; a.gs = gs;
        a.epi = epi; a.batch = batch; a.xq = s->gq; a.xs = s->gsc; a.eps = m->eps;
        a.seg[0].row_end = w.o;
        return a;
    };
    // one token: the GEMV makes its input row; prompts: a kernel does, once
    auto input = [&](Q8gArgs& a, const float* x, const float* norm_w, int n) -> hipError_t {
        if (one) {
            a.pro = norm_w ? 2 : 1;
            a.x = x;
            a.norm_w = norm_w;
            return hipSuccess;
        }
        hipError_t e = hipSuccess;
        if (norm_w) {
            e = launch_rmsnorm(-1, x, norm_w, n, m->eps, batch, s->xn, nullptr, nullptr, st);
            x = s->xn;
        }
        if (e == hipSuccess) e = launch_quantize_gs(x, s->gq, s->gsc, gs, (size_t)batch * n, st);
        return e;
    };
    auto xbytes = [&](int n) { return B * (one ? (uint64_t)n * 4 : (uint64_t)n + (uint64_t)(n / gs) * 4); };
    hipError_t e = hipSuccess;
    switch (cls) {
    case kOpQkv: {
        if (bytes) *bytes = L.qkv.bytes() + xbytes(m->dim) + B * ((uint64_t)m->att + 2ull * m->kv) * 4;
        if (l == 0) e = launch_embed(m->emb, tok, batch, s->x, st);
        Q8gArgs a = args(L.qkv, 0);
        if (e == hipSuccess) e = input(a, s->x, L.rms_att, m->dim);
        // q [t][att] from 0; K [kv][kv_ld] and V [pos][kv] from position pos, `+=`
        a.nseg = 3;
        a.perm_hd = m->hd;
        a.st = s->st;
        a.seg[0] = Q8gSegArgs{s->sq, 0, 1, m->att, m->att, 0};
        a.seg[1] = Q8gSegArgs{kc, 1, m->kv_ld, 1, m->att + m->kv, m->kv / 4 * 4};
        a.seg[2] = Q8gSegArgs{vc, m->kv, 1, m->kv, m->att + 2 * m->kv, m->kv / 4 * 4};
        if (e == hipSuccess) e = launch_matmul_q8g(a, st);
        if (e == hipSuccess)
            e = launch_rope_cache(m->rope_cos, m->rope_sin, s->st, batch, s->sq, kc, m->att, m->kv, m->hd, m->kv_ld,
                                  m->hf_rope, st);
        return e;
    }
    case kOpAttn:
        if (bytes) *bytes = attn_bytes(m, s, batch);
        return enqueue_attn_f32(m, s, batch, kc, vc);
    case kOpWo: {
        if (bytes) *bytes = L.wo.bytes() + xbytes(m->att) + B * (uint64_t)m->dim * 8;
        Q8gArgs a = args(L.wo, 1);
        e = input(a, s->attf, nullptr, m->att);
        a.seg[0] = Q8gSegArgs{s->x, 0, 1, m->dim, m->dim, 0};
        if (e == hipSuccess) e = launch_matmul_q8g(a, st);
        return e;
    }
    case kOpW13: {
        if (bytes) *bytes = L.w13.bytes() + xbytes(m->dim) + B * (uint64_t)m->hidden * 4;
        Q8gArgs a = args(L.w13, 2);
        a.pair_rows = m->pair_rows;
        e = input(a, s->x, L.rms_ffn, m->dim);
        a.seg[0] = Q8gSegArgs{s->hf, 0, 1, m->hidden, L.w13.o, 0};
        if (e == hipSuccess) e = launch_matmul_q8g(a, st);
        return e;
    }
    case kOpW2: {
        if (bytes) *bytes = L.w2.bytes() + xbytes(m->hidden) + B * (uint64_t)m->dim * 8;
        Q8gArgs a = args(L.w2, 1);
        e = input(a, s->hf, nullptr, m->hidden);
        a.seg[0] = Q8gSegArgs{s->x, 0, 1, m->dim, m->dim, 0};
        if (e == hipSuccess) e = launch_matmul_q8g(a, st);
        return e;
    }
    default:
        return hipErrorInvalidValue;
    }
}

// One op class of any model's forward pass (the GGUF quantized path, F16,
// or Q8 with f32 group scales).
hipError_t enqueue_class(const yl_model* m, yl_session* s, int cls, int l, int batch, const uint32_t* tok,
                         int advance, uint64_t* bytes, bool prologue = true) {
    if (m->f16) return enqueue_op_f16(m, s, cls, l, batch, tok, advance, bytes);
    // f32-scaled Q8 with group size 32: one token takes the GGUF path's
    // GEMVs (32-blocks, f32 scales), prompts the tile kernel
    if (m->q8g && (batch > 1 || !m->q8_gemv)) return enqueue_op_q8g(m, s, cls, l, batch, tok, advance, bytes);
    return enqueue_op(m, s, cls, l, batch, tok, advance, bytes, prologue);
}

hipError_t enqueue_forward(const yl_model* m, yl_session* s, int batch, const uint32_t* tok, int advance) {
    for (int l = 0; l < m->n_layers; l++)
        for (int c = kOpQkv; c <= kOpW2; c++) {
            const hipError_t e = enqueue_class(m, s, c, l, batch, tok, advance, nullptr);
            if (e != hipSuccess) return e;
        }
    return enqueue_class(m, s, kOpLogits, 0, batch, tok, advance, nullptr);
}

// Decode attention is sized for a context bucket: 4096 positions (the one
// kernel of short contexts), then powers of two, capped at ctx_len, so a
// model loaded with a long context decodes short conversations on the same
// kernels as a short-context model.
int decode_bucket(const yl_model* m, uint64_t seq_end) {
    uint64_t b = 4096;
    while (b < seq_end) b *= 2;
    return (int)(b < (uint64_t)m->ctx ? b : (uint64_t)m->ctx);
}

// The graph of one decode step whose context ends at seq_end (<= ctx_len),
// captured on first use.
hipGraphExec_t ensure_graph(const yl_model* m, yl_session* s, uint64_t seq_end) {
    const int bucket = decode_bucket(m, seq_end);
    for (const auto& dg : s->graphs)
        if (dg.max_seq == bucket) return dg.exec;
    s->dec_seq = bucket;
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        set_error("hipStreamBeginCapture failed");
        return nullptr;
    }
    const hipError_t e = enqueue_forward(m, s, 1, &s->st->token, 1);
    const hipError_t e2 = hipStreamEndCapture(s->stream, &g);
    if (e != hipSuccess || e2 != hipSuccess) {
        set_error(std::string("decode graph capture failed: ") + hipGetErrorString(e != hipSuccess ? e : e2));
        if (g) hipGraphDestroy(g);
        return nullptr;
    }
    hipGraphExec_t ge = nullptr;
    const hipError_t e3 = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e3 != hipSuccess) {
        set_error(std::string("hipGraphInstantiate failed: ") + hipGetErrorString(e3));
        return nullptr;
    }
    s->graphs.push_back({bucket, ge});
    return ge;
}

// Positions a decode step can attend over for this model's head layout.
bool decode_in_range(const yl_model* m, const yl_session* s, uint64_t seq_end, const char* what) {
    if (s->attn_mode == YL_ATTN_SPLIT) return true;   // the split kernel reads any context length
    const int lim = attn_decode_limit(m->n_heads, m->n_kv, m->hd);
    if (seq_end <= (uint64_t)lim) return true;
    set_error(std::string(what) + ": decode attention for this head layout (head_size " + std::to_string(m->hd) +
              ", " + std::to_string(m->n_heads / m->n_kv) + " query heads per kv head) reaches " +
              std::to_string(lim) + " positions");
    return false;
}

yl_status hip_fail(hipError_t e, const char* what) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return YL_ERR_HIP;
}

yl_status put_state(yl_session* s, int32_t pos, uint32_t token) {
    const hipError_t e = launch_set_state(s->st, pos, token, s->stream);
    return e == hipSuccess ? YL_OK : hip_fail(e, "state upload");
}

// A word of pinned host memory that kernels set when one of their bounded
// waits gives up; every synchronizing call reads and clears it.
std::mutex g_fault_mu;
unsigned* g_fault = nullptr;

yl_status check_wait_fault(const char* what) {
    unsigned* f = wait_fault_word(false);
    if (f && __atomic_exchange_n(f, 0u, __ATOMIC_ACQ_REL)) {
        set_error(std::string(what) + ": a kernel's bounded wait timed out; the results of this call are invalid");
        return YL_ERR_HIP;
    }
    return YL_OK;
}

}  // namespace

unsigned* yl::wait_fault_word(bool allocate) {
    std::lock_guard<std::mutex> lk(g_fault_mu);
    if (!g_fault && allocate) {
        void* p = nullptr;
        if (hipHostMalloc(&p, 64, hipHostMallocCoherent | hipHostMallocPortable) == hipSuccess) {
            g_fault = static_cast<unsigned*>(p);
            *g_fault = 0u;
        }
    }
    return g_fault;
}

// ============================================================== C ABI ====

extern "C" {

const char* yl_last_error(void) { return g_err.c_str(); }

yl_status yl_device_count(int* count) {
    if (!count) return YL_ERR_ARG;
    const hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) { *count = 0; return hip_fail(e, "hipGetDeviceCount"); }
    return YL_OK;
}

void* yl_malloc(size_t bytes) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) { hip_fail(e, "hipMalloc"); return nullptr; }
    return p;
}
void yl_free(void* p) { if (p) hipFree(p); }
yl_status yl_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? YL_OK : hip_fail(e, "hipMemcpy H2D");
}
yl_status yl_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? YL_OK : hip_fail(e, "hipMemcpy D2H");
}

yl_status yl_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
    return e == hipSuccess ? YL_OK : hip_fail(e, "hipMemcpy D2D");
}
yl_status yl_memset_d(void* dst, int value, size_t bytes) {
    const hipError_t e = hipMemset(dst, value, bytes);
    return e == hipSuccess ? YL_OK : hip_fail(e, "hipMemset");
}
yl_status yl_synchronize(void) {
    const hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? check_wait_fault("yl_synchronize") : hip_fail(e, "hipDeviceSynchronize");
}

yl_status yl_quantize(yl_format fmt, int8_t* q, float* scale, const float* x, size_t n, uint32_t gs, void* stream) {
    if (gs != 32) { set_error("group size must be 32 (GGUF blocks)"); return YL_ERR_UNSUPPORTED; }
    if (fmt != YL_Q8_0 && fmt != YL_Q4_0) { set_error("quantize: F16 has no quantized form"); return YL_ERR_FORMAT; }
    if (n % 32 || (n && (!q || !scale || !x))) { set_error("quantize: n must be a multiple of 32"); return YL_ERR_ARG; }
    const hipError_t e = launch_quantize(fmt, q, scale, x, n, (hipStream_t)stream);
    return e == hipSuccess ? YL_OK : hip_fail(e, "quantize launch");
}

yl_weight* yl_weight_upload(yl_format fmt, const int8_t* qv, const float* sf, size_t o, size_t n) {
    if ((fmt != YL_Q8_0 && fmt != YL_Q4_0) || !qv || !sf || !o || n % 32) {
        set_error("yl_weight_upload: Q8_0/Q4_0 [o][n] with n a multiple of 32");
        return nullptr;
    }
    HostQMat h;
    h.fmt = fmt == YL_Q4_0 ? kQ4 : kQ8;
    h.o = o; h.n = n; h.nb = n / 32;
    h.d.resize(o * h.nb);
    for (size_t i = 0; i < h.d.size(); i++) {
        if (!float_to_half_exact(sf[i], &h.d[i])) {
            set_error("yl_weight_upload: scale " + std::to_string(i) + " is not exactly representable in binary16");
            return nullptr;
        }
    }
    if (h.fmt == kQ8) {
        h.qs.assign((const uint8_t*)qv, (const uint8_t*)qv + o * n);
    } else {
        h.qs.resize(o * n / 2);
        for (size_t i = 0; i < o * n / 2; i++) {
            const int lo = qv[2 * i], hi = qv[2 * i + 1];
            if (lo < 0 || lo > 15 || hi < 0 || hi > 15) {
                set_error("yl_weight_upload: Q4_0 values must be nibbles 0..15");
                return nullptr;
            }
            h.qs[i] = (uint8_t)(lo | (hi << 4));
        }
    }
    wait_fault_word(true);
    auto* w = new yl_weight();
    std::string err;
    if (!upload_qmat(h, &w->m, &err)) { set_error(err); free_qmat(&w->m); delete w; return nullptr; }
    return w;
}

yl_weight* yl_weight_upload_gguf(yl_format fmt, const void* blocks, size_t o, size_t n) {
    if ((fmt != YL_Q8_0 && fmt != YL_Q4_0) || !blocks || !o || n % 32) {
        set_error("yl_weight_upload_gguf: Q8_0/Q4_0 [o][n] with n a multiple of 32");
        return nullptr;
    }
    HostQMat h;
    std::string err;
    const uint32_t type = fmt == YL_Q4_0 ? kGgmlQ4_0 : kGgmlQ8_0;
    if (!host_from_gguf(type, (const uint8_t*)blocks, ~0ull, o, n, &h, &err)) { set_error(err); return nullptr; }
    wait_fault_word(true);
    auto* w = new yl_weight();
    if (!upload_qmat(h, &w->m, &err)) { set_error(err); free_qmat(&w->m); delete w; return nullptr; }
    return w;
}

void yl_weight_free(yl_weight* w) {
    if (!w) return;
    free_qmat(&w->m);
    delete w;
}

size_t yl_weight_bytes(const yl_weight* w) { return w ? w->m.bytes() : 0; }

yl_weight* yl_weight_upload_f16(const uint16_t* bits, size_t o, size_t n) {
    if (!bits || !o || n % 32) {
        set_error("yl_weight_upload_f16: binary16 [o][n] with n a multiple of 32");
        return nullptr;
    }
    HostQMat h;
    h.fmt = kF16;
    h.o = o; h.n = n; h.nb = 0;
    h.qs.assign((const uint8_t*)bits, (const uint8_t*)bits + o * n * 2);
    auto* w = new yl_weight();
    std::string err;
    if (!upload_qmat(h, &w->m, &err)) { set_error(err); free_qmat(&w->m); delete w; return nullptr; }
    return w;
}

yl_status yl_matmul_f32(float* out, const float* x, size_t batch, const yl_weight* w, size_t n, size_t o, void* stream) {
    if (!w || !out || !x) { set_error("yl_matmul_f32: null argument"); return YL_ERR_ARG; }
    if (w->m.fmt != kF16) { set_error("matmul: format/variant mismatch or mixed formats"); return YL_ERR_FORMAT; }
    if ((int)n != w->m.n || (int)o != w->m.o) { set_error("yl_matmul_f32: n/o do not match the weight"); return YL_ERR_ARG; }
    if (batch == 0) return YL_OK;
    if (batch > 65535) { set_error("yl_matmul_f32: batch > 65535"); return YL_ERR_ARG; }
    const hipError_t e = launch_matmul_f16((const uint16_t*)w->m.qs, (int)n, (int)o, x, (int)batch, out, (int)o, 0,
                                           (hipStream_t)stream);
    return e == hipSuccess ? YL_OK : hip_fail(e, "matmul_f32 launch");
}

yl_status yl_matmul(float* out, yl_format fmt, const int8_t* xq, const float* xs, size_t batch, const yl_weight* w,
                    size_t n, size_t o, uint32_t gs, void* stream) {
    if (!w || !out || !xq || !xs) { set_error("yl_matmul: null argument"); return YL_ERR_ARG; }
    if ((fmt == YL_Q4_0 ? kQ4 : (fmt == YL_Q8_0 ? kQ8 : -1)) != w->m.fmt) {
        set_error("matmul: format/variant mismatch or mixed formats");
        return YL_ERR_FORMAT;
    }
    if (gs != 32) { set_error("group size must be 32 (GGUF blocks)"); return YL_ERR_UNSUPPORTED; }
    if ((int)n != w->m.n || (int)o != w->m.o) { set_error("yl_matmul: n/o do not match the weight"); return YL_ERR_ARG; }
    if (batch == 0) return YL_OK;
    if (batch > 65535) { set_error("yl_matmul: batch > 65535"); return YL_ERR_ARG; }
    GemvArgs a{};
    a.qs = w->m.qs; a.d = w->m.d; a.n = w->m.n; a.o = w->m.o; a.nb = w->m.nb;
    a.xq = xq; a.xs = xs; a.out = out; a.accumulate_cols = (int)(o / 4 * 4);
    const bool mfma = batch >= (size_t)kGemmMinTokens && gemm_supported(a, w->m.fmt, kEpiStore, (int)batch);
    const hipError_t e = mfma ? launch_gemm(a, w->m.fmt, kEpiStore, (int)batch, (hipStream_t)stream)
                              : launch_gemv(a, w->m.fmt, kEpiStore, (int)batch, (hipStream_t)stream);
    return e == hipSuccess ? YL_OK : hip_fail(e, "matmul launch");
}

yl_status yl_matmul_bench(const yl_weight* const* ws, size_t count, const int8_t* xq, const float* xs, size_t batch,
                          float* out, uint32_t reps, double* us_per_launch) {
    if (!ws || count == 0 || !xq || !xs || !out || reps == 0 || batch == 0 || batch > 65535) {
        set_error("matmul_bench: bad arguments");
        return YL_ERR_ARG;
    }
    for (size_t i = 0; i < count; i++)
        if (!ws[i] || ws[i]->m.n != ws[0]->m.n || ws[i]->m.o != ws[0]->m.o || ws[i]->m.fmt != ws[0]->m.fmt) {
            set_error("matmul_bench: weights must share format and shape");
            return YL_ERR_ARG;
        }
    hipStream_t st = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "matmul_bench stream");
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    hipError_t ec = hipSuccess;
    for (size_t i = 0; i < count && e == hipSuccess && ec == hipSuccess; i++) {
        const QMat& w = ws[i]->m;
        GemvArgs a{};
        a.qs = w.qs; a.d = w.d; a.n = w.n; a.o = w.o; a.nb = w.nb;
        a.xq = xq; a.xs = xs; a.out = out; a.accumulate_cols = 0;
        const bool mfma = batch >= (size_t)kGemmMinTokens && gemm_supported(a, w.fmt, kEpiStore, (int)batch);
        ec = mfma ? launch_gemm(a, w.fmt, kEpiStore, (int)batch, st) : launch_gemv(a, w.fmt, kEpiStore, (int)batch, st);
    }
    if (e == hipSuccess) e = hipStreamEndCapture(st, &g);
    if (e == hipSuccess) e = ec;
    if (e == hipSuccess) e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipGraphLaunch(ge, st);
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    for (uint32_t r = 0; r < reps && e == hipSuccess; r++) e = hipGraphLaunch(ge, st);
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (ge) hipGraphExecDestroy(ge);
    if (g) hipGraphDestroy(g);
    hipStreamDestroy(st);
    if (e != hipSuccess) return hip_fail(e, "matmul_bench");
    if (check_wait_fault("matmul_bench") != YL_OK) return YL_ERR_HIP;
    if (us_per_launch) *us_per_launch = (double)ms * 1000.0 / ((double)reps * (double)count);
    return YL_OK;
}

yl_status yl_rmsnorm_quantize(const float* x, const float* weight, size_t size, float eps, size_t batch, float* xn,
                              int32_t qfmt, int8_t* q, float* scale, void* stream) {
    if (!x || !weight || !size || size > 8192) { set_error("rmsnorm: bad arguments (size <= 8192)"); return YL_ERR_ARG; }
    if (qfmt >= 0 && (size % 32 || !q || !scale || qfmt > 1)) { set_error("rmsnorm: quantized output needs size % 32 == 0"); return YL_ERR_ARG; }
    if (batch == 0) return YL_OK;
    const hipError_t e = launch_rmsnorm(qfmt, x, weight, (int)size, eps, (int)batch, xn, q, scale, (hipStream_t)stream);
    return e == hipSuccess ? YL_OK : hip_fail(e, "rmsnorm launch");
}

yl_status yl_rope_gguf(const yl_rope_params* p, float* q, float* k, size_t batch, uint32_t start_pos, void* stream) {
    if (!p || !q || !k || p->head_size % 2 || !p->head_size) { set_error("rope: bad arguments"); return YL_ERR_ARG; }
    if (batch == 0) return YL_OK;
    const size_t half = p->head_size / 2;
    std::vector<float> c(batch * half), s(batch * half);
    rope_table(*p, start_pos, (uint32_t)batch, c.data(), s.data());
    float *dc = nullptr, *ds = nullptr;
    StepState* dst = nullptr;
    StepState hst{};
    hst.pos = 0;
    hipStream_t strm = (hipStream_t)stream;
    hipError_t e = hipMalloc(&dc, c.size() * 4);
    if (e == hipSuccess) e = hipMalloc(&ds, s.size() * 4);
    if (e == hipSuccess) e = hipMalloc(&dst, sizeof(StepState));
    if (e == hipSuccess) e = hipMemcpy(dc, c.data(), c.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(ds, s.data(), s.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dst, &hst, sizeof hst, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_rope(dc, ds, dst, (int)batch, q, k, p->n_heads, p->n_kv_heads, p->head_size, strm);
    if (e == hipSuccess) e = hipStreamSynchronize(strm);
    if (dc) hipFree(dc);
    if (ds) hipFree(ds);
    if (dst) hipFree(dst);
    return e == hipSuccess ? YL_OK : hip_fail(e, "rope");
}

}  // extern "C"

namespace {

// Buffers an attention op call needs beyond its inputs and outputs: the
// step state (the call's first position), the keys transposed to the
// kernels' [kv_dim][ld] layout (the caller's are [seq][kv_dim]), and the
// scores scratch of long decode contexts or of tiled prompt batches.
struct AttnBuffers {
    int ld = 0, kv_dim = 0;
    size_t kt_bytes = 0, sc_bytes = 0;
};

yl_status attention_plan(const float* out, const float* q, const float* kc, const float* vc, size_t batch,
                         uint32_t start_pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t hd, AttnBuffers* B) {
    if (!out || !q || !kc || !vc || !n_heads || !n_kv_heads || n_heads % n_kv_heads || hd % 8 || !hd) {
        set_error("attention: bad arguments");
        return YL_ERR_ARG;
    }
    const size_t seq = start_pos + batch;
    if (seq >= (1u << 30) || (uint64_t)seq * n_kv_heads * hd * 4 >= (1ull << 31)) {
        set_error("attention: the cache must stay below 2 GiB");
        return YL_ERR_UNSUPPORTED;
    }
    // one token: the decode kernels (as in a decode step); several: the
    // prompt kernels (one score row per workgroup, or tiled)
    const bool tiled = prompt_attn_applies((int)batch, (int)seq, (int)hd);
    if (tiled && hd != 32 && hd != 64 && hd != 128) {
        set_error("attention: tiled prompt attention needs head_size 32, 64 or 128");
        return YL_ERR_UNSUPPORTED;
    }
    if (batch == 1 && (hd % 32 || hd > 128 || !attn_decode_fits((int)seq, (int)n_heads, (int)n_kv_heads, (int)hd))) {
        set_error("attention: unsupported head size or seq_len for the decode kernel");
        return YL_ERR_UNSUPPORTED;
    }
    B->kv_dim = (int)(n_kv_heads * hd);
    B->ld = ((int)seq + 3) & ~3;
    B->kt_bytes = ((size_t)B->ld * B->kv_dim * 4 + 255) & ~(size_t)255;
    B->sc_bytes = batch == 1 ? attn_scores_bytes((int)n_heads, (int)seq)
                  : tiled    ? prompt_attn_bytes((int)n_heads, (int)seq, (int)batch)
                             : 0;
    return YL_OK;
}

// Enqueues one attention op call on `strm` over the buffers of `B`.
hipError_t attention_enqueue(float* out, const float* q, const float* kc, const float* vc, size_t batch,
                             uint32_t start_pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t hd, float attn_scale,
                             const AttnBuffers& B, StepState* dst, float* kt, float* sc, hipStream_t strm) {
    const int seq = (int)(start_pos + batch);
    hipError_t e = launch_set_state(dst, (int32_t)start_pos, 0u, strm);
    if (e == hipSuccess) e = launch_transpose(kc, kt, seq, B.kv_dim, B.ld, strm);
    if (e != hipSuccess) return e;
    if (batch == 1)
        return launch_attn_decode(q, kt, vc, dst, seq, B.ld, (int)n_heads, (int)n_kv_heads, (int)hd, attn_scale, -1,
                                  nullptr, nullptr, out, sc, strm);
    if (sc)
        return launch_prompt_attention(q, kt, vc, dst, (int)batch, seq, B.ld, (int)n_heads, (int)n_kv_heads, (int)hd,
                                       attn_scale, -1, nullptr, nullptr, out, sc, strm);
    return launch_attention(q, kt, vc, dst, (int)batch, seq, B.ld, (int)n_heads, (int)n_kv_heads, (int)hd,
                            attn_scale, -1, nullptr, nullptr, out, strm);
}

}  // namespace

extern "C" {

yl_status yl_attention(float* out, const float* q, const float* kc, const float* vc, size_t batch, uint32_t start_pos,
                       uint32_t n_heads, uint32_t n_kv_heads, uint32_t hd, float attn_scale, void* stream) {
    AttnBuffers B;
    const yl_status st = attention_plan(out, q, kc, vc, batch, start_pos, n_heads, n_kv_heads, hd, &B);
    if (st != YL_OK || batch == 0) return st;
    StepState* dst = nullptr;
    float *kt = nullptr, *sc = nullptr;
    hipStream_t strm = (hipStream_t)stream;
    hipError_t e = hipMalloc(&dst, sizeof(StepState));
    if (e == hipSuccess) e = hipMalloc(&kt, B.kt_bytes);
    if (e == hipSuccess && B.sc_bytes) e = hipMalloc(&sc, B.sc_bytes);
    if (e == hipSuccess)
        e = attention_enqueue(out, q, kc, vc, batch, start_pos, n_heads, n_kv_heads, hd, attn_scale, B, dst, kt, sc,
                              strm);
    if (e == hipSuccess) e = hipStreamSynchronize(strm);
    if (dst) hipFree(dst);
    if (kt) hipFree(kt);
    if (sc) hipFree(sc);
    return e == hipSuccess ? YL_OK : hip_fail(e, "attention");
}

yl_status yl_attention_split(float* out, const float* q, const float* kc, const float* vc, uint32_t start_pos,
                             uint32_t n_heads, uint32_t n_kv_heads, uint32_t hd, float attn_scale, void* stream) {
    if (!out || !q || !kc || !vc || !n_kv_heads || n_heads % n_kv_heads ||
        !attn_split_supported((int)n_heads, (int)n_kv_heads, (int)hd)) {
        set_error("attention_split: head size 64 or 128 with 1, 2, 4 or 8 query heads per kv head");
        return YL_ERR_ARG;
    }
    const size_t seq = (size_t)start_pos + 1, kv_dim = (size_t)n_kv_heads * hd;
    if (seq >= (1u << 30) || seq * kv_dim * 4 >= (1ull << 31)) {
        set_error("attention_split: the cache must stay below 2 GiB");
        return YL_ERR_UNSUPPORTED;
    }
    const int ld = ((int)seq + 3) & ~3;
    const size_t kt_bytes = (size_t)ld * kv_dim * 4, sp_bytes = attn_split_bytes((int)n_heads, (int)n_kv_heads, (int)hd);
    StepState* dst = nullptr;
    float *kt = nullptr, *sp = nullptr;
    hipStream_t strm = (hipStream_t)stream;
    hipError_t e = hipMalloc(&dst, sizeof(StepState));
    if (e == hipSuccess) e = hipMalloc(&kt, kt_bytes);
    if (e == hipSuccess) e = hipMalloc(&sp, sp_bytes);
    if (e == hipSuccess) e = hipMemsetAsync(sp, 0, sp_bytes, strm);
    if (e == hipSuccess) e = launch_set_state(dst, (int32_t)start_pos, 0u, strm);
    if (e == hipSuccess) e = launch_transpose(kc, kt, (int)seq, (int)kv_dim, ld, strm);
    if (e == hipSuccess)
        e = launch_attn_split(q, kt, vc, dst, ld, (int)n_heads, (int)n_kv_heads, (int)hd, attn_scale, -1, nullptr,
                              nullptr, out, sp, strm);
    if (e == hipSuccess) e = hipStreamSynchronize(strm);
    if (dst) hipFree(dst);
    if (kt) hipFree(kt);
    if (sp) hipFree(sp);
    return e == hipSuccess ? YL_OK : hip_fail(e, "attention_split");
}

}  // extern "C"

// ---------------------------------------------- allocation-free attention
// yl_attention_noalloc keeps the step state, the transposed keys and the
// scores scratch of a call in this array instead of hipMalloc'ed buffers.
// Every GPU the library runs on holds its own copy until the process ends;
// host code reaches a device's copy only through the address that
// hipGetSymbolAddress returns with that device current (the array's name is
// a host-side stand-in, not a device address).
constexpr size_t kNoAllocScratchBytes = 64ull << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_dev[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up on the first call on
// each device.
yl_status scratch_of_current_device(unsigned char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("attention_noalloc: device index beyond " + std::to_string(kMaxDevices));
        return YL_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) {
            set_error("hipGetSymbolAddress(scratch) returned a null address");
            return YL_ERR_HIP;
        }
        g_scratch_dev[dev] = static_cast<unsigned char*>(p);
    }
    *out = g_scratch_dev[dev];
    return YL_OK;
}

}  // namespace

extern "C" {

yl_status yl_attention_noalloc(float* out, const float* q, const float* kc, const float* vc, size_t batch,
                               uint32_t start_pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t hd,
                               float attn_scale, void* stream) {
    AttnBuffers B;
    yl_status st = attention_plan(out, q, kc, vc, batch, start_pos, n_heads, n_kv_heads, hd, &B);
    if (st != YL_OK || batch == 0) return st;
    const size_t sc_off = 256 + B.kt_bytes;
    const size_t need = sc_off + ((B.sc_bytes + 255) & ~(size_t)255);
    if (need > kNoAllocScratchBytes) {
        set_error("attention_noalloc: the call needs " + std::to_string(need) + " bytes of scratch, more than the " +
                  std::to_string(kNoAllocScratchBytes) + " the library holds per GPU");
        return YL_ERR_RANGE;
    }
    unsigned char* base = nullptr;
    st = scratch_of_current_device(&base);
    if (st != YL_OK) return st;
    StepState* dst = reinterpret_cast<StepState*>(base);
    float* kt = reinterpret_cast<float*>(base + 256);
    float* sc = B.sc_bytes ? reinterpret_cast<float*>(base + sc_off) : nullptr;
    const hipError_t e = attention_enqueue(out, q, kc, vc, batch, start_pos, n_heads, n_kv_heads, hd, attn_scale, B,
                                           dst, kt, sc, (hipStream_t)stream);
    return e == hipSuccess ? YL_OK : hip_fail(e, "attention_noalloc");
}

yl_status yl_swiglu_quantize(const float* gate, const float* up, size_t hidden, size_t batch, float* h, int32_t qfmt,
                             int8_t* q, float* scale, void* stream) {
    if (!gate || !up || !hidden) { set_error("swiglu: bad arguments"); return YL_ERR_ARG; }
    if (qfmt >= 0 && (hidden % 32 || !q || !scale || qfmt > 1)) { set_error("swiglu: quantized output needs hidden % 32 == 0"); return YL_ERR_ARG; }
    if (batch == 0) return YL_OK;
    const hipError_t e = launch_swiglu_quant(qfmt, gate, up, (int)hidden, (int)batch, h, q, scale, (hipStream_t)stream);
    return e == hipSuccess ? YL_OK : hip_fail(e, "swiglu launch");
}

yl_status yl_math_selftest(const float* x, size_t n, float* exp_out, float* sqrt_out, float* recip_out, float* f16_out) {
    if (!n) return YL_OK;
    hipError_t e = launch_math_selftest(x, (int)n, exp_out, sqrt_out, recip_out, f16_out, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return e == hipSuccess ? YL_OK : hip_fail(e, "math selftest");
}

yl_status yl_serial_sum_selftest(const float* v, const uint32_t* offsets, size_t cases, uint32_t segment,
                                 float* out) {
    if ((!v || !offsets || !out) && cases) return YL_ERR_ARG;
    if (segment > (1u << 30) && segment < 0xFFFFFFFEu) return YL_ERR_ARG;
    wait_fault_word(true);
    const int seg = segment == 0xFFFFFFFFu ? -1 : (segment == 0xFFFFFFFEu ? -2 : (int)segment);
    hipError_t e = launch_serial_sum_selftest(v, offsets, (int)cases, seg, out, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess && check_wait_fault("serial sum self-test") != YL_OK) return YL_ERR_HIP;
    return e == hipSuccess ? YL_OK : hip_fail(e, "serial sum self-test");
}

// ---------------------------------------------------------------- model

// The extension of a path as Rust's Path::extension gives it (lib.rs:112):
// the file name is the last component (trailing separators and "."
// components ignored; none for "/" or a ".." component), and the extension
// is what follows its last '.', unless it has no '.' or only a leading one.
// `has` is false when there is none.
static std::string path_extension(const std::string& path, bool* has) {
    *has = false;
    std::string p = path;
    for (;;) {
        while (p.size() > 1 && p.back() == '/') p.pop_back();
        if (p.size() >= 2 && p.compare(p.size() - 2, 2, "/.") == 0) { p.resize(p.size() - 2); continue; }
        break;
    }
    if (p.empty() || p == "/" || p == ".") return "";
    const size_t slash = p.rfind('/');
    const std::string name = slash == std::string::npos ? p : p.substr(slash + 1);
    if (name.empty() || name == "..") return "";
    const size_t dot = name.rfind('.');
    if (dot == std::string::npos || dot == 0) return "";
    *has = true;
    return name.substr(dot + 1);
}

yl_model* yl_load(const char* path, uint32_t max_ctx_len, int32_t fmt_override) {
    if (!path) { set_error("null path"); return nullptr; }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) { set_error("no HIP device"); return nullptr; }
    yl_status st;
    // lib.rs:107-133: the loader by file extension
    const std::string p(path);
    bool has_ext = false;
    const std::string ext = path_extension(p, &has_ext);
    if (has_ext && (ext == "safetensors" || ext == "lmrs")) {
        HostModel h;
        std::string err;
        const bool ok = ext == "lmrs" ? load_lmrs(p, max_ctx_len, fmt_override, &h, &err)
                                      : load_safetensors(p, max_ctx_len, fmt_override, &h, &err);
        if (!ok) { set_error(err); return nullptr; }
        return model_from_host(h, &st);
    }
    return load_model(path, max_ctx_len, fmt_override, &st);
}

void yl_model_free(yl_model* m) { model_release(m); }
const char* yl_model_name(const yl_model* m) { return m ? m->name.c_str() : ""; }
yl_status yl_wait_fault_selftest(void) {
    unsigned* f = wait_fault_word(true);
    if (!f) { set_error("wait_fault_selftest: no fault word (pinned allocation failed)"); return YL_ERR_HIP; }
    const hipError_t e = launch_raise_fault(f, nullptr);
    return e == hipSuccess ? YL_OK : hip_fail(e, "wait_fault_selftest");
}

yl_status yl_model_shape(const yl_model* m, yl_shape* out) {
    if (!m || !out) return YL_ERR_ARG;
    *out = m->shape;
    return YL_OK;
}
size_t yl_vocab_size(const yl_model* m) { return m ? (size_t)m->vocab : 0; }
uint32_t yl_max_ctx_len(const yl_model* m) { return m ? (uint32_t)m->ctx : 2048; }
uint32_t yl_bos_token(const yl_model* m) { return m ? m->bos : 0; }
uint32_t yl_eos_token(const yl_model* m) { return m ? m->eos : 0; }
size_t yl_model_weight_bytes(const yl_model* m) { return m ? m->weight_bytes : 0; }
size_t yl_model_embedding_bytes(const yl_model* m) { return m ? m->emb_bytes : 0; }

yl_status yl_get_embeddings(const yl_model* m, const uint32_t* tokens, size_t n, float* out) {
    if (!m || (!tokens && n) || (!out && n)) return YL_ERR_ARG;
    if (!n) return YL_OK;
    float* x = nullptr;
    uint32_t* t = nullptr;
    hipError_t e = hipMalloc(&x, n * m->dim * 4);
    if (e == hipSuccess) e = hipMalloc(&t, n * 4);
    if (e == hipSuccess) e = hipMemcpy(t, tokens, n * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_embed(m->emb, t, (int)n, x, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, x, n * m->dim * 4, hipMemcpyDeviceToHost);
    if (x) hipFree(x);
    if (t) hipFree(t);
    return e == hipSuccess ? YL_OK : hip_fail(e, "get_embeddings");
}

yl_session* yl_create_session(const yl_model* m) {
    if (!m) { set_error("null model"); return nullptr; }
    wait_fault_word(true);
    auto* s = new yl_session();
    s->m = m;
    s->kv_floats = (size_t)m->n_layers * m->kv_ld * m->kv;
    s->ring_cap = (uint32_t)m->ctx;
    bool ok = hipStreamCreate(&s->stream) == hipSuccess &&
              hipMalloc(&s->kc, s->kv_floats * 4 + 256) == hipSuccess &&
              hipMalloc(&s->vc, s->kv_floats * 4 + 256) == hipSuccess &&
              hipMemset(s->kc, 0, s->kv_floats * 4) == hipSuccess &&
              hipMemset(s->vc, 0, s->kv_floats * 4) == hipSuccess &&
              hipMalloc(&s->st, sizeof(StepState)) == hipSuccess &&
              hipMemset(s->st, 0, sizeof(StepState)) == hipSuccess &&
              hipHostMalloc(&s->st_host, sizeof(StepState), 0) == hipSuccess &&
              hipMalloc(&s->logits, (size_t)m->vocab * 4 + 256) == hipSuccess &&
              hipMalloc(&s->ring, (size_t)s->ring_cap * 4 + 256) == hipSuccess &&
              session_grow(s, 1);
    const size_t sc_bytes = attn_scores_bytes(m->n_heads, m->ctx);
    if (ok && sc_bytes) ok = hipMalloc(&s->sc, sc_bytes) == hipSuccess;
    if (!ok) {
        if (yl_last_error()[0] == 0) set_error("session allocation failed");
        yl_session_free(s);
        return nullptr;
    }
    return s;
}

void yl_session_free(yl_session* s) {
    if (!s) return;
    if (s->stream) hipStreamSynchronize(s->stream);
    for (auto& g : s->graphs) hipGraphExecDestroy(g.exec);
    void* dev[] = {s->kc, s->vc, s->st, s->logits, s->ring, s->x, s->sq, s->aq, s->hq,
                   s->as_, s->hs, s->nq, s->ns, s->tokens, s->sc, s->psc, s->split,
                   s->xn, s->qkv_raw, s->attf, s->gate, s->up, s->hf, s->gq, s->gsc};
    for (void* p : dev) if (p) hipFree(p);
    if (s->st_host) hipHostFree(s->st_host);
    if (s->stream) hipStreamDestroy(s->stream);
    delete s;
}

yl_status yl_session_set_attention(yl_session* s, int32_t mode) {
    if (!s || (mode != YL_ATTN_EXACT && mode != YL_ATTN_SPLIT)) { set_error("set_attention: bad arguments"); return YL_ERR_ARG; }
    const yl_model* m = s->m;
    if (mode == YL_ATTN_SPLIT && !attn_split_supported(m->n_heads, m->n_kv, m->hd)) {
        set_error("set_attention: the split decode attention takes head size 64 or 128 with 1, 2, 4 or 8 query "
                  "heads per kv head");
        return YL_ERR_UNSUPPORTED;
    }
    if (mode == s->attn_mode) return YL_OK;
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e, "set_attention");
    if (mode == YL_ATTN_SPLIT && !s->split) {
        // the counts must start at zero; every launch leaves them zero
        const size_t bytes = attn_split_bytes(m->n_heads, m->n_kv, m->hd);
        e = hipMalloc(&s->split, bytes);
        if (e == hipSuccess) e = hipMemset(s->split, 0, bytes);
        if (e != hipSuccess) {
            if (s->split) hipFree(s->split);
            s->split = nullptr;
            return hip_fail(e, "set_attention scratch");
        }
    }
    // the decode graphs captured the other attention
    for (auto& g : s->graphs) hipGraphExecDestroy(g.exec);
    s->graphs.clear();
    s->attn_mode = mode;
    return YL_OK;
}

yl_status yl_session_reset(yl_session* s) {
    if (!s) return YL_ERR_ARG;
    hipError_t e = hipMemsetAsync(s->kc, 0, s->kv_floats * 4, s->stream);
    if (e == hipSuccess) e = hipMemsetAsync(s->vc, 0, s->kv_floats * 4, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    s->pos = 0;
    return e == hipSuccess ? YL_OK : hip_fail(e, "session reset");
}

uint32_t yl_session_pos(const yl_session* s) { return s ? s->pos : 0; }
void yl_session_set_pos(yl_session* s, uint32_t pos) { if (s) s->pos = pos; }

yl_status yl_session_kv(yl_session* s, float** k, float** v, size_t* floats) {
    if (!s) return YL_ERR_ARG;
    if (k) *k = s->kc;
    if (v) *v = s->vc;
    if (floats) *floats = s->kv_floats;
    return YL_OK;
}

yl_status yl_forward_x(const yl_model* m, const uint32_t* tokens, size_t n, uint32_t start_pos, yl_session* s,
                       float* logits, uint32_t* argmax) {
    if (!m || !s || s->m != m || !tokens) { set_error("forward_x: null model/session/tokens"); return YL_ERR_ARG; }
    if (n == 0) { set_error("forward_x: empty token batch"); return YL_ERR_ARG; }
    if ((uint64_t)start_pos + n > (uint64_t)m->ctx) {
        set_error("forward_x: positions beyond ctx_len " + std::to_string(m->ctx));
        return YL_ERR_RANGE;
    }
    if (n > 65535) { set_error("forward_x: more than 65535 tokens in one call"); return YL_ERR_ARG; }
    if (n == 1 && !decode_in_range(m, s, (uint64_t)start_pos + 1, "forward_x")) return YL_ERR_RANGE;
    yl_status rs = put_state(s, (int32_t)start_pos, tokens[0]);
    if (rs != YL_OK) return rs;
    hipError_t e;
    if (n == 1) {
        hipGraphExec_t ge = ensure_graph(m, s, (uint64_t)start_pos + 1);
        if (!ge) return YL_ERR_HIP;
        e = hipGraphLaunch(ge, s->stream);
        if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
    } else {
        if (!session_grow(s, (int)n) || !prompt_scratch(s, (int)n, start_pos)) return YL_ERR_NOMEM;
        e = hipMemcpyAsync(s->tokens, tokens, n * 4, hipMemcpyHostToDevice, s->stream);
        if (e != hipSuccess) return hip_fail(e, "token upload");
        e = enqueue_forward(m, s, (int)n, s->tokens, 0);
        if (e != hipSuccess) return hip_fail(e, "forward launch");
    }
    if (logits) {
        e = hipMemcpyAsync(logits, s->logits, (size_t)m->vocab * 4, hipMemcpyDeviceToHost, s->stream);
        if (e != hipSuccess) return hip_fail(e, "logits download");
    }
    e = hipMemcpyAsync(s->st_host, s->st, sizeof(StepState), hipMemcpyDeviceToHost, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return hip_fail(e, "forward_x");
    if (check_wait_fault("forward_x") != YL_OK) return YL_ERR_HIP;
    if (argmax) *argmax = s->st_host->token;
    return YL_OK;
}

yl_status yl_generate_greedy(const yl_model* m, yl_session* s, uint32_t token, uint32_t start_pos, uint32_t n_steps,
                             uint32_t* out_tokens) {
    if (!m || !s || s->m != m) { set_error("generate: null model/session"); return YL_ERR_ARG; }
    if (n_steps == 0) return YL_OK;
    if ((uint64_t)start_pos + n_steps > (uint64_t)m->ctx) {
        set_error("generate: positions beyond ctx_len " + std::to_string(m->ctx));
        return YL_ERR_RANGE;
    }
    if (!decode_in_range(m, s, (uint64_t)start_pos + n_steps, "generate")) return YL_ERR_RANGE;
    yl_status rs = put_state(s, (int32_t)start_pos, token);
    if (rs != YL_OK) return rs;
    // steps of one context bucket replay that bucket's graph (the position
    // and token live on the device, so the graphs hand over seamlessly)
    for (uint32_t i = 0; i < n_steps;) {
        const uint64_t seq = (uint64_t)start_pos + i + 1;
        const int bucket = decode_bucket(m, seq);
        hipGraphExec_t ge = ensure_graph(m, s, seq);
        if (!ge) return YL_ERR_HIP;
        const uint32_t end = (uint64_t)bucket - start_pos < n_steps ? (uint32_t)(bucket - start_pos) : n_steps;
        for (; i < end; i++) {
            const hipError_t e = hipGraphLaunch(ge, s->stream);
            if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
        }
    }
    hipError_t e = hipSuccess;
    if (out_tokens) e = hipMemcpyAsync(out_tokens, s->ring, (size_t)n_steps * 4, hipMemcpyDeviceToHost, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    return e == hipSuccess ? check_wait_fault("generate") : hip_fail(e, "generate");
}

yl_status yl_profile_kernel(const yl_model* m, yl_session* s, uint32_t token, uint32_t start_pos, uint32_t batch,
                            int32_t kernel_class, uint32_t reps, double* us_per_launch, uint64_t* bytes_per_launch,
                            uint32_t* launches) {
    if (!m || !s || s->m != m || kernel_class < kOpQkv || kernel_class > kOpLogits || reps == 0 || batch == 0 ||
        batch > 65535) {
        set_error("profile: bad arguments");
        return YL_ERR_ARG;
    }
    if ((uint64_t)start_pos + batch > (uint64_t)m->ctx) { set_error("profile: position beyond ctx_len"); return YL_ERR_RANGE; }
    if (batch == 1 && !decode_in_range(m, s, (uint64_t)start_pos + 1, "profile")) return YL_ERR_RANGE;
    s->dec_seq = decode_bucket(m, (uint64_t)start_pos + 1);
    s->prof_seq = (uint64_t)start_pos + batch;
    if (batch > 1 && (!session_grow(s, (int)batch) || !prompt_scratch(s, (int)batch, start_pos)))
        return YL_ERR_NOMEM;
    yl_status rs = put_state(s, (int32_t)start_pos, token);
    if (rs != YL_OK) return rs;
    // one graph: this class's launches of one step, back to back
    const int n_launch = kernel_class == kOpLogits ? 1 : m->n_layers;
    uint64_t nbytes = 0;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(e, "profile capture");
    hipError_t ec = hipSuccess;
    for (int l = 0; l < n_launch && ec == hipSuccess; l++) {
        uint64_t b = 0;
        ec = enqueue_class(m, s, kernel_class, l, (int)batch, batch == 1 ? &s->st->token : s->tokens, 0, &b, false);
        nbytes += b;
    }
    e = hipStreamEndCapture(s->stream, &g);
    if (ec != hipSuccess || e != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return hip_fail(ec != hipSuccess ? ec : e, "profile capture");
    }
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "profile instantiate");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    for (int w = 0; w < 2 && e == hipSuccess; w++) e = hipGraphLaunch(ge, s->stream);
    if (e == hipSuccess) e = hipEventRecord(e0, s->stream);
    for (uint32_t r = 0; r < reps && e == hipSuccess; r++) e = hipGraphLaunch(ge, s->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, s->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    hipGraphExecDestroy(ge);
    if (e != hipSuccess) return hip_fail(e, "profile");
    if (check_wait_fault("profile") != YL_OK) return YL_ERR_HIP;
    if (us_per_launch) *us_per_launch = (double)ms * 1000.0 / ((double)reps * n_launch);
    // (the replays leave the prompt buffers of the session in use)
    if (bytes_per_launch) *bytes_per_launch = nbytes / (uint64_t)n_launch;
    if (launches) *launches = (uint32_t)n_launch;
    return YL_OK;
}


yl_status yl_profile_step(const yl_model* m, yl_session* s, uint32_t token, uint32_t start_pos, int32_t skip_class,
                          uint32_t reps, double* us_per_step) {
    if (!m || !s || s->m != m || skip_class < -1 || skip_class > kOpLogits || reps == 0 || !us_per_step) {
        set_error("profile_step: bad arguments");
        return YL_ERR_ARG;
    }
    if ((uint64_t)start_pos + 1 > (uint64_t)m->ctx) { set_error("profile_step: position beyond ctx_len"); return YL_ERR_RANGE; }
    if (!decode_in_range(m, s, (uint64_t)start_pos + 1, "profile_step")) return YL_ERR_RANGE;
    s->dec_seq = decode_bucket(m, (uint64_t)start_pos + 1);
    s->prof_seq = (uint64_t)start_pos + 1;
    yl_status rs = put_state(s, (int32_t)start_pos, token);
    if (rs != YL_OK) return rs;
    // one decode step as its graph launches it, without the skipped class's
    // launches (the logits kernel leaves the position where it is)
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(e, "profile_step capture");
    hipError_t ec = hipSuccess;
    for (int l = 0; l < m->n_layers && ec == hipSuccess; l++)
        for (int c = kOpQkv; c <= kOpW2 && ec == hipSuccess; c++)
            if (c != skip_class) ec = enqueue_class(m, s, c, l, 1, &s->st->token, 0, nullptr);
    if (ec == hipSuccess && skip_class != kOpLogits) ec = enqueue_class(m, s, kOpLogits, 0, 1, &s->st->token, 0, nullptr);
    e = hipStreamEndCapture(s->stream, &g);
    if (ec != hipSuccess || e != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return hip_fail(ec != hipSuccess ? ec : e, "profile_step capture");
    }
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "profile_step instantiate");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    for (int w = 0; w < 2 && e == hipSuccess; w++) e = hipGraphLaunch(ge, s->stream);
    if (e == hipSuccess) e = hipEventRecord(e0, s->stream);
    for (uint32_t r = 0; r < reps && e == hipSuccess; r++) e = hipGraphLaunch(ge, s->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, s->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    hipGraphExecDestroy(ge);
    if (e != hipSuccess) return hip_fail(e, "profile_step");
    if (check_wait_fault("profile_step") != YL_OK) return YL_ERR_HIP;
    *us_per_step = (double)ms * 1000.0 / (double)reps;
    return YL_OK;
}

yl_status yl_profile_stream(const yl_model* m, yl_session* s, int32_t kernel_class, uint32_t reps,
                            double* us_per_launch, uint64_t* bytes_per_launch) {
    if (!m || !s || s->m != m || reps == 0 || !us_per_launch ||
        (kernel_class != kOpQkv && kernel_class != kOpWo && kernel_class != kOpW13 && kernel_class != kOpW2)) {
        set_error("profile_stream: bad arguments");
        return YL_ERR_ARG;
    }
    if (m->f16 || m->q8g) { set_error("profile_stream: GGUF Q8_0/Q4_0 weights only"); return YL_ERR_UNSUPPORTED; }
    const int epi = kernel_class == kOpQkv ? kEpiQkvRope : kernel_class == kOpW13 ? kEpiSwiglu : kEpiResid;
    // the class's weight bytes of every layer, streamed by as many
    // workgroups of the same size as its one-token GEMV launches
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    uint64_t nbytes = 0;
    hipError_t e = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(e, "profile_stream capture");
    hipError_t ec = hipSuccess;
    for (int l = 0; l < m->n_layers && ec == hipSuccess; l++) {
        const Layer& L = m->layers[l];
        const QMat& w = kernel_class == kOpQkv ? L.qkv : kernel_class == kOpWo ? L.wo : kernel_class == kOpW13 ? L.w13 : L.w2;
        int grid = 0, threads = 0;
        if (!gemv_launch_shape(w.o, w.nb, epi, w.fmt, &grid, &threads)) { ec = hipErrorInvalidValue; break; }
        const size_t qb = (size_t)w.o * (w.fmt == kQ4 ? w.n / 2 : w.n), db = (size_t)w.o * w.nb * 2;
        nbytes = qb + db;
        ec = launch_stream(w.qs, qb, w.d, db, grid, threads, reinterpret_cast<unsigned*>(s->logits), s->stream);
    }
    e = hipStreamEndCapture(s->stream, &g);
    if (ec != hipSuccess || e != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return hip_fail(ec != hipSuccess ? ec : e, "profile_stream capture");
    }
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "profile_stream instantiate");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    for (int w = 0; w < 2 && e == hipSuccess; w++) e = hipGraphLaunch(ge, s->stream);
    if (e == hipSuccess) e = hipEventRecord(e0, s->stream);
    for (uint32_t r = 0; r < reps && e == hipSuccess; r++) e = hipGraphLaunch(ge, s->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, s->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    hipGraphExecDestroy(ge);
    if (e != hipSuccess) return hip_fail(e, "profile_stream");
    *us_per_launch = (double)ms * 1000.0 / ((double)reps * m->n_layers);
    if (bytes_per_launch) *bytes_per_launch = nbytes;
    return YL_OK;
}

// ------------------------------------------------ tokenizer and sampler

namespace {

// The opening of a conversation as the CLI builds it (main.rs:148-152):
// the system template when the GGUF has no chat template, else the BOS
// token when add_bos_token is set.
bool conversation_prefix(const Tokenizer& t, std::vector<uint32_t>* out, std::string* err) {
    if (!t.has_chat_template()) return t.apply_system_template("", out, err);
    if (t.add_bos_token()) out->push_back(t.bos());
    return true;
}

// One chat turn's generation (main.rs:186-216): prefill the prompt at the
// session's position, then sample, print and feed tokens until EOS, the end
// of the context or max_tokens (0: no limit).
yl_status run_turn(const yl_model* m, yl_session* s, Sampler& smp, const std::vector<uint32_t>& prompt,
                   uint32_t max_tokens, std::string* text, std::vector<uint32_t>* ids) {
    if (prompt.empty()) { set_error("generate: empty prompt"); return YL_ERR_ARG; }
    if ((uint64_t)s->pos + prompt.size() > (uint64_t)m->ctx) {
        set_error("generate: the prompt does not fit the context (" + std::to_string(m->ctx) + " positions)");
        return YL_ERR_RANGE;
    }
    std::vector<float> logits((size_t)m->vocab);
    yl_status st = yl_forward_x(m, prompt.data(), prompt.size(), s->pos, s, logits.data(), nullptr);
    if (st != YL_OK) return st;
    s->pos += (uint32_t)prompt.size();
    uint32_t next = 0;
    if (!smp.sample(logits.data(), &next)) { set_error("sampler: no token above the top-p cutoff"); return YL_ERR_ARG; }
    const uint64_t max_gen = max_tokens ? max_tokens : 0xFFFFFFFFull;
    uint64_t gen = 0;
    while (next != m->eos && s->pos < (uint32_t)m->ctx && gen < max_gen) {
        *text += m->tok->t.decode({next});
        if (ids) ids->push_back(next);
        st = yl_forward_x(m, &next, 1, s->pos, s, logits.data(), nullptr);
        if (st != YL_OK) return st;
        s->pos += 1;
        gen++;
        if (!smp.sample(logits.data(), &next)) { set_error("sampler: no token above the top-p cutoff"); return YL_ERR_ARG; }
    }
    return YL_OK;
}

char* dup_string(const std::string& t) {
    char* r = (char*)malloc(t.size() + 1);
    if (r) memcpy(r, t.c_str(), t.size() + 1);
    return r;
}

}  // namespace

const yl_tokenizer* yl_model_tokenizer(const yl_model* m) { return m ? m->tok.get() : nullptr; }

yl_status yl_generate_text(const yl_model* m, yl_session* s, yl_sampler* smp, const uint32_t* prompt, size_t n_prompt,
                           uint32_t max_tokens, char** text, uint32_t* out_ids, size_t out_cap, size_t* n_generated) {
    if (!m || !s || s->m != m || !smp || !prompt || !text) { set_error("generate_text: null argument"); return YL_ERR_ARG; }
    *text = nullptr;
    std::string out;
    std::vector<uint32_t> ids;
    const yl_status st = run_turn(m, s, sampler_of(smp), std::vector<uint32_t>(prompt, prompt + n_prompt), max_tokens, &out, &ids);
    if (n_generated) *n_generated = ids.size();
    if (out_ids) memcpy(out_ids, ids.data(), std::min(ids.size(), out_cap) * 4);
    if (st != YL_OK) return st;
    *text = dup_string(out);
    return *text ? YL_OK : YL_ERR_NOMEM;
}

// ------------------------------------------------------- product FFI

static std::mutex g_ffi_mu;
static yl_model* g_current = nullptr;
// The conversation infer_ffi continues, as the CLI's loop does over its turns
// (main.rs:161-219: one session and one Sampler(vocab, 0.7, 0.9, 42) for the
// life of the model; the first turn opens with the conversation prefix).
static yl_session* g_chat = nullptr;
static Sampler* g_chat_sampler = nullptr;
static bool g_chat_started = false;
static uint32_t g_infer_max_tokens = 0;

static void chat_close() {
    if (g_chat) yl_session_free(g_chat);
    g_chat = nullptr;
    delete g_chat_sampler;
    g_chat_sampler = nullptr;
    g_chat_started = false;
}

bool load_transformer_ffi(const char* model_path) {
    if (!model_path) return false;
    // lib.rs:141-142: a path that is not UTF-8 becomes "", which has no
    // extension and so is refused
    const std::string p = valid_utf8(model_path) ? std::string(model_path) : std::string();
    bool has_ext = false;
    const std::string ext = path_extension(p, &has_ext);
    if (!has_ext || (ext != "gguf" && ext != "lmrs" && ext != "safetensors")) {
        set_error("Unsupported model extension for path: " + p);
        return false;
    }
    yl_model* m = yl_load(model_path, 0xFFFFFFFFu, -1);
    if (!m) return false;
    std::lock_guard<std::mutex> lk(g_ffi_mu);
    chat_close();
    if (g_current) model_release(g_current);
    g_current = m;
    return true;
}

const yl_model* yl_ffi_model(void) {
    std::lock_guard<std::mutex> lk(g_ffi_mu);
    return g_current;
}

void yl_infer_set_max_tokens(uint32_t max_tokens) {
    std::lock_guard<std::mutex> lk(g_ffi_mu);
    g_infer_max_tokens = max_tokens;
}

void yl_infer_reset(void) {
    std::lock_guard<std::mutex> lk(g_ffi_mu);
    chat_close();
}

char* infer_ffi(const char* prompt) {
    std::lock_guard<std::mutex> lk(g_ffi_mu);
    if (!prompt || !g_current) { set_error("infer_ffi: no prompt or no model loaded"); return nullptr; }
    if (!valid_utf8(prompt)) { set_error("infer_ffi: prompt is not UTF-8"); return nullptr; }
    const std::string user = trim_unicode(prompt);
    if (user.empty()) { set_error("infer_ffi: empty prompt"); return nullptr; }
    if (!g_chat) {
        g_chat = yl_create_session(g_current);
        if (!g_chat) return nullptr;
        g_chat_sampler = new Sampler((size_t)g_current->vocab, 0.7f, 0.9f, 42);
        g_chat_started = false;
    }
    const Tokenizer& t = g_current->tok->t;
    std::vector<uint32_t> ids;
    std::string err;
    if ((!g_chat_started && !conversation_prefix(t, &ids, &err)) || !t.apply_turn_template(user, true, &ids, &err)) {
        set_error("infer_ffi: " + err);
        return nullptr;
    }
    g_chat_started = true;
    std::string out;
    if (run_turn(g_current, g_chat, *g_chat_sampler, ids, g_infer_max_tokens, &out, nullptr) != YL_OK) return nullptr;
    char* r = dup_string(out);
    if (!r) set_error("infer_ffi: out of memory");
    return r;
}

void free_string(char* s) { free(s); }

}  // extern "C"
