/*
 * yl_oracle.c -- CPU restatement of yaLLMa3's quantized LLaMA forward path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * product library.  Build: oracle/Makefile (-O3 -ffp-contract=off -fopenmp).
 *
 * Each function cites the reference file:line it restates.  Results do not
 * depend on the OpenMP thread count: every output element is produced by
 * one thread in the reference's own operation order, as with Rayon there.
 */
#define _GNU_SOURCE
#include "yl_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static __thread char g_err[512];
static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
const char *yo_last_error(void) { return g_err; }
int yo_num_threads(void) { return omp_get_max_threads(); }

/* ------------------------------------------------------------------------ */
/* scalar building blocks                                                    */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact (half::f16::to_f32). */
float yo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* exp evaluated in binary64 and rounded once to binary32.
 * x*log2(e) -> k (nearest), r = (x - k*ln2_hi) - k*ln2_lo with the fdlibm
 * split of ln2 (e_exp.c), e^r by a degree-13 Taylor polynomial (Horner, one
 * fused multiply-add per degree, like the device's evaluation),
 * then scaled by 2^k.  Stands in for f32::exp (forward.rs:358) and
 * wide::f32x8::exp (forward.rs:230). */
float yo_expf(float xf) {
    if (xf != xf) return xf;
    if (xf > 88.8f) return INFINITY;
    if (xf < -104.0f) return 0.0f;
    const double x = (double)xf;
    const double log2e = 0x1.71547652b82fep+0;
    const double ln2_hi = 0x1.62e42fee00000p-1;
    const double ln2_lo = 0x1.a39ef35793c76p-33;
    double kd = nearbyint(x * log2e);
    double r = (x - kd * ln2_hi) - kd * ln2_lo;
    double p = 0x1.6124613a86d09p-33;          /* 1/13! */
    p = fma(p, r, 0x1.1eed8eff8d898p-29);         /* 1/12! */
    p = fma(p, r, 0x1.ae64567f544e4p-26);         /* 1/11! */
    p = fma(p, r, 0x1.27e4fb7789f5cp-22);         /* 1/10! */
    p = fma(p, r, 0x1.71de3a556c734p-19);         /* 1/9!  */
    p = fma(p, r, 0x1.a01a01a01a01ap-16);         /* 1/8!  */
    p = fma(p, r, 0x1.a01a01a01a01ap-13);         /* 1/7!  */
    p = fma(p, r, 0x1.6c16c16c16c17p-10);         /* 1/6!  */
    p = fma(p, r, 0x1.1111111111111p-7);          /* 1/5!  */
    p = fma(p, r, 0x1.5555555555555p-5);          /* 1/4!  */
    p = fma(p, r, 0x1.5555555555555p-3);          /* 1/3!  */
    p = fma(p, r, 0x1.0000000000000p-1);          /* 1/2!  */
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    return (float)ldexp(p, (int)kd);
}

/* wide::f32x8::reduce_add without AVX: the two f32x4 halves each summed
 * left to right (array iter().sum()), then added. */
float yo_reduce_add8(const float l[8]) {
    float a = ((l[0] + l[1]) + l[2]) + l[3];
    float b = ((l[4] + l[5]) + l[6]) + l[7];
    return a + b;
}

/* Rust `f32::round() as i8`: half away from zero, saturating, NaN -> 0. */
static inline int8_t round_to_i8(float v) {
    if (v != v) return 0;
    float r = roundf(v);
    if (r >= 127.0f) return 127;
    if (r <= -128.0f) return -128;
    return (int8_t)r;
}

/* ------------------------------------------------------------------------ */
/* L1 ops                                                                    */
/* ------------------------------------------------------------------------ */

/* quantization.rs:29-52 */
void yo_quantize_q8(int8_t *q, float *s, const float *x, size_t n, uint32_t gs) {
    uint32_t num_groups = (uint32_t)n / gs;
    for (uint32_t g = 0; g < num_groups; g++) {
        float wmax = 0.0f;
        for (uint32_t i = 0; i < gs; i++) {
            float v = fabsf(x[g * gs + i]);
            if (v > wmax) wmax = v;
        }
        float scale = wmax / 127.0f;
        s[g] = scale;
        for (uint32_t i = 0; i < gs; i++) q[g * gs + i] = round_to_i8(x[g * gs + i] / scale);
    }
}

/* weight_type.rs:52-74 */
void yo_quantize_q4(int8_t *q, float *s, const float *x, size_t n, uint32_t gs) {
    uint32_t num_groups = (uint32_t)n / gs;
    for (uint32_t g = 0; g < num_groups; g++) {
        float wmax = 0.0f;
        for (uint32_t i = 0; i < gs; i++) {
            float v = fabsf(x[g * gs + i]);
            if (v > wmax) wmax = v;
        }
        float scale = wmax / 7.0f;
        s[g] = scale;
        for (uint32_t i = 0; i < gs; i++) {
            int8_t v = round_to_i8(x[g * gs + i] / scale);
            q[g * gs + i] = v < -7 ? -7 : (v > 7 ? 7 : v);
        }
    }
}

/* weight_type.rs:76-90 */
int yo_quantize(int fmt, int8_t *q, float *s, float *f, const float *x, size_t n, uint32_t gs) {
    switch (fmt) {
    case YO_Q8_0: yo_quantize_q8(q, s, x, n, gs); return 0;
    case YO_Q4_0: yo_quantize_q4(q, s, x, n, gs); return 0;
    case YO_F16: memcpy(f, x, n * sizeof(float)); return 0;
    default: set_err("quantize: unknown format %d", fmt); return -1;
    }
}

/* weight_type.rs:122-226.  Columns c < 4*floor(o/4) accumulate into out
 * (`+=`, :190-201) and see only whole 8-element runs of each group
 * (n_simd = remaining/8, :148); tail columns are assigned (:207-224) and see
 * every element.  Per block: acc += ((float)isum * w_scale) * x_scale. */
void yo_matmul_q8_slices(float *out, const int8_t *x, const float *x_scale,
                         const int8_t *w, const float *w_scale,
                         size_t n, size_t o, size_t gs, size_t batch) {
    const size_t chunks = o / 4;
    const size_t handled = chunks * 4;
    for (size_t r = 0; r < batch; r++) {
        const size_t xi = r * n;
        float *row = out + r * o;
#pragma omp parallel for schedule(dynamic, 8)
        for (size_t ch = 0; ch < chunks; ch++) {
            for (size_t cc = 0; cc < 4; cc++) {
                const size_t c = ch * 4 + cc;
                const size_t ni = c * n;
                float acc = row[c];
                for (size_t g0 = 0; g0 < n; g0 += gs) {
                    size_t g1 = g0 + gs < n ? g0 + gs : n;
                    size_t cnt = ((g1 - g0) / 8) * 8;
                    const int8_t *xp = x + xi + g0;
                    const int8_t *wp = w + ni + g0;
                    int32_t isum = 0;
                    for (size_t k = 0; k < cnt; k++) isum += (int32_t)xp[k] * (int32_t)wp[k];
                    float t = (float)isum * w_scale[(ni + g0) / gs];
                    t = t * x_scale[(xi + g0) / gs];
                    acc = acc + t;
                }
                row[c] = acc;
            }
        }
        for (size_t c = handled; c < o; c++) {
            const size_t ni = c * n;
            float sum = 0.0f;
            for (size_t g0 = 0; g0 < n; g0 += gs) {
                size_t g1 = g0 + gs < n ? g0 + gs : n;
                int32_t bsum = 0;
                for (size_t k = g0; k < g1; k++) bsum += (int32_t)x[xi + k] * (int32_t)w[ni + k];
                float t = (float)bsum * w_scale[(ni + g0) / gs];
                t = t * x_scale[(xi + g0) / gs];
                sum = sum + t;
            }
            row[c] = sum;
        }
    }
}

/* weight_type.rs:228-270 (assigns; four scalar column sums in i order) */
void yo_matmul_f32(float *out, const float *x, const float *w, size_t n, size_t o, size_t batch) {
    for (size_t r = 0; r < batch; r++) {
        const float *xr = x + r * n;
#pragma omp parallel for schedule(dynamic, 8)
        for (size_t c = 0; c < o; c++) {
            float sum = 0.0f;
            for (size_t i = 0; i < n; i++) sum = sum + xr[i] * w[c * n + i];
            out[r * o + c] = sum;
        }
    }
}

/* util.rs:389-426.  Lane j of the f32x8 accumulator sums x[8i+j]^2 for
 * i = 0..size/8 in order; elements past 8*floor(size/8) are neither summed
 * nor written. */
void yo_rmsnorm(float *o, const float *x, const float *weight, size_t size, float eps) {
    const size_t n_simd = size / 8;
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t i = 0; i < n_simd; i++)
        for (int j = 0; j < 8; j++) {
            float v = x[i * 8 + j];
            l[j] = l[j] + v * v;
        }
    float ss = yo_reduce_add8(l);
    ss = ss / (float)size;
    ss = ss + eps;
    ss = 1.0f / sqrtf(ss);
    for (size_t i = 0; i < n_simd * 8; i++) o[i] = weight[i] * (ss * x[i]);
}

/* util.rs:720-724.  Rust's f32 max/min return the other operand when one
 * is NaN, which is C's fmaxf/fminf. */
static float rope_yarn_ramp(float low, float high, float i0) {
    const float y = (i0 * 0.5f - low) / fmaxf(high - low, 0.001f);
    return 1.0f - fminf(1.0f, fmaxf(y, 0.0f));
}

/* The per-pair (cos, sin) of util.rs:653-718 at position `pos`. */
void yo_rope_cos_sin(const yo_rope_params *p, uint32_t pos, float *cos_out, float *sin_out) {
    const float beta_fast = 32.0f, beta_slow = 1.0f;
    const float two_pi = 2.0f * 3.14159265358979323846f;
    const size_t n_pairs = p->head_size / 2;
    const float theta_scale = powf(p->rope_theta, -2.0f / (float)p->head_size);
    const float n_ctx_orig = (float)p->original_ctx_len;
    float corr_start = fmaf(logf(n_ctx_orig / (beta_fast * two_pi)), (float)p->head_size, 0.0f) /
                       (2.0f * logf(p->rope_theta));
    corr_start = fmaxf(floorf(corr_start), 0.0f);
    float corr_end = fmaf(logf(n_ctx_orig / (beta_slow * two_pi)), (float)p->head_size, 0.0f) /
                     (2.0f * logf(p->rope_theta));
    float corr_dims_1 = fminf(corr_start, corr_end) + fminf(corr_end, (float)n_pairs) - fmaxf(corr_start, 0.0f);

    float theta = (float)pos;
    for (size_t kp = 0; kp < n_pairs; kp++) {
        const float ff = 1.0f;
        float theta_interp = p->freq_scale * theta / ff;
        float t = theta_interp;
        if (p->ext_factor != 0.0f) {
            float i0 = (float)(kp * 2);
            float ramp_mix = rope_yarn_ramp(corr_start, corr_dims_1, i0) * p->ext_factor;
            t = theta_interp * (1.0f - ramp_mix) + theta / ff * ramp_mix;
        }
        cos_out[kp] = cosf(t) * p->attn_factor;
        sin_out[kp] = sinf(t) * p->attn_factor;
        theta = theta * theta_scale;
    }
}

/* util.rs:653-718: consecutive pairs (2k, 2k+1) of every q and kv head. */
void yo_rope_gguf(const yo_rope_params *p, float *sq, float *k, uint32_t pos) {
    const size_t hs = p->head_size, n_pairs = hs / 2;
    float cs[512], sn[512];
    yo_rope_cos_sin(p, pos, cs, sn);
    for (size_t kp = 0; kp < n_pairs; kp++) {
        const float c = cs[kp], s = sn[kp];
        const size_t col0 = kp * 2;
        for (size_t h = 0; h < p->n_heads; h++) {
            size_t off = h * hs + col0;
            float v0 = sq[off], v1 = sq[off + 1];
            sq[off] = v0 * c - v1 * s;
            sq[off + 1] = v0 * s + v1 * c;
        }
        for (size_t h = 0; h < p->n_kv_heads; h++) {
            size_t off = h * hs + col0;
            float v0 = k[off], v1 = k[off + 1];
            k[off] = v0 * c - v1 * s;
            k[off + 1] = v0 * s + v1 * c;
        }
    }
}

/* forward.rs:299-400 */
/* util::rope (util.rs:589-635): HF layout, element j of a head rotates with
 * element j + head_size/2; llama3 frequency scaling with the model's ctx_len
 * as the original context length. */
void yo_rope_hf(uint32_t head_size, uint32_t n_heads, uint32_t n_kv_heads, float rope_theta, uint32_t ctx_len,
                float *sq, float *k, uint32_t pos) {
    const float rope_factor = 32.0f, low_freq_factor = 1.0f, high_freq_factor = 4.0f;
    const float old_context_len = (float)ctx_len;
    const float low_freq_wavelen = old_context_len / low_freq_factor;
    const float high_freq_wavelen = old_context_len / high_freq_factor;
    const uint32_t half = head_size / 2;
    for (uint32_t j = 0; j < half; j++) {
        const uint32_t head_dim = j * 2;
        float freq = powf(rope_theta, -(float)head_dim / (float)head_size);
        const float wavelen = (2.0f * (float)M_PI) / freq;
        if (wavelen > low_freq_wavelen) {
            freq /= rope_factor;
        } else if (wavelen <= low_freq_wavelen && wavelen >= high_freq_wavelen) {
            const float smooth = (old_context_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
            freq = (1.0f - smooth) * freq / rope_factor + smooth * freq;
        }
        const float val = (float)pos * freq;
        const float fcr = cosf(val), fci = sinf(val);
        for (uint32_t h = 0; h < n_heads; h++) {
            float *v = sq + h * head_size + j;
            const float v0 = v[0], v1 = v[half];
            v[0] = v0 * fcr - v1 * fci;
            v[half] = v0 * fci + v1 * fcr;
        }
        for (uint32_t h = 0; h < n_kv_heads; h++) {
            float *v = k + h * head_size + j;
            const float v0 = v[0], v1 = v[half];
            v[0] = v0 * fcr - v1 * fci;
            v[half] = v0 * fci + v1 * fcr;
        }
    }
}

void yo_fused_attention(float *output, float *scores, const float *sq,
                        const float *key_cache, const float *value_cache,
                        size_t seq_len, size_t batch, size_t n_heads, size_t n_kv_heads,
                        size_t head_size, uint32_t start_pos, size_t kv_dim, float attn_scale) {
    const size_t kv_mul = n_heads / n_kv_heads;
    const size_t rows = n_heads * batch;
    /* score rows, :316-366 */
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t idx = 0; idx < rows; idx++) {
        float *score_row = scores + idx * seq_len;
        const size_t qh = idx / batch, t1 = idx % batch, kvh = qh / kv_mul;
        const size_t abs_pos = (size_t)start_pos + t1;
        const size_t max_t2 = abs_pos < seq_len - 1 ? abs_pos : seq_len - 1;
        const float *q = sq + t1 * (n_heads * head_size) + qh * head_size;
        float max_score = -1e10f;
        const size_t n_simd = head_size / 8;
        for (size_t t2 = 0; t2 <= max_t2; t2++) {
            const float *kk = key_cache + t2 * kv_dim + kvh * head_size;
            float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (size_t s = 0; s < n_simd; s++)
                for (int j = 0; j < 8; j++) l[j] = l[j] + q[s * 8 + j] * kk[s * 8 + j];
            float sum = yo_reduce_add8(l);
            for (size_t d = n_simd * 8; d < head_size; d++) sum = sum + q[d] * kk[d];
            float s_val = sum * attn_scale;
            score_row[t2] = s_val;
            if (s_val > max_score) max_score = s_val;
        }
        for (size_t t2 = max_t2 + 1; t2 < seq_len; t2++) score_row[t2] = -1e10f;
        float sum_exp = 0.0f;
        for (size_t t2 = 0; t2 < seq_len; t2++) {
            float e = yo_expf(score_row[t2] - max_score);
            score_row[t2] = e;
            sum_exp = sum_exp + e;
        }
        float inv_sum = sum_exp > 0.0f ? 1.0f / sum_exp : 0.0f;
        for (size_t t2 = 0; t2 < seq_len; t2++) score_row[t2] = score_row[t2] * inv_sum;
    }
    /* P.V per token, :368-399 */
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t t1 = 0; t1 < batch; t1++) {
        float *out_token = output + t1 * (n_heads * head_size);
        for (size_t qh = 0; qh < n_heads; qh++) {
            const size_t kvh = qh / kv_mul;
            const size_t out_base = qh * head_size;
            const size_t s_base = qh * (batch * seq_len) + t1 * seq_len;
            const size_t n_simd = seq_len / 8;
            for (size_t d = 0; d < head_size; d++) {
                float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (size_t c = 0; c < n_simd; c++) {
                    const size_t t2 = c * 8;
                    for (int j = 0; j < 8; j++)
                        l[j] = l[j] + scores[s_base + t2 + j] *
                                          value_cache[(t2 + j) * kv_dim + kvh * head_size + d];
                }
                float sum = yo_reduce_add8(l);
                for (size_t t2 = n_simd * 8; t2 < seq_len; t2++)
                    sum = sum + scores[s_base + t2] * value_cache[t2 * kv_dim + kvh * head_size + d];
                out_token[out_base + d] = sum;
            }
        }
    }
}

/* forward.rs:220-237: gate = (g / (1 + exp(-g))) * up */
void yo_swiglu(float *gate, const float *up, size_t hidden_dim) {
    for (size_t i = 0; i < hidden_dim; i++) {
        float g = gate[i];
        float silu = g / (1.0f + yo_expf(-g));
        gate[i] = silu * up[i];
    }
}

/* forward.rs:261-279 (serial over the vocabulary, as there) */
void yo_logits(float *logits, const float *last, const float *emb, size_t vocab, size_t dim) {
    const size_t n_simd = dim / 8;
    for (size_t v = 0; v < vocab; v++) {
        const float *e = emb + v * dim;
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (size_t s = 0; s < n_simd; s++)
            for (int j = 0; j < 8; j++) l[j] = l[j] + last[s * 8 + j] * e[s * 8 + j];
        float acc = yo_reduce_add8(l);
        for (size_t d = n_simd * 8; d < dim; d++) acc = acc + last[d] * e[d];
        logits[v] = acc;
    }
}

/* sampler.rs:67-79 */
uint32_t yo_argmax(const float *p, size_t n) {
    uint32_t max_i = 0;
    float max_p = p[0];
    for (size_t i = 1; i < n; i++)
        if (p[i] > max_p) { max_i = (uint32_t)i; max_p = p[i]; }
    return max_i;
}

/* ------------------------------------------------------------------------ */
/* GGUF v3 loader, transformer_llama_gguf.rs:183-655                         */
/* ------------------------------------------------------------------------ */

enum { GG_F32 = 0, GG_F16 = 1, GG_Q4_0 = 2, GG_Q8_0 = 8 };

typedef struct {
    int fmt;          /* YO_Q8_0 / YO_Q4_0 / YO_F16 */
    int8_t *q;        /* quant_vals (nibbles 0..15 for Q4_0) */
    float *s;         /* scale_factor per 32 */
    float *f;         /* F16 variant: widened values */
    size_t n;         /* element count */
} yo_qt;

struct yo_model {
    uint32_t dim, hidden, n_layers, n_heads, n_kv_heads, head_size, vocab, ctx_len;
    float eps, attention_scale;
    yo_rope_params rope;
    int weight_format;
    uint32_t gs;         /* shape.group_size: 32 for GGUF, from the file for lm.rs / safetensors */
    int hf_rope;         /* 1: util::rope (lm.rs, safetensors); 0: rope_gguf */
    float *token_embedding;            /* vocab*dim f32 */
    float *w_rms_final;
    float **w_rms_att, **w_rms_ffn;
    yo_qt *wq, *wk, *wv, *wo, *w1, *w2, *w3;
};

struct yo_session {
    const yo_model *m;
    float *key_cache, *value_cache;
    size_t cache_len;
};

typedef struct { const uint8_t *p; size_t len, off; int bad; } rd_t;
static int rd_need(rd_t *r, size_t k) {
    if (r->bad || r->off + k > r->len) { r->bad = 1; return 0; }
    return 1;
}
static uint64_t rd_u(rd_t *r, int nbytes) {
    if (!rd_need(r, (size_t)nbytes)) return 0;
    uint64_t v = 0;
    for (int i = 0; i < nbytes; i++) v |= (uint64_t)r->p[r->off + i] << (8 * i);
    r->off += (size_t)nbytes;
    return v;
}

typedef struct {
    int type;          /* GGUF value type, -1 = absent */
    uint64_t u;        /* integer payload (unsigned types, bool) */
    int64_t i;         /* signed payload */
    double f;          /* float payload */
    const uint8_t *str; size_t str_len;
    uint64_t arr_len;  /* arrays: element count */
} gv_t;

static const char *K_WANT[] = {
    "general.architecture", "llama.embedding_length", "llama.feed_forward_length",
    "llama.block_count", "llama.attention.head_count", "llama.attention.head_count_kv",
    "llama.attention.layer_norm_rms_epsilon", "general.file_type", "llama.rope.freq_base",
    "llama.context_length", "tokenizer.ggml.tokens", "llama.rope.scaling.factor",
    "llama.rope.scaling.ext_factor", "llama.rope.scaling.attn_factor",
    "llama.rope.scaling.original_context_length", "llama.attention.scale", "general.alignment",
};
enum { KW_ARCH, KW_DIM, KW_FFN, KW_LAYERS, KW_HEADS, KW_KVHEADS, KW_EPS, KW_FTYPE, KW_THETA,
       KW_CTX, KW_TOKENS, KW_RS_FACTOR, KW_RS_EXT, KW_RS_ATTN, KW_RS_ORIG, KW_ATT_SCALE, KW_ALIGN, KW_N };

/* read_gguf_value, transformer_llama_gguf.rs:80-107 */
static int gv_read(rd_t *r, uint32_t type, gv_t *out) {
    gv_t v; memset(&v, 0, sizeof v); v.type = (int)type;
    switch (type) {
    case 0: v.u = rd_u(r, 1); break;
    case 1: v.i = (int8_t)rd_u(r, 1); break;
    case 2: v.u = rd_u(r, 2); break;
    case 3: v.i = (int16_t)rd_u(r, 2); break;
    case 4: v.u = rd_u(r, 4); break;
    case 5: v.i = (int32_t)rd_u(r, 4); break;
    case 6: { uint32_t b = (uint32_t)rd_u(r, 4); float f; memcpy(&f, &b, 4); v.f = f; break; }
    case 7: v.u = rd_u(r, 1) != 0; break;
    case 8: { uint64_t len = rd_u(r, 8); if (!rd_need(r, len)) return -1;
              v.str = r->p + r->off; v.str_len = len; r->off += len; break; }
    case 9: { uint32_t et = (uint32_t)rd_u(r, 4); uint64_t n = rd_u(r, 8); v.arr_len = n;
              for (uint64_t k = 0; k < n && !r->bad; k++) { gv_t tmp; if (gv_read(r, et, &tmp)) return -1; }
              break; }
    case 10: v.u = rd_u(r, 8); break;
    case 11: v.i = (int64_t)rd_u(r, 8); break;
    case 12: { uint64_t b = rd_u(r, 8); double d; memcpy(&d, &b, 8); v.f = d; break; }
    default: set_err("Unknown GGUF metadata value type: %u", type); return -1;
    }
    if (r->bad) { set_err("GGUF truncated"); return -1; }
    if (out) *out = v;
    return 0;
}

/* get_metadata_u64 (:123-129) accepts u64/u32 only */
static int meta_u64(const gv_t *v, uint64_t *o) {
    if (v->type == 10 || v->type == 4) { *o = v->u; return 1; }
    return 0;
}
/* get_metadata_f32 (:131-137) accepts f32/f64 */
static int meta_f32(const gv_t *v, float *o) {
    if (v->type == 6 || v->type == 12) { *o = (float)v->f; return 1; }
    return 0;
}

static void qt_free(yo_qt *t) { free(t->q); free(t->s); free(t->f); memset(t, 0, sizeof *t); }

/* load_q8_0_tensor (:345-373), load_q4_0_tensor (:375-410), load_f16_tensor (:412-421) */
static int load_qt(const uint8_t *base, size_t avail, uint32_t ttype, size_t n, yo_qt *t) {
    memset(t, 0, sizeof *t);
    t->n = n;
    size_t blocks = (n + 31) / 32;
    if (ttype == GG_Q8_0) {
        if (blocks * 34 > avail) { set_err("Q8_0 tensor exceeds file"); return -1; }
        t->fmt = YO_Q8_0;
        t->q = (int8_t *)malloc(n ? n : 1); t->s = (float *)malloc(blocks * 4 + 4);
#pragma omp parallel for schedule(static)
        for (size_t b = 0; b < blocks; b++) {
            const uint8_t *blk = base + b * 34;
            t->s[b] = yo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            for (size_t j = 0; j < 32; j++) if (b * 32 + j < n) t->q[b * 32 + j] = (int8_t)blk[2 + j];
        }
        return 0;
    }
    if (ttype == GG_Q4_0) {
        if (blocks * 18 > avail) { set_err("Q4_0 tensor exceeds file"); return -1; }
        t->fmt = YO_Q4_0;
        t->q = (int8_t *)malloc(n ? n : 1); t->s = (float *)malloc(blocks * 4 + 4);
#pragma omp parallel for schedule(static)
        for (size_t b = 0; b < blocks; b++) {
            const uint8_t *blk = base + b * 18;
            t->s[b] = yo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            for (size_t j = 0; j < 16; j++) {
                uint8_t by = blk[2 + j];
                size_t lo = b * 32 + j * 2, hi = lo + 1;
                if (lo < n) t->q[lo] = (int8_t)(by & 0x0f);
                if (hi < n) t->q[hi] = (int8_t)((by >> 4) & 0x0f);
            }
        }
        return 0;
    }
    if (ttype == GG_F16) {
        if (n * 2 > avail) { set_err("F16 tensor exceeds file"); return -1; }
        t->fmt = YO_F16;
        t->f = (float *)malloc(n * 4 + 4);
        for (size_t i = 0; i < n; i++) t->f[i] = yo_f16_to_f32((uint16_t)(base[2 * i] | (base[2 * i + 1] << 8)));
        return 0;
    }
    set_err("Unsupported tensor type %u -- only Q8_0, Q4_0, and F16 are supported", ttype);
    return -1;
}

typedef struct { const uint8_t *name; size_t name_len; uint32_t type; uint64_t off; size_t n; } tinfo_t;

static const tinfo_t *find_tensor(const tinfo_t *ti, size_t cnt, const char *name) {
    size_t L = strlen(name);
    for (size_t i = 0; i < cnt; i++)
        if (ti[i].name_len == L && memcmp(ti[i].name, name, L) == 0) return &ti[i];
    return NULL;
}

void yo_model_free(yo_model *m) {
    if (!m) return;
    free(m->token_embedding);
    free(m->w_rms_final);
    for (uint32_t l = 0; l < m->n_layers; l++) {
        if (m->w_rms_att) free(m->w_rms_att[l]);
        if (m->w_rms_ffn) free(m->w_rms_ffn[l]);
        yo_qt *all[7] = {m->wq, m->wk, m->wv, m->wo, m->w1, m->w2, m->w3};
        for (int k = 0; k < 7; k++) if (all[k]) qt_free(&all[k][l]);
    }
    free(m->w_rms_att); free(m->w_rms_ffn);
    free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->w1); free(m->w2); free(m->w3);
    free(m);
}

yo_model *yo_model_load(const char *path, uint32_t max_ctx_len, int fmt_override) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) { set_err("cannot open %s", path); return NULL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) { close(fd); set_err("bad file %s", path); return NULL; }
    size_t flen = (size_t)st.st_size;
    const uint8_t *map = (const uint8_t *)mmap(NULL, flen, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) { set_err("mmap failed"); return NULL; }
    yo_model *m = NULL;
    tinfo_t *ti = NULL;
    rd_t r = {map, flen, 0, 0};
    gv_t kv[KW_N];
    for (int i = 0; i < KW_N; i++) kv[i].type = -1;

    if (rd_u(&r, 4) != 0x46554747u) { set_err("Not a GGUF file (bad magic)"); goto fail; }
    uint32_t version = (uint32_t)rd_u(&r, 4);
    if (version != 3) { set_err("Only GGUF version 3 is supported, got version %u", version); goto fail; }
    uint64_t tensor_count = rd_u(&r, 8), kv_count = rd_u(&r, 8);
    for (uint64_t i = 0; i < kv_count; i++) {
        uint64_t klen = rd_u(&r, 8);
        if (!rd_need(&r, klen)) { set_err("GGUF truncated"); goto fail; }
        const uint8_t *key = r.p + r.off; r.off += klen;
        uint32_t vt = (uint32_t)rd_u(&r, 4);
        gv_t v;
        if (gv_read(&r, vt, &v)) goto fail;
        for (int k = 0; k < KW_N; k++)
            if (strlen(K_WANT[k]) == klen && memcmp(K_WANT[k], key, klen) == 0) kv[k] = v;
    }
    if (kv[KW_ARCH].type != 8 || kv[KW_ARCH].str_len != 5 || memcmp(kv[KW_ARCH].str, "llama", 5) != 0) {
        set_err("Architecture must be 'llama'"); goto fail;
    }
    m = (yo_model *)calloc(1, sizeof *m);
    uint64_t u;
    float f;
#define REQ_U(idx, dst) do { if (!meta_u64(&kv[idx], &u)) { set_err("Missing or wrong type for metadata key: %s", K_WANT[idx]); goto fail; } dst = (uint32_t)u; } while (0)
    REQ_U(KW_DIM, m->dim);
    REQ_U(KW_FFN, m->hidden);
    REQ_U(KW_LAYERS, m->n_layers);
    REQ_U(KW_HEADS, m->n_heads);
    m->n_kv_heads = meta_u64(&kv[KW_KVHEADS], &u) ? (uint32_t)u : m->n_heads;
    if (!meta_f32(&kv[KW_EPS], &m->eps)) { set_err("Missing or wrong type for metadata key: %s", K_WANT[KW_EPS]); goto fail; }
    uint64_t file_type = meta_u64(&kv[KW_FTYPE], &u) ? u : 7;
    float rope_theta = meta_f32(&kv[KW_THETA], &f) ? f : 10000.0f;
    uint32_t seq_len;
    REQ_U(KW_CTX, seq_len);
#undef REQ_U
    if (m->n_heads == 0 || m->dim % m->n_heads != 0) { set_err("dim must be divisible by n_heads"); goto fail; }
    m->head_size = m->dim / m->n_heads;
    m->ctx_len = seq_len < max_ctx_len ? seq_len : max_ctx_len;
    if (kv[KW_TOKENS].type != 9) { set_err("tokenizer.ggml.tokens must be an array of strings"); goto fail; }
    m->vocab = (uint32_t)kv[KW_TOKENS].arr_len;
    float raw = meta_f32(&kv[KW_RS_FACTOR], &f) ? f : 1.0f;
    m->rope.freq_scale = raw != 0.0f ? 1.0f / raw : 1.0f;
    m->rope.ext_factor = meta_f32(&kv[KW_RS_EXT], &f) ? f : 0.0f;
    m->rope.attn_factor = meta_f32(&kv[KW_RS_ATTN], &f) ? f : 1.0f;
    m->rope.original_ctx_len = meta_u64(&kv[KW_RS_ORIG], &u) ? (uint32_t)u : seq_len;
    m->attention_scale = meta_f32(&kv[KW_ATT_SCALE], &f) ? f : 0.0f;
    m->rope.rope_theta = rope_theta;
    m->gs = 32;
    m->hf_rope = 0;
    m->rope.head_size = m->head_size;
    m->rope.n_heads = m->n_heads;
    m->rope.n_kv_heads = m->n_kv_heads;
    if (fmt_override >= 0) {
        m->weight_format = fmt_override;
    } else {
        if (file_type == 1) m->weight_format = YO_F16;
        else if (file_type == 2) m->weight_format = YO_Q4_0;
        else if (file_type == 7) m->weight_format = YO_Q8_0;
        else { set_err("Unsupported GGUF file_type: %llu", (unsigned long long)file_type); goto fail; }
    }

    ti = (tinfo_t *)calloc(tensor_count ? tensor_count : 1, sizeof *ti);
    for (uint64_t i = 0; i < tensor_count; i++) {
        uint64_t nl = rd_u(&r, 8);
        if (!rd_need(&r, nl)) { set_err("GGUF truncated"); goto fail; }
        ti[i].name = r.p + r.off; ti[i].name_len = nl; r.off += nl;
        uint32_t nd = (uint32_t)rd_u(&r, 4);
        size_t ne = 1;
        for (uint32_t d = 0; d < nd; d++) ne *= (size_t)rd_u(&r, 8);
        ti[i].n = ne;
        ti[i].type = (uint32_t)rd_u(&r, 4);
        ti[i].off = rd_u(&r, 8);
        if (r.bad) { set_err("GGUF truncated"); goto fail; }
    }
    uint64_t alignment = meta_u64(&kv[KW_ALIGN], &u) ? u : 32;
    if (alignment == 0 || (alignment & (alignment - 1))) { set_err("GGUF alignment must be a power of 2"); goto fail; }
    const uint64_t data_start = (r.off + alignment - 1) / alignment * alignment;

#define TENSOR(name_, out_) do { \
        out_ = find_tensor(ti, tensor_count, name_); \
        if (!out_) { set_err("Missing tensor: %s", name_); goto fail; } \
        if (data_start + out_->off > flen) { set_err("tensor %s beyond file", name_); goto fail; } \
    } while (0)
    const tinfo_t *t;
    /* token embedding: load quantized, dequantize to f32 (:453-489) */
    TENSOR("token_embd.weight", t);
    {
        yo_qt e;
        if (load_qt(map + data_start + t->off, flen - (data_start + t->off), t->type, t->n, &e)) goto fail;
        m->token_embedding = (float *)malloc(t->n * sizeof(float) + 4);
        if (e.fmt == YO_F16) {
            memcpy(m->token_embedding, e.f, t->n * sizeof(float));
        } else {
            const size_t groups = (t->n + 31) / 32;
#pragma omp parallel for schedule(static)
            for (size_t g = 0; g < groups; g++)
                for (size_t j = 0; j < 32 && g * 32 + j < t->n; j++)
                    m->token_embedding[g * 32 + j] = (float)e.q[g * 32 + j] * e.s[g];
        }
        qt_free(&e);
        if (t->n < (size_t)m->vocab * m->dim) { set_err("token_embd.weight smaller than vocab*dim"); goto fail; }
    }
    /* F32 norms (:334-343, :491-519) */
    TENSOR("output_norm.weight", t);
    if (t->type != GG_F32) { set_err("Expected F32 tensor"); goto fail; }
    m->w_rms_final = (float *)malloc(t->n * 4 + 4);
    memcpy(m->w_rms_final, map + data_start + t->off, t->n * 4);
    const uint32_t L = m->n_layers;
    m->w_rms_att = (float **)calloc(L, sizeof(float *));
    m->w_rms_ffn = (float **)calloc(L, sizeof(float *));
    m->wq = (yo_qt *)calloc(L, sizeof(yo_qt)); m->wk = (yo_qt *)calloc(L, sizeof(yo_qt));
    m->wv = (yo_qt *)calloc(L, sizeof(yo_qt)); m->wo = (yo_qt *)calloc(L, sizeof(yo_qt));
    m->w1 = (yo_qt *)calloc(L, sizeof(yo_qt)); m->w2 = (yo_qt *)calloc(L, sizeof(yo_qt));
    m->w3 = (yo_qt *)calloc(L, sizeof(yo_qt));
    char name[128];
    for (uint32_t l = 0; l < L; l++) {
        snprintf(name, sizeof name, "blk.%u.attn_norm.weight", l); TENSOR(name, t);
        if (t->type != GG_F32) { set_err("Expected F32 tensor"); goto fail; }
        m->w_rms_att[l] = (float *)malloc(t->n * 4 + 4); memcpy(m->w_rms_att[l], map + data_start + t->off, t->n * 4);
        snprintf(name, sizeof name, "blk.%u.ffn_norm.weight", l); TENSOR(name, t);
        if (t->type != GG_F32) { set_err("Expected F32 tensor"); goto fail; }
        m->w_rms_ffn[l] = (float *)malloc(t->n * 4 + 4); memcpy(m->w_rms_ffn[l], map + data_start + t->off, t->n * 4);
        const char *proj[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_down", "ffn_up"};
        yo_qt *dst[7] = {&m->wq[l], &m->wk[l], &m->wv[l], &m->wo[l], &m->w1[l], &m->w2[l], &m->w3[l]};
        for (int k = 0; k < 7; k++) {
            snprintf(name, sizeof name, "blk.%u.%s.weight", l, proj[k]); TENSOR(name, t);
            if (load_qt(map + data_start + t->off, flen - (data_start + t->off), t->type, t->n, dst[k])) goto fail;
        }
    }
#undef TENSOR
    free(ti);
    munmap((void *)map, flen);
    return m;
fail:
    free(ti);
    yo_model_free(m);
    munmap((void *)map, flen);
    return NULL;
}

/* A model built from arrays: the lm.rs and safetensors loaders are restated
 * in Python (oracle/loaders.py), which hands the weights over here.
 * shape: dim, hidden, n_layers, n_heads, n_kv_heads, head_size, vocab, ctx_len. */
yo_model *yo_model_new(const uint32_t shape[8], float eps, float rope_theta, uint32_t gs, int hf_rope,
                       int weight_format, const float *embedding, const float *rms_final) {
    yo_model *m = (yo_model *)calloc(1, sizeof *m);
    m->dim = shape[0]; m->hidden = shape[1]; m->n_layers = shape[2]; m->n_heads = shape[3];
    m->n_kv_heads = shape[4]; m->head_size = shape[5]; m->vocab = shape[6]; m->ctx_len = shape[7];
    m->eps = eps;
    m->attention_scale = 0.0f;
    memset(&m->rope, 0, sizeof m->rope);
    m->rope.rope_theta = rope_theta;
    m->rope.head_size = m->head_size;
    m->rope.n_heads = m->n_heads;
    m->rope.n_kv_heads = m->n_kv_heads;
    m->rope.freq_scale = 1.0f;
    m->rope.attn_factor = 1.0f;
    m->rope.original_ctx_len = m->ctx_len;
    m->gs = gs;
    m->hf_rope = hf_rope;
    m->weight_format = weight_format;
    const size_t ne = (size_t)m->vocab * m->dim, L = m->n_layers;
    m->token_embedding = (float *)malloc(ne * sizeof(float) + 4);
    memcpy(m->token_embedding, embedding, ne * sizeof(float));
    m->w_rms_final = (float *)malloc(m->dim * sizeof(float) + 4);
    memcpy(m->w_rms_final, rms_final, m->dim * sizeof(float));
    m->w_rms_att = (float **)calloc(L, sizeof(float *));
    m->w_rms_ffn = (float **)calloc(L, sizeof(float *));
    m->wq = (yo_qt *)calloc(L, sizeof(yo_qt)); m->wk = (yo_qt *)calloc(L, sizeof(yo_qt));
    m->wv = (yo_qt *)calloc(L, sizeof(yo_qt)); m->wo = (yo_qt *)calloc(L, sizeof(yo_qt));
    m->w1 = (yo_qt *)calloc(L, sizeof(yo_qt)); m->w2 = (yo_qt *)calloc(L, sizeof(yo_qt));
    m->w3 = (yo_qt *)calloc(L, sizeof(yo_qt));
    return m;
}

void yo_model_set_norms(yo_model *m, uint32_t layer, const float *rms_att, const float *rms_ffn) {
    m->w_rms_att[layer] = (float *)malloc(m->dim * sizeof(float) + 4);
    m->w_rms_ffn[layer] = (float *)malloc(m->dim * sizeof(float) + 4);
    memcpy(m->w_rms_att[layer], rms_att, m->dim * sizeof(float));
    memcpy(m->w_rms_ffn[layer], rms_ffn, m->dim * sizeof(float));
}

/* which: 0 q, 1 k, 2 v, 3 o, 4 gate (w1), 5 down (w2), 6 up (w3); Q8_0 values q
 * with f32 scales s (n / gs of them), or F16 values f as f32 */
void yo_model_set_weight(yo_model *m, uint32_t layer, int which, int fmt, const int8_t *q, const float *s,
                         const float *f, size_t n) {
    yo_qt *all[7] = {m->wq, m->wk, m->wv, m->wo, m->w1, m->w2, m->w3};
    yo_qt *t = &all[which][layer];
    memset(t, 0, sizeof *t);
    t->fmt = fmt;
    t->n = n;
    if (fmt == YO_F16) {
        t->f = (float *)malloc(n * sizeof(float) + 4);
        memcpy(t->f, f, n * sizeof(float));
    } else {
        t->q = (int8_t *)malloc(n + 4);
        t->s = (float *)malloc(n / m->gs * sizeof(float) + 4);
        memcpy(t->q, q, n);
        memcpy(t->s, s, n / m->gs * sizeof(float));
    }
}

void yo_model_shape(const yo_model *m, uint32_t out[8]) {
    out[0] = m->dim; out[1] = m->hidden; out[2] = m->n_layers; out[3] = m->n_heads;
    out[4] = m->n_kv_heads; out[5] = m->head_size; out[6] = m->vocab; out[7] = m->ctx_len;
}
float yo_model_rope_theta(const yo_model *m) { return m->rope.rope_theta; }
const float *yo_model_embedding(const yo_model *m) { return m->token_embedding; }

/* base_transformer.rs:89-98 */
yo_session *yo_session_new(const yo_model *m) {
    yo_session *s = (yo_session *)calloc(1, sizeof *s);
    s->m = m;
    s->cache_len = (size_t)m->n_layers * m->ctx_len * (m->n_kv_heads * m->head_size);
    s->key_cache = (float *)calloc(s->cache_len ? s->cache_len : 1, sizeof(float));
    s->value_cache = (float *)calloc(s->cache_len ? s->cache_len : 1, sizeof(float));
    if (!s->key_cache || !s->value_cache) { yo_session_free(s); set_err("out of memory"); return NULL; }
    return s;
}
void yo_session_reset(yo_session *s) {
    memset(s->key_cache, 0, s->cache_len * sizeof(float));
    memset(s->value_cache, 0, s->cache_len * sizeof(float));
}
void yo_session_free(yo_session *s) {
    if (!s) return;
    free(s->key_cache); free(s->value_cache); free(s);
}
float *yo_session_key_cache(yo_session *s) { return s->key_cache; }
float *yo_session_value_cache(yo_session *s) { return s->value_cache; }

/* workspace for one activation quantization in a weight's format */
typedef struct { int8_t *q; float *s; float *f; } xq_t;

static void quant_for(const yo_qt *w, xq_t *xq, const float *x, size_t n, uint32_t gs) {
    yo_quantize(w->fmt, xq->q, xq->s, xq->f, x, n, gs);
}

/* ForwardKernel::matmul for the weight's format (forward.rs:39-43,61-65,83-87) */
static void matmul_for(float *out, const xq_t *xq, const yo_qt *w, size_t n, size_t o, size_t batch, uint32_t gs) {
    if (w->fmt == YO_F16) yo_matmul_f32(out, xq->f, w->f, n, o, batch);
    else yo_matmul_q8_slices(out, xq->q, xq->s, w->q, w->s, n, o, gs, batch);
}

/* forward.rs:120-280 */
int yo_forward_x(const yo_model *m, const uint32_t *tokens, size_t n_tokens,
                 uint32_t start_pos, yo_session *s, float *logits) {
    const size_t batch = n_tokens;
    if (batch == 0) { set_err("empty token batch"); return -1; }
    const size_t dim = m->dim, hidden = m->hidden;
    const size_t att_dim = (size_t)m->n_heads * m->head_size;
    const size_t kv_dim = (size_t)m->n_kv_heads * m->head_size;
    const size_t seq_len = (size_t)start_pos + batch;
    if (seq_len > m->ctx_len) { set_err("position beyond ctx_len"); return -1; }
    const size_t gs = m->gs;

    /* embeddings (base_transformer.rs:143-161): out-of-range ids -> zeros */
    float *x = (float *)calloc(batch * dim, sizeof(float));
    float *xn = (float *)calloc(batch * dim, sizeof(float));
    size_t max_q = batch * dim;
    if (batch * att_dim > max_q) max_q = batch * att_dim;
    if (batch * hidden > max_q) max_q = batch * hidden;
    xq_t xq = {(int8_t *)calloc(max_q, 1), (float *)calloc(max_q / gs + 1, sizeof(float)),
               (float *)calloc(max_q, sizeof(float))};
    float *sq = (float *)calloc(batch * att_dim, sizeof(float));
    float *scores = (float *)calloc((size_t)m->n_heads * batch * seq_len, sizeof(float));
    float *att = (float *)calloc(batch * att_dim, sizeof(float));
    float *hg = (float *)calloc(batch * hidden, sizeof(float));
    float *hu = (float *)calloc(batch * hidden, sizeof(float));
    float *ffn = (float *)calloc(batch * dim, sizeof(float));
    for (size_t t = 0; t < batch; t++) {
        size_t idx = (size_t)tokens[t] * dim;
        if (idx + dim <= (size_t)m->vocab * dim) memcpy(x + t * dim, m->token_embedding + idx, dim * sizeof(float));
    }
    const float attn_scale = m->attention_scale != 0.0f ? m->attention_scale : 1.0f / sqrtf((float)m->head_size);
    const size_t total = batch * dim;

    for (uint32_t layer = 0; layer < m->n_layers; layer++) {
        const size_t cache_off = (size_t)layer * m->ctx_len * kv_dim;
        const size_t write_off = (size_t)start_pos * kv_dim;
        for (size_t t = 0; t < batch; t++) yo_rmsnorm(xn + t * dim, x + t * dim, m->w_rms_att[layer], dim, m->eps);
        quant_for(&m->wq[layer], &xq, xn, batch * dim, m->gs);
        memset(sq, 0, batch * att_dim * sizeof(float));
        matmul_for(sq, &xq, &m->wq[layer], dim, att_dim, batch, m->gs);
        float *k = s->key_cache + cache_off + write_off;
        float *v = s->value_cache + cache_off + write_off;
        matmul_for(k, &xq, &m->wk[layer], dim, kv_dim, batch, m->gs);
        matmul_for(v, &xq, &m->wv[layer], dim, kv_dim, batch, m->gs);
        for (size_t t = 0; t < batch; t++) {
            if (m->hf_rope)
                yo_rope_hf(m->head_size, m->n_heads, m->n_kv_heads, m->rope.rope_theta, m->ctx_len, sq + t * att_dim,
                           k + t * kv_dim, start_pos + (uint32_t)t);
            else
                yo_rope_gguf(&m->rope, sq + t * att_dim, k + t * kv_dim, start_pos + (uint32_t)t);
        }
        yo_fused_attention(att, scores, sq, s->key_cache + cache_off, s->value_cache + cache_off,
                           seq_len, batch, m->n_heads, m->n_kv_heads, m->head_size, start_pos, kv_dim, attn_scale);
        quant_for(&m->wo[layer], &xq, att, batch * att_dim, m->gs);
        memset(ffn, 0, batch * dim * sizeof(float));
        matmul_for(ffn, &xq, &m->wo[layer], att_dim, dim, batch, m->gs);
        for (size_t i = 0; i < total; i++) x[i] = x[i] + ffn[i];          /* :196-204 */
        for (size_t t = 0; t < batch; t++) yo_rmsnorm(xn + t * dim, x + t * dim, m->w_rms_ffn[layer], dim, m->eps);
        quant_for(&m->w1[layer], &xq, xn, batch * dim, m->gs);
        memset(hg, 0, batch * hidden * sizeof(float));
        memset(hu, 0, batch * hidden * sizeof(float));
        matmul_for(hg, &xq, &m->w1[layer], dim, hidden, batch, m->gs);
        matmul_for(hu, &xq, &m->w3[layer], dim, hidden, batch, m->gs);
#pragma omp parallel for schedule(static)
        for (size_t t = 0; t < batch; t++) yo_swiglu(hg + t * hidden, hu + t * hidden, hidden);
        quant_for(&m->w2[layer], &xq, hg, batch * hidden, m->gs);
        memset(ffn, 0, batch * dim * sizeof(float));
        matmul_for(ffn, &xq, &m->w2[layer], hidden, dim, batch, m->gs);
        for (size_t i = 0; i < total; i++) x[i] = x[i] + ffn[i];          /* :245-253 */
    }
    for (size_t t = 0; t < batch; t++) yo_rmsnorm(xn + t * dim, x + t * dim, m->w_rms_final, dim, m->eps);
    if (logits) yo_logits(logits, xn + (batch - 1) * dim, m->token_embedding, m->vocab, dim);

    free(x); free(xn); free(xq.q); free(xq.s); free(xq.f); free(sq); free(scores); free(att);
    free(hg); free(hu); free(ffn);
    return 0;
}
