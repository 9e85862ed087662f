/*
 * yl_oracle.h -- CPU restatement of yaLLMa3's quantized LLaMA forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP path is compared
 * against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library never links or calls it.
 *
 * Every function restates, from the Rust source read as text, the reference
 * function cited beside it (paths relative to the reference repository).
 * Numerics follow the Rust loops operation by operation: the same products,
 * the same accumulation order, no fused multiply-add (build with
 * -ffp-contract=off), IEEE division and square root.
 *
 * Choices where the reference's bits come from third-party code that cannot
 * be run here (and are therefore pinned only to tolerance, not to the bit):
 *   - wide::f32x8::reduce_add: the SSE2 fallback of wide 0.7.33, i.e.
 *     ((l0+l1)+l2)+l3 + ((l4+l5)+l6)+l7, which is what the reference's own
 *     `cargo build --release` (no target-cpu flag, so no AVX) compiles to.
 *   - f32::exp (softmax) and wide::f32x8::exp (SwiGLU): yo_expf, an exp
 *     evaluated in binary64 (Cody-Waite reduction with the fdlibm ln2 split,
 *     degree-13 Taylor polynomial) and rounded once to binary32, so it is the
 *     correctly rounded expf except with probability ~1e-9 per call.
 *   - cosf/sinf/powf (rope_gguf): the C library's, as the Rust std calls them.
 */
#ifndef YL_ORACLE_H
#define YL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* WeightFormat, weight_type.rs:17-22 */
enum { YO_Q8_0 = 0, YO_Q4_0 = 1, YO_F16 = 2 };

/* ---- scalar building blocks ------------------------------------------- */
float yo_f16_to_f32(uint16_t h);                 /* half::f16::to_f32 */
float yo_expf(float x);                          /* documented exp, see above */
float yo_reduce_add8(const float l[8]);          /* wide f32x8::reduce_add (SSE2) */

/* ---- L1 ops ------------------------------------------------------------ */
/* quantization::quantize, quantization.rs:29-52 (qmax 127) */
void yo_quantize_q8(int8_t *q, float *s, const float *x, size_t n, uint32_t gs);
/* weight_type::q4_0_quantize, weight_type.rs:52-74 (qmax 7, clamp +-7) */
void yo_quantize_q4(int8_t *q, float *s, const float *x, size_t n, uint32_t gs);
/* weight_type::quantize dispatch, weight_type.rs:76-90; F16 copies x */
int yo_quantize(int fmt, int8_t *q, float *s, float *f, const float *x, size_t n, uint32_t gs);

/* weight_type::matmul_q8_slices, weight_type.rs:122-226.
 * out has `batch` rows of `o` columns; x has batch*n int8 values. */
void yo_matmul_q8_slices(float *out, const int8_t *x, const float *x_scale,
                         const int8_t *w, const float *w_scale,
                         size_t n, size_t o, size_t gs, size_t batch);
/* weight_type::matmul_f32, weight_type.rs:228-270 */
void yo_matmul_f32(float *out, const float *x, const float *w, size_t n, size_t o, size_t batch);

/* util::rmsnorm, util.rs:389-426 (add_unit_offset = false) */
void yo_rmsnorm(float *o, const float *x, const float *weight, size_t size, float eps);

typedef struct {
    uint32_t head_size, n_heads, n_kv_heads;
    float rope_theta, freq_scale, ext_factor, attn_factor;
    uint32_t original_ctx_len;
} yo_rope_params;
/* util::rope_gguf, util.rs:653-718 (+ rope_yarn_ramp :720-724) */
void yo_rope_gguf(const yo_rope_params *p, float *sq, float *k, uint32_t pos);
/* util::rope (util.rs:589-635), HF layout with llama3 scaling */
void yo_rope_hf(uint32_t head_size, uint32_t n_heads, uint32_t n_kv_heads, float rope_theta, uint32_t ctx_len,
                float *sq, float *k, uint32_t pos);
/* cos/sin of every pair at `pos`, exactly as rope_gguf derives them */
void yo_rope_cos_sin(const yo_rope_params *p, uint32_t pos, float *cos_out, float *sin_out);

/* forward.rs fused_attention, forward.rs:299-400.
 * scores must hold n_heads*batch*seq_len floats (scratch). */
void yo_fused_attention(float *output, float *scores, const float *sq,
                        const float *key_cache, const float *value_cache,
                        size_t seq_len, size_t batch, size_t n_heads, size_t n_kv_heads,
                        size_t head_size, uint32_t start_pos, size_t kv_dim, float attn_scale);

/* SwiGLU in place on gate, forward.rs:220-237 (one token of hidden_dim) */
void yo_swiglu(float *gate, const float *up, size_t hidden_dim);

/* tied-embedding logits for one token, forward.rs:261-279 */
void yo_logits(float *logits, const float *last, const float *emb, size_t vocab, size_t dim);

/* Sampler::sample_argmax, sampler.rs:67-79 (first index of the maximum) */
uint32_t yo_argmax(const float *p, size_t n);

/* ---- model (GGUF loader + forward) ------------------------------------- */
typedef struct yo_model yo_model;
typedef struct yo_session yo_session;

/* TransformerLlamaGguf::load_model_inner, transformer_llama_gguf.rs:183-655.
 * fmt_override: -1 = none, else YO_Q8_0/YO_Q4_0/YO_F16.  Per-tensor formats
 * are kept as stored (the mixed-format extension); NULL on error. */
yo_model *yo_model_load(const char *path, uint32_t max_ctx_len, int fmt_override);
/* a model from arrays (lm.rs / safetensors loaders restated in oracle/loaders.py) */
yo_model *yo_model_new(const uint32_t shape[8], float eps, float rope_theta, uint32_t gs, int hf_rope,
                       int weight_format, const float *embedding, const float *rms_final);
void yo_model_set_norms(yo_model *m, uint32_t layer, const float *rms_att, const float *rms_ffn);
void yo_model_set_weight(yo_model *m, uint32_t layer, int which, int fmt, const int8_t *q, const float *s,
                         const float *f, size_t n);
void yo_model_free(yo_model *m);
const char *yo_last_error(void);
/* shape query: dim, hidden, n_layers, n_heads, n_kv_heads, head_size, vocab, ctx_len */
void yo_model_shape(const yo_model *m, uint32_t out[8]);
float yo_model_rope_theta(const yo_model *m);
/* dequantized f32 token embedding (vocab*dim), gguf.rs:453-489 */
const float *yo_model_embedding(const yo_model *m);

/* InferenceSession::new / reset, base_transformer.rs:89-104 */
yo_session *yo_session_new(const yo_model *m);
void yo_session_reset(yo_session *s);
void yo_session_free(yo_session *s);
float *yo_session_key_cache(yo_session *s);
float *yo_session_value_cache(yo_session *s);

/* llama_forward_x, forward.rs:120-297: logits (vocab floats) of the last
 * token.  Returns 0 on success. */
int yo_forward_x(const yo_model *m, const uint32_t *tokens, size_t n_tokens,
                 uint32_t start_pos, yo_session *s, float *logits);

/* thread count OpenMP will use for the parallel regions */
int yo_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
