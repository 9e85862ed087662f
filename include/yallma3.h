/*
 * yallma3.h -- C ABI of the MI355X-native quantized LLaMA forward path.
 *
 * Library: libyallma3_amd.so (HIP for gfx950 + C++ host).  Every entry
 * point is `extern "C"`, takes plain pointers and sizes, and reports errors
 * through a status code plus yl_last_error() instead of panicking.
 *
 * Reference interfaces replaced (paths relative to the reference repo):
 *   load_transformer_ffi   src_llm/lib.rs:135-152
 *   infer_ffi, free_string README.md:81-92, PoC_Bun_load.js:12-38 (documented,
 *                          not implemented by the reference)
 *   yl_load                lib.rs:107-133 load_transformer: ".gguf" ->
 *                          transformer_llama_gguf.rs:179-655; ".lmrs" ->
 *                          transformer_llama_lmrs.rs:60-434; ".safetensors" ->
 *                          transformer_llama_st.rs:36-300
 *   yl_forward_x           Transformer::forward_x, transformer.rs:53 ->
 *                          forward.rs:282-297 llama_forward_x
 *   yl_create_session      Transformer::create_session, transformer.rs:56;
 *                          InferenceSession::new, base_transformer.rs:89-98
 *   yl_session_reset       InferenceSession::reset, base_transformer.rs:100-104
 *   yl_get_embeddings      Transformer::get_embeddings_batch, transformer.rs:42;
 *                          base_transformer.rs:143-161
 *   yl_quantize            weight_type::quantize, weight_type.rs:76-90
 *                          (quantization.rs:29-52 / weight_type.rs:52-74)
 *   yl_matmul              weight_type::matmul, weight_type.rs:92-106 ->
 *                          matmul_q8_slices, weight_type.rs:122-226
 *   yl_rmsnorm_quantize    util::rmsnorm, util.rs:389-426 (+ quantize)
 *   yl_rope_gguf           util::rope_gguf, util.rs:653-718
 *   yl_attention           forward.rs fused_attention, forward.rs:299-400
 *   yl_swiglu_quantize     forward.rs:220-237 (+ quantize)
 *   (greedy argmax, Sampler::sample_argmax sampler.rs:67-79, is the
 *    `argmax` output of yl_forward_x and the chaining of yl_generate_greedy)
 *
 * Memory: functions documented "device" take pointers from yl_malloc (or
 * any HIP device allocation on the current device); "host" pointers are
 * ordinary process memory.  `stream` is a hipStream_t or NULL (the null
 * stream).  Not thread-safe per model/session; distinct models may be used
 * from distinct threads.
 */
#ifndef YALLMA3_H
#define YALLMA3_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
typedef int32_t yl_status;
#define YL_OK               0
#define YL_ERR_ARG         -1  /* bad argument / shape */
#define YL_ERR_FORMAT      -2  /* format/variant mismatch (weight_type.rs:88,104) */
#define YL_ERR_IO          -3  /* file cannot be opened or read */
#define YL_ERR_GGUF        -4  /* malformed or unsupported GGUF (gguf.rs:189-267 asserts) */
#define YL_ERR_HIP         -5  /* HIP runtime error / no GPU */
#define YL_ERR_UNSUPPORTED -6  /* valid for the reference, not built here (see yl_last_error) */
#define YL_ERR_NOMEM       -7
#define YL_ERR_RANGE       -8  /* position beyond ctx_len */

/* Message of the last failure on this thread ("" if none). */
const char *yl_last_error(void);

/* WeightFormat, weight_type.rs:17-22 */
typedef enum { YL_Q8_0 = 0, YL_Q4_0 = 1, YL_F16 = 2 } yl_format;

/* Model and session handles (defined by the library). */
typedef struct yl_model yl_model;
typedef struct yl_session yl_session;

/* ------------------------------------------------ product ABI (unchanged) */
/* lib.rs:135-152: loads a model into the process-wide current transformer,
 * replacing the previous one; the loader is chosen by the path's extension
 * as load_transformer does (lib.rs:107-133): ".gguf", ".lmrs" or
 * ".safetensors".  false on NULL, a path that is not UTF-8 (the reference
 * maps it to ""), no or another extension, or any load error. */
bool load_transformer_ffi(const char *model_path);
/* README.md:81-92 (documented by the reference, which leaves it
 * unimplemented): one chat turn with the current model, as the reference's
 * CLI runs a turn (main.rs:161-219).  The prompt (UTF-8) is trimmed and
 * wrapped by the GGUF's chat template (tokenizer.rs:496-543; the first turn
 * of a conversation opens with the system template, or the BOS token when a
 * chat template exists), prefilled, and tokens are sampled with
 * Sampler(vocab, temperature 0.7, top-p 0.9, seed 42) (sampler.rs) until
 * EOS, the end of the context or the yl_infer_set_max_tokens limit.  The
 * conversation continues across calls in one KV cache, as the CLI's does;
 * yl_infer_reset() starts a new one.  Returns the decoded pieces as a
 * library-owned NUL-terminated string (release with free_string), or NULL on
 * error (no model, empty or non-UTF-8 prompt, template error, context full). */
char *infer_ffi(const char *prompt);
/* Releases a string returned by infer_ffi or yl_generate_text; NULL is ignored. */
void free_string(char *s);
/* Limit of generated tokens per infer_ffi call (0, the default: none, as the
 * CLI's --max-tokens 0, main.rs:131-136). */
void yl_infer_set_max_tokens(uint32_t max_tokens);
/* Ends infer_ffi's conversation: the next call starts a fresh KV cache and
 * sampler.  Loading a model through load_transformer_ffi does the same. */
void yl_infer_reset(void);
/* The model load_transformer_ffi installed (the reference's `static mut`
 * current transformer, lib.rs:135-152), or NULL before the first successful
 * load; owned by the library and freed by the next successful load.  Lets a
 * host that loads through the product ABI reach the model API above. */
const yl_model *yl_ffi_model(void);

/* ------------------------------------------------------- device helpers */
yl_status yl_device_count(int *count);
void *yl_malloc(size_t bytes);                      /* device memory, 256-B aligned */
void yl_free(void *p);
yl_status yl_memcpy_h2d(void *dst_dev, const void *src_host, size_t bytes);
yl_status yl_memcpy_d2h(void *dst_host, const void *src_dev, size_t bytes);
yl_status yl_memcpy_d2d(void *dst_dev, const void *src_dev, size_t bytes);
yl_status yl_memset_d(void *dst_dev, int value, size_t bytes);
yl_status yl_synchronize(void);

/* -------------------------------------------------------------- L1 ops */
/* quantization::quantize (Q8_0) / weight_type::q4_0_quantize (Q4_0) of n
 * device floats in groups of gs (gs must be 32; n a multiple of 32).
 * q: n int8 (device), scale: n/32 f32 (device). */
yl_status yl_quantize(yl_format fmt, int8_t *q, float *scale, const float *x, size_t n,
                      uint32_t gs, void *stream);

/* A quantized weight matrix [o][n] resident on the device
 * (QuantizedTensor::{Q8,Q4_0}, weight_type.rs:30-50). */
typedef struct yl_weight yl_weight;
/* From the reference's in-memory form (host): quant_vals o*n int8 (Q4_0:
 * unsigned nibble values 0..15 per element, as load_q4_0_tensor produces,
 * transformer_llama_gguf.rs:394-405) and scale_factor o*n/32 f32.  Scales
 * must be exactly representable in binary16 (every GGUF scale is). */
yl_weight *yl_weight_upload(yl_format fmt, const int8_t *quant_vals, const float *scale_factor,
                            size_t o, size_t n);
/* From raw GGUF blocks (host): Q8_0 34-byte / Q4_0 18-byte blocks of a
 * row-major [o][n] tensor (transformer_llama_gguf.rs:345-410). */
yl_weight *yl_weight_upload_gguf(yl_format fmt, const void *blocks, size_t o, size_t n);
/* An F16 matrix (QuantizedTensor::F16) from binary16 bits [o][n] (host); the
 * values are exactly the reference's widened f32 weights. */
yl_weight *yl_weight_upload_f16(const uint16_t *bits, size_t o, size_t n);
void yl_weight_free(yl_weight *w);
/* Bytes the matrix occupies on the device (quantized values + f16 scales). */
size_t yl_weight_bytes(const yl_weight *w);

/* weight_type::matmul for quantized formats.  x: batch*n int8 + batch*n/32
 * f32 scales (device), out: batch*o f32 (device).  Columns c < 4*floor(o/4)
 * accumulate into out (`+=`, weight_type.rs:190-201), the rest are assigned
 * (:207-224); each column sums its block terms ((float)isum*w_scale)*x_scale
 * in block order.  gs must be 32.  YL_ERR_FORMAT if fmt differs from w's. */
yl_status yl_matmul(float *out, yl_format fmt, const int8_t *xq, const float *xs, size_t batch,
                    const yl_weight *w, size_t n, size_t o, uint32_t gs, void *stream);
/* weight_type::matmul's F16 branch, matmul_f32 (weight_type.rs:228-270):
 * out[r][c] = sum over i in order of x[r][i] * w[c][i] (f32 products and adds,
 * one accumulator per column), assigned for every column.  out: batch*o f32,
 * x: batch*n f32 (device); w: an F16 matrix. */
yl_status yl_matmul_f32(float *out, const float *x, size_t batch, const yl_weight *w, size_t n, size_t o,
                        void *stream);

/* Timing of yl_matmul (`=` into out, no accumulation): the count weights
 * (same format and shape, device-resident) are multiplied by the same
 * activations one after another in a HIP graph, the graph is replayed `reps`
 * times between two HIP events, and the elapsed time is divided by the
 * launches.  Rotating through distinct weight copies larger in total than
 * the 256 MiB MALL measures HBM, not cache.  xq/xs/out: device. */
yl_status yl_matmul_bench(const yl_weight *const *ws, size_t count, const int8_t *xq, const float *xs,
                          size_t batch, float *out, uint32_t reps, double *us_per_launch);

/* util::rmsnorm per row (batch rows of size floats, device), optionally
 * followed by quantization of the normalized row.  qfmt: YL_Q8_0 / YL_Q4_0
 * to quantize into q/scale, or -1 for none.  xn (nullable) receives the f32
 * normalized rows. */
yl_status yl_rmsnorm_quantize(const float *x, const float *weight, size_t size, float eps,
                              size_t batch, float *xn, int32_t qfmt, int8_t *q, float *scale,
                              void *stream);

/* RoPE parameters (TransformerShape fields read by rope_gguf). */
typedef struct {
    uint32_t head_size, n_heads, n_kv_heads;
    float rope_theta, freq_scale, ext_factor, attn_factor;
    uint32_t original_ctx_len;
} yl_rope_params;

/* util::rope_gguf in place on q [batch][n_heads*head_size] and k
 * [batch][n_kv_heads*head_size] (device) at positions start_pos+t. */
yl_status yl_rope_gguf(const yl_rope_params *p, float *q, float *k, size_t batch,
                       uint32_t start_pos, void *stream);

/* fused_attention over a cache [seq][kv_dim] (device): out [batch][n_heads*
 * head_size] f32 for query rows q [batch][n_heads*head_size], positions
 * start_pos..start_pos+batch-1, seq_len = start_pos+batch. */
yl_status yl_attention(float *out, const float *q, const float *key_cache, const float *value_cache,
                       size_t batch, uint32_t start_pos, uint32_t n_heads, uint32_t n_kv_heads,
                       uint32_t head_size, float attn_scale, void *stream);

/* The split decode attention of YL_ATTN_SPLIT as an op (no counterpart in
 * the reference: fused_attention's quantity with the context split over many
 * workgroups, equal to it up to rounding): one query row q [n_heads*head_size]
 * at position start_pos over a cache [start_pos+1][kv_dim] (device), out
 * [n_heads*head_size] f32.  Head size 64 or 128 with 1, 2, 4 or 8 query heads
 * per kv head. */
yl_status yl_attention_split(float *out, const float *q, const float *key_cache, const float *value_cache,
                             uint32_t start_pos, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_size,
                             float attn_scale, void *stream);

/* yl_attention without any allocation: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as yl_attention, but the step state, the transposed keys and the
 * scores scratch live in a 64 MiB array the library holds per GPU for the
 * life of the process; calls that would need more (keys of seq_len *
 * n_kv_heads * head_size floats plus the scores) return YL_ERR_RANGE.  The
 * work is enqueued on `stream` and not waited for: synchronize before
 * reading `out`.  Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (different streams or threads) race. */
yl_status yl_attention_noalloc(float *out, const float *q, const float *key_cache, const float *value_cache,
                               size_t batch, uint32_t start_pos, uint32_t n_heads, uint32_t n_kv_heads,
                               uint32_t head_size, float attn_scale, void *stream);

/* SwiGLU (forward.rs:220-237) of gate/up [batch][hidden] (device) into h
 * (nullable, f32), optionally quantized (qfmt -1 = none). */
yl_status yl_swiglu_quantize(const float *gate, const float *up, size_t hidden, size_t batch,
                             float *h, int32_t qfmt, int8_t *q, float *scale, void *stream);

/* --------------------------------------------------- model and session */

typedef struct {                 /* TransformerShape, base_transformer.rs:25-44 */
    uint32_t dimension, hidden_dimension, n_heads, head_size, n_kv_heads, vocab_size;
    uint32_t n_layers, ctx_len;
    float rms_norm_eps, rope_theta;
    uint32_t group_size;
    float rope_freq_scale, rope_ext_factor, rope_attn_factor;
    uint32_t rope_original_ctx_len;
    float attention_scale;
    int32_t weight_format;       /* yl_format the file declares (general.file_type) */
} yl_shape;

/* Load a model onto the current device; the extension picks the loader.
 *   .gguf: GGUF v3 llama.  max_ctx_len caps llama.context_length
 *     (gguf.rs:233); fmt_override -1 = none.  Tensors keep their own stored
 *     format (a Q4_0 FFN beside Q8_0 attention works).
 *   .lmrs: the lm.rs format (Q8 with f32 group scales, the file's group
 *     size; tokenizer.bin beside it), HF-layout RoPE (util.rs:589-635).
 *   .safetensors: config.json + tokenizer.json (or tokenizer.bin) beside it;
 *     F16 weights, or MLX 8-bit affine groups requantized symmetric on load
 *     (util.rs:452-503); HF-layout RoPE.  Q4_0 here is refused (the
 *     reference loads such tensors as Q8 and runs its Q4_0 kernel on them). */
yl_model *yl_load(const char *path, uint32_t max_ctx_len, int32_t fmt_override);
void yl_model_free(yl_model *m);
const char *yl_model_name(const yl_model *m);
yl_status yl_model_shape(const yl_model *m, yl_shape *out);
size_t yl_vocab_size(const yl_model *m);
uint32_t yl_max_ctx_len(const yl_model *m);
uint32_t yl_bos_token(const yl_model *m);
uint32_t yl_eos_token(const yl_model *m);
/* Bytes of quantized layer weights read per decoded token (all seven
 * projections of every layer) and of the logits embedding pass. */
size_t yl_model_weight_bytes(const yl_model *m);
size_t yl_model_embedding_bytes(const yl_model *m);

/* get_embeddings_batch: n rows of dimension floats (host); out-of-range ids
 * give zero rows. */
yl_status yl_get_embeddings(const yl_model *m, const uint32_t *tokens, size_t n, float *out);

yl_session *yl_create_session(const yl_model *m);
void yl_session_free(yl_session *s);
yl_status yl_session_reset(yl_session *s);

/* Decode attention of a session (one token per forward_x / generate step).
 * YL_ATTN_EXACT (the default) is fused_attention (forward.rs:299-400) in the
 * reference's operation order, bit for bit.  YL_ATTN_SPLIT has no
 * counterpart in the reference: it computes the same softmax-weighted sum
 * with the context split over many workgroups (running maxima and sums
 * combined in f32, a hardware exp2), so its results differ in rounding only,
 * for callers whose bar is a tolerance rather than identical bits; it reads
 * contexts of any length.  Head size 64 or 128 with 1, 2, 4 or 8 query heads
 * per kv head, else YL_ERR_UNSUPPORTED.  Prompt batches stay exact. */
#define YL_ATTN_EXACT 0
#define YL_ATTN_SPLIT 1
yl_status yl_session_set_attention(yl_session *s, int32_t mode);
/* InferenceSession.pos: kept for the caller, as in the reference (the
 * forward pass itself only reads start_pos). */
uint32_t yl_session_pos(const yl_session *s);
void yl_session_set_pos(yl_session *s, uint32_t pos);
/* Device pointers of the KV cache (f32), each `floats` = n_layers * kv_ld *
 * kv_dim long, kv_ld = ctx_len rounded up to a multiple of 4: values
 * [n_layers][kv_ld][kv_dim] as in the reference (rows past ctx_len unused),
 * keys transposed per layer, [n_layers][kv_dim][kv_ld]. */
yl_status yl_session_kv(yl_session *s, float **key_cache, float **value_cache, size_t *floats);

/* Transformer::forward_x: tokens (host) at start_pos..start_pos+n-1; writes
 * the last token's logits (host, vocab floats) when logits != NULL and its
 * greedy argmax when argmax != NULL.  K/V accumulate into the session's
 * cache as in the reference (forward.rs:166-169). */
yl_status yl_forward_x(const yl_model *m, const uint32_t *tokens, size_t n, uint32_t start_pos,
                       yl_session *s, float *logits, uint32_t *argmax);

/* Greedy decode: n_steps forward_x calls of one token each, the first on
 * `token` at start_pos, each next one on the previous step's argmax, without
 * host round trips (tokens stay on the device; each step is one HIP graph
 * launch).  out_tokens (host, n_steps) receives the argmax of every step. */
yl_status yl_generate_greedy(const yl_model *m, yl_session *s, uint32_t token, uint32_t start_pos,
                             uint32_t n_steps, uint32_t *out_tokens);

/* ------------------------------------------------------------ profiling */
/* Timing of one kernel class of a forward step over `batch` tokens at
 * positions start_pos..start_pos+batch-1 (batch 1: a decode step): the
 * class's launches of one step (one per layer; one for logits) are
 * captured back to back in a HIP graph, replayed `reps` times between two
 * HIP events on the session's stream, and the elapsed time is divided by
 * the launches.  kernel_class: 0 = QKV projection (RoPE/KV epilogue; at
 * batch 1 with its RMSNorm prologue), 1 = attention, 2 = Wo projection,
 * 3 = gate/up projection (SwiGLU epilogue; at batch 1 with its RMSNorm
 * prologue), 4 = down projection, 5 = logits.  For batch >= 16 the
 * projections are the int8-MFMA GEMM alone (the row normalization before
 * it is not captured).  Returns the average launch time (us), the
 * algorithmic bytes one launch reads and writes (attention: the keys and
 * values of all start_pos + batch positions, the queries and the quantized
 * output) and the
 * launches per step.  Leaves the session's KV cache at those positions, its
 * residual stream and its activations modified (the replays repeat the `+=`
 * steps): reset the session afterwards. */
yl_status yl_profile_kernel(const yl_model *m, yl_session *s, uint32_t token, uint32_t start_pos,
                            uint32_t batch, int32_t kernel_class, uint32_t reps, double *us_per_launch,
                            uint64_t *bytes_per_launch, uint32_t *launches);

/* Timing of one decode step at start_pos as its graph launches it (every
 * layer's five kernels, then the logits kernel, which here leaves the
 * position unchanged), without the launches of kernel_class (the classes of
 * yl_profile_kernel; -1: none): the graph is replayed `reps` times between
 * two HIP events on the session's stream.  A class's cost inside the step,
 * with the kernel boundaries it brings, is the full step's time minus the
 * time without it.  No counterpart in the reference: a measurement hook for
 * benchmarks.  Leaves the session's state modified, as yl_profile_kernel. */
yl_status yl_profile_step(const yl_model *m, yl_session *s, uint32_t token, uint32_t start_pos,
                          int32_t kernel_class, uint32_t reps, double *us_per_step);

/* Timing of a plain stream of one GEMV class's weights (kernel_class 0, 2,
 * 3 or 4 of yl_profile_kernel; GGUF Q8_0/Q4_0 models): per layer, one
 * launch of as many workgroups of the same size as that class's one-token
 * GEMV, each reading its slice of the layer's quantized values and scales
 * with 16-byte non-temporal loads; the layers' launches in one graph,
 * replayed `reps` times.  Returns us per launch and the bytes one launch
 * reads: the floor a GEMV of this shape can reach with kernels per layer.
 * No counterpart in the reference: a measurement hook for benchmarks. */
yl_status yl_profile_stream(const yl_model *m, yl_session *s, int32_t kernel_class, uint32_t reps,
                            double *us_per_launch, uint64_t *bytes_per_launch);

/* Elementwise probe of the device arithmetic the path relies on (device
 * pointers, n floats): exp, sqrt(|x|), 1/x and f16 widening of (i & 0xffff). */
yl_status yl_math_selftest(const float *x, size_t n, float *exp_out, float *sqrt_out,
                           float *recip_out, float *f16_out);

/* Probe of the one-wavefront serial sum behind the decode softmax
 * denominator (forward.rs:356-361): out[c] = ((0 + v[a]) + v[a+1]) + ... +
 * v[b-1] in f32 for a = offsets[c], b = offsets[c+1], values >= 0 (device
 * pointers; offsets holds cases + 1 entries).  segment 0 sums each case in
 * one pass; segment k > 0 in consecutive pieces of k values, each piece
 * continuing from the previous piece's sum (the long-context path);
 * segment 0xFFFFFFFF by the segmented sum of the decode attention (four
 * wavefronts, candidate starts per segment; cases up to 37,000 values);
 * segment 0xFFFFFFFE by the wide segmented sum of the long-context softmax
 * (eight wavefronts, 128 candidate starts per segment). */
yl_status yl_serial_sum_selftest(const float *v, const uint32_t *offsets, size_t cases, uint32_t segment,
                                 float *out);

/* Probe of the timeout report: a kernel on the null stream marks the process's
 * fault word the way a GEMV's bounded internal wait does when it gives up, so
 * the next synchronizing call (yl_synchronize, yl_forward_x, ...) returns
 * YL_ERR_HIP with a message, and clears the word. */
yl_status yl_wait_fault_selftest(void);

/* ----------------------------------------------------- tokenizer, sampler */
/* The GGUF tokenizer (tokenizer.ggml.* and tokenizer.chat_template metadata,
 * transformer_llama_gguf.rs:584-641; Tokenizer, tokenizer.rs).  Host only.
 * Id outputs: `out` holds `cap` ids; *n receives the result's length;
 * YL_ERR_RANGE (nothing written) when cap is smaller.  Where the reference
 * panics, YL_ERR_ARG. */
typedef struct yl_tokenizer yl_tokenizer;
/* From a file alone (no weights, no GPU): a Hugging Face tokenizer.json
 * (Tokenizer::from_json, tokenizer.rs:134-224), a llama2.c tokenizer.bin
 * (Tokenizer::new, tokenizer.rs:226-268), else a GGUF file's metadata
 * (Tokenizer::from_gguf_parts, tokenizer.rs:77-132). */
yl_tokenizer *yl_tokenizer_load(const char *path);
void yl_tokenizer_free(yl_tokenizer *t);
/* The tokenizer of a loaded model (owned by the model). */
const yl_tokenizer *yl_model_tokenizer(const yl_model *m);
size_t yl_tokenizer_vocab_size(const yl_tokenizer *t);
/* Tokenizer::encode(text, bos, eos), tokenizer.rs:325-380 (text non-empty UTF-8) */
yl_status yl_tokenize(const yl_tokenizer *t, const char *text, int32_t bos, int32_t eos, uint32_t *out, size_t cap,
                      size_t *n);
/* Tokenizer::decode, tokenizer.rs:545-568: UTF-8 (invalid bytes replaced by
 * U+FFFD), NUL-terminated into out[cap]; *len receives its byte length. */
yl_status yl_detokenize(const yl_tokenizer *t, const uint32_t *ids, size_t n, char *out, size_t cap, size_t *len);
/* which = 0: apply_system_template(text) (tokenizer.rs:496-514);
 *         1: apply_turn_template(text, flag) (tokenizer.rs:516-543);
 *         2: encode_wrap_n_header(text, "", flag) (tokenizer.rs:243-286). */
yl_status yl_chat_template(const yl_tokenizer *t, int32_t which, const char *text, int32_t flag, uint32_t *out,
                           size_t cap, size_t *n);
/* The first turn's prompt ids as the CLI builds them (main.rs:148-152,183):
 * conversation prefix + apply_turn_template(trim(user), true). */
yl_status yl_chat_prompt(const yl_tokenizer *t, const char *user, uint32_t *out, size_t cap, size_t *n);
/* The GPT-2 pre-tokenizer split (tokenizer.rs:29-31) of UTF-8 text: byte
 * offsets [begin, end) of each piece, 2 per piece, into bounds[cap]. */
yl_status yl_pretokenize(const char *text, uint32_t *bounds, size_t cap, size_t *n);

/* Sampler::new / Sampler::sample (sampler.rs:40-180).  sample() rescales and
 * normalizes `logits` (host, vocab floats) in place as the reference does;
 * the draw uses the seed unchanged every call (sampler.rs:170). */
typedef struct yl_sampler yl_sampler;
yl_sampler *yl_sampler_new(size_t vocab, float temperature, float top_p, uint64_t seed);
yl_status yl_sampler_sample(yl_sampler *s, float *logits, uint32_t *token);
void yl_sampler_free(yl_sampler *s);

/* One turn of generation (main.rs:186-216) on session `s` from its current
 * position: prefill `prompt`, then sample and feed tokens until EOS, the end
 * of the context or `max_tokens` (0: no limit).  *text receives the decoded
 * pieces (release with free_string); out_ids (nullable, out_cap ids) the
 * generated ids; *n_generated their count.  The session's position advances. */
yl_status yl_generate_text(const yl_model *m, yl_session *s, yl_sampler *smp, const uint32_t *prompt,
                           size_t n_prompt, uint32_t max_tokens, char **text, uint32_t *out_ids, size_t out_cap,
                           size_t *n_generated);

/* ----------------------------------------------------- synthetic models */
typedef struct {
    uint32_t dim, hidden, n_layers, n_heads, n_kv_heads, vocab, ctx_len;
    float rope_theta, rms_eps, weight_std;
    int32_t attn_format;   /* yl_format of attn_q/k/v/output */
    int32_t ffn_format;    /* yl_format of ffn_gate/up/down */
    int32_t embd_format;   /* yl_format of token_embd (Q8_0 or Q4_0) */
    int32_t file_type;     /* general.file_type written (1, 2 or 7) */
    uint64_t seed;
    /* llama.rope.scaling.{factor, ext_factor, attn_factor,
     * original_context_length}: written when rope_scaling is nonzero */
    int32_t rope_scaling;
    float rope_scaling_factor, rope_ext_factor, rope_attn_factor;
    uint32_t rope_original_ctx;
    float attention_scale;  /* llama.attention.scale: written when nonzero */
} yl_synth_config;

/* Writes a deterministic GGUF v3 llama model: every weight ~N(0, weight_std)
 * from splitmix64 + Box-Muller (element index -> value, thread-count
 * independent), quantized GGML-style (Q8_0: d = absmax/127, q = round(x/d);
 * Q4_0: d = max/-8, q = min(15, (int)(x/d + 8.5)), element j in the low
 * nibble of byte j and j+16 in the high nibble), norms = 1.0, and a vocabulary
 * of placeholder token strings.  Host only (no GPU needed). */
yl_status yl_write_synthetic_gguf(const char *path, const yl_synth_config *cfg);

/* Tokenizer metadata for yl_write_synthetic_gguf_tok: `tokens` (n_tokens =
 * cfg->vocab strings) and `merges` ("left right" strings) become
 * tokenizer.ggml.tokens/merges; pre and chat_template (nullable: omitted)
 * tokenizer.ggml.pre and tokenizer.chat_template; add_bos_token and
 * add_space_prefix (-1: omitted, else 0/1) the boolean keys. */
typedef struct {
    const char *const *tokens;
    size_t n_tokens;
    const char *const *merges;
    size_t n_merges;
    uint32_t bos, eos;
    const char *pre;
    const char *chat_template;
    int32_t add_bos_token, add_space_prefix;
} yl_synth_tokenizer;
/* yl_write_synthetic_gguf with this tokenizer instead of the placeholder
 * vocabulary. */
yl_status yl_write_synthetic_gguf_tok(const char *path, const yl_synth_config *cfg, const yl_synth_tokenizer *tok);

/* Fills `out` (host, count floats) with the generator's N(0, std) stream
 * `stream` starting at element `first` (same values the writer uses). */
yl_status yl_synthetic_normal(uint64_t seed, uint64_t stream, uint64_t first, size_t count,
                              float std_dev, float *out);

#ifdef __cplusplus
}
#endif
#endif
