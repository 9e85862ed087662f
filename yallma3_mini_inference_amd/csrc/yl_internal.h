// yl_internal.h -- host-side declarations shared by the library's sources.
//
// Device data layout (HBM), all allocations 256-byte aligned:
//   Quantized matrix [o][n] (a reference QuantizedTensor after GGUF decode):
//     qs : Q8_0 -> int8  [o][n]            (one byte per weight)
//          Q4_0 -> uint8 [o][n/2]          (16 B per 32-block, the reference's
//                                           nibble order: byte j of a block holds
//                                           element 2j in its low nibble and 2j+1
//                                           in its high nibble, values 0..15)
//     d  : f16 bits [o][n/32]              (the GGUF block scale, widened exactly
//                                           in registers)
//   Token embedding for the logits pass and the embedding lookup, Q8_0,
//   interleaved so a wavefront reading 64 consecutive vocabulary rows issues
//   one contiguous 1 KiB load per 16-element chunk:
//     eq : uint8 [vocab/64][dim/16][64][16], holding u = q + 128 (so the
//          logits pass widens it with one unsigned-byte conversion)
//     ed : f16   [vocab/64][dim/32][64]
//   KV cache (InferenceSession, base_transformer.rs:81-98), f32:
//     values [n_layers][ctx_len][kv_dim] (the reference's layout);
//     keys   [n_layers][kv_dim][kv_ld], transposed (kv_ld = ctx_len rounded
//            up to a multiple of 4), so that decode attention loads one key
//            dimension of 4 consecutive positions per 16-byte lane access.
//   Both caches hold n_layers * kv_ld * kv_dim floats.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace yl {

enum Fmt : int { kQ8 = 0, kQ4 = 1, kF16 = 2 };   // WeightFormat, weight_type.rs:17-22
// The GEMV's weight format for Q8 rows whose 32-blocks carry f32 scales
// (QMat::sf: lm.rs and safetensors Q8 with group size 32); activations and
// results as for kQ8.
constexpr int kQ8S = 3;
// The same with one f32 scale per group of 64 (two 32-blocks) or 128 (four)
// elements: activations are quantized in those groups, and a group's block
// dots are added as integers before its one f32 term.
constexpr int kQ8S64 = 4;
constexpr int kQ8S128 = 5;
// F16 gate/up matrices interleave blocks of this many gate rows with the
// same up rows (the SwiGLU tiles of the F16 GEMV: 32 + 32 rows); the gate
// and up row counts are multiples of 32.
constexpr int kF16PairRows = 32;

// The column of stored row c of a q or k projection whose heads (hd a
// power of two) hold their rows in the order 0, h, 1, h+1, ..., h-1, 2h-1
// (h = hd/2), so that util::rope's pairs (j, j + h) are adjacent rows: row
// 2j+e of a head holds column j + e*h.  c itself when `hf` is 0.
__host__ __device__ __forceinline__ int qk_column(int c, int hd, int hf) {
    if (!hf) return c;
    const int within = c & (hd - 1);
    return c - within + (within >> 1) + (within & 1) * (hd >> 1);
}

struct QMat {          // device-resident quantized matrix
    int fmt = 0;       // kQ8 / kQ4 / kF16
    int o = 0, n = 0, nb = 0;
    uint8_t* qs = nullptr;
    uint16_t* d = nullptr;
    float* sf = nullptr;   // Q8 with f32 scales [o][n/gs] (lm.rs, safetensors); d unused then
    int gs = 32;
    size_t bytes() const {
        if (sf) return (size_t)o * n + (size_t)o * (n / gs) * 4;
        return fmt == kF16 ? (size_t)o * n * 2 : (size_t)o * (fmt == kQ4 ? n / 2 : n) + (size_t)o * nb * 2;
    }
};

struct EmbQ8 {         // interleaved token embedding
    int vocab = 0, dim = 0, tiles = 0;
    int dimp = 0;      // dim rounded up to 64: the padding has scale 0 (Q8) or value 0 (F16)
    int fmt = 0;       // 0: Q8_0 (q = u8 values, d = f16 scales); 1: F16 (q = f16 values);
                       // 3: Q8 with f32 scales per gs group (q = int8 values, d32 = scales)
    int8_t* q = nullptr;
    uint16_t* d = nullptr;
    float* d32 = nullptr;   // fmt 3: scale of group g of row (tile, lane) at d32[(g * tiles + tile) * 64 + lane]
    int gs = 32;
};
// Layout: vocabulary rows in tiles of 64 (lane = row % 64).  Chunk k (16
// values, bytes u = q + 128) of every row of every tile lies together,
// [k][tile][lane][16], and so do the f16 scales of 32-block b,
// [b/2][tile][lane][2] (one 4-byte load per block pair): wavefronts that walk
// their tiles chunk by chunk read neighbouring kibibytes, which HBM serves
// much faster than one separate stream per wavefront.
__host__ __device__ inline size_t emb_q_off(int tiles, size_t tile, int k16, int lane) {
    return (((size_t)k16 * tiles + tile) * 64 + lane) * 16;
}
__host__ __device__ inline size_t emb_d_idx(int tiles, size_t tile, int b, int lane) {
    return (((size_t)(b >> 1) * tiles + tile) * 64 + lane) * 2 + (b & 1);
}

// Per-session step state on the device: read by every kernel of a decode
// step, advanced by the final kernel so greedy steps chain without the host.
struct StepState {
    int32_t pos;               // position of the first token of this call
    uint32_t token;            // decode input token (next greedy token after a step)
    uint32_t n_out;            // tokens written to the output ring so far
    uint32_t logits_done;      // logits workgroups done in this step (zero between steps)
    unsigned long long argmax; // packed argmax key of the current step
};

// Epilogue kinds of the quantized GEMV kernel.
enum Epi : int {
    kEpiStore = 0,    // out[r] = (accumulate ? out[r] : 0) + sum of block terms
    kEpiQkvRope = 1,  // rows [q | k | v]: q stored, k/v accumulate into the cache, RoPE on q,k
                      // (prologue: RMSNorm + quantize of the residual stream)
    kEpiResid = 2,    // x[r] += sum (residual add)
    kEpiSwiglu = 3,   // 64-row groups [32 gate | 32 up] -> SwiGLU -> quantize one 32-block (or f32 h only)
    kEpiResidQ = 4,   // as kEpiResid, the input an f32 row xf that the prologue quantizes
};

struct GemvArgs {
    // weights and activations
    const uint8_t* qs; const uint16_t* d; int n, o, nb;
    const float* sf;                           // kQ8S / kQ8S64 / kQ8S128: f32 scales [o][nb], [o][nb / 2], [o][nb / 4] (d unused)
    const float* xf;                           // kEpiResidQ: f32 input rows [batch][n]
    const int8_t* xq; const float* xs;        // [batch][n], [batch][nb] (staged prologue)
    // kEpiQkvRope / kEpiSwiglu prologue: RMSNorm + quantize of x [batch][n]
    float* x; const float* norm_w; float eps;
    EmbQ8 emb; const uint32_t* tokens;         // emb.q set: x starts as the tokens' embedding rows
    // kEpiStore
    float* out; int accumulate_cols;           // columns < accumulate_cols start from out[]
    // kEpiQkvRope
    float* q_out; float* k_cache; float* v_cache;   // k_cache [kv_dim][kv_ld], v_cache [positions][kv_dim]
    int att_dim, kv_dim, head_size, kv_ld;
    const float* rope_cos; const float* rope_sin;  // [ctx][head_size/2]
    const StepState* state;
    // nonzero: util::rope pairs (j, j + head_size/2), with the q and k rows
    // of each head stored in the order 0, h, 1, h+1, ..., h-1, 2h-1
    // (h = head_size/2) so a pair's rows are adjacent; row 2j+e of a head
    // holds column j + e*h, where its result is written
    int hf_rows;
    // kEpiSwiglu
    int8_t* hq; float* hs; float* h_f32; int hidden; int h_fmt;
    // set to nonzero when a bounded wait inside the kernel gives up (its
    // results are then invalid); a word of pinned host memory, or null
    unsigned* fault;
};
// The process's fault word (pinned host memory, allocated on the first call
// with `allocate`; null before that or if the allocation failed).
unsigned* wait_fault_word(bool allocate);

// kernel launchers; all return the hipError_t of the launch
hipError_t launch_set_state(StepState* st, int32_t pos, uint32_t token, hipStream_t s);
hipError_t launch_gemv(const GemvArgs& a, int wfmt, int epi, int batch, hipStream_t s);
// the one-token GEMV's grid and workgroup size for o rows of nb blocks in
// weight format wfmt
bool gemv_launch_shape(int o, int nb, int epi, int wfmt, int* grid, int* threads);
// a plain stream of abytes at a then bbytes at b (multiples of 16) by `grid`
// workgroups of `threads` (measurement only; sink is never written in practice)
hipError_t launch_stream(const void* a, size_t abytes, const void* b, size_t bbytes, int grid, int threads,
                         unsigned* sink, hipStream_t s);
hipError_t launch_quantize(int fmt, int8_t* q, float* scale, const float* x, size_t n, hipStream_t s);
// many-token matmul on int8 MFMA (same epilogues and results as the GEMV;
// activations always pre-quantized in xq/xs, M = tokens)
bool gemm_supported(const GemvArgs& a, int wfmt, int epi, int M);
size_t gemm_lds_bytes(int wfmt, int tm);
hipError_t launch_gemm(const GemvArgs& a, int wfmt, int epi, int M, hipStream_t s);
// out[c * out_ld + r] = in[r][c] for an in[rows][cols] f32 matrix
hipError_t launch_transpose(const float* in, float* out, int rows, int cols, int out_ld, hipStream_t s);
hipError_t launch_rmsnorm(int qfmt, const float* x, const float* w, int dim, float eps, int batch,
                          float* xn, int8_t* xq, float* xs, hipStream_t s);
hipError_t launch_embed(const EmbQ8& e, const uint32_t* tokens, int batch, float* x, hipStream_t s);
// kc: keys [kv_dim][kv_ld] (transposed), vc: values [max_seq][kv_dim];
// max_seq = the call's seq_len, which attention_row_fits() must accept
bool attention_row_fits(int seq_len, int head_size);
hipError_t launch_attention(const float* sq, const float* kc, const float* vc, const StepState* st,
                            int batch, int max_seq, int kv_ld, int n_heads, int n_kv_heads, int head_size,
                            float scale, int qfmt, int8_t* aq, float* as, float* att_f32,
                            hipStream_t s);
size_t attn_decode_lds_bytes(int max_seq);
// The longest context one decode step attends over for this head layout,
// and whether a context of max_seq positions is within it.
int attn_decode_limit(int n_heads, int n_kv_heads, int head_size);
bool attn_decode_fits(int max_seq, int n_heads, int n_kv_heads, int head_size);
hipError_t launch_attn_decode(const float* sq, const float* kc, const float* vc, const StepState* st,
                              int max_seq, int kv_ld, int n_heads, int n_kv_heads, int head_size, float scale,
                              int qfmt, int8_t* aq, float* as, float* att_f32, float* sc, hipStream_t s);
// sc: scratch for the scores of long contexts, attn_scores_bytes() bytes
// (0: the context is short enough for the single decode kernel; sc may be null)
// Prompt batches of 64 or more tokens, and shorter ones whose seq_len is
// too long for k_attention's LDS row: tiled attention over a scratch of
// prompt_attn_bytes(n_heads, seq_len, batch); seq_ld = pos + batch (host side)
bool prompt_attn_applies(int batch, int seq_len, int head_size);
size_t prompt_attn_bytes(int n_heads, int seq_ld, int batch);
hipError_t launch_prompt_attention(const float* sq, const float* kc, const float* vc, const StepState* st, int batch,
                                   int seq_ld, int kv_ld, int n_heads, int n_kv_heads, int head_size, float scale,
                                   int qfmt, int8_t* aq, float* as, float* att_f32, float* scratch, hipStream_t s);
bool attn_decode_split(int max_seq);
size_t attn_scores_bytes(int n_heads, int max_seq);
hipError_t launch_rope(const float* cos_t, const float* sin_t, const StepState* st, int batch,
                       float* q, float* k, int n_heads, int n_kv_heads, int head_size, hipStream_t s);
hipError_t launch_swiglu_quant(int qfmt, const float* gate, const float* up, int hidden, int batch,
                               float* h_f32, int8_t* hq, float* hs, hipStream_t s);
size_t logits_lds_bytes(int dim);
// logits pass (keys: logits_blocks() per-workgroup argmax keys) + finalize
hipError_t launch_logits(const EmbQ8& e, const float* x, const float* norm_w, float eps, float* logits,
                         StepState* st, uint32_t* ring, uint32_t ring_cap, int advance,
                         hipStream_t s);
hipError_t launch_math_selftest(const float* x, int n, float* exp_out, float* sqrt_out,
                                float* div_out, float* f16_out, hipStream_t s);

hipError_t launch_raise_fault(unsigned* fault, hipStream_t s);
// F16 weights (matmul_f32): out[t * out_ld + r] (= or +=, epi 0/1) of f16 w [o][n]
// and f32 x [batch][n]; the QKV step (RoPE, `=` into the caches)
hipError_t launch_matmul_f16(const uint16_t* w, int n, int o, const float* x, int batch, float* out, int out_ld,
                             int epi, hipStream_t s);
// Q8 with f32 scales and group size gs (see yl_q8g.hip).  Output rows
// [seg[i-1].row_end, seg[i].row_end) go to segment i: element (token t,
// column c) at out[pos * pos_stride + t * stride_tok + c * stride_row], pos =
// st->pos (0 without st); columns below acc_cols start from the output's value.
struct Q8gSegArgs {
    float* out = nullptr;
    long pos_stride = 0, stride_row = 1, stride_tok = 0;
    int row_end = 0, acc_cols = 0;
};
struct Q8gArgs {
    const int8_t* w = nullptr;    // [o][n]
    const float* wsc = nullptr;   // [o][n/gs]
    int n = 0, o = 0, gs = 32;
    int pro = 0;   // 0: quantized rows xq/xs; 1: quantize the f32 rows x; 2: RMSNorm(x, norm_w, eps), then quantize
    int epi = 0;   // 0: store (segments); 1: add to the output (segment 0); 2: SwiGLU of gate/up tile pairs -> seg 0
    const int8_t* xq = nullptr;
    const float* xs = nullptr;
    const float* x = nullptr;
    const float* norm_w = nullptr;
    float eps = 0.0f;
    int batch = 1;
    const StepState* st = nullptr;
    int nseg = 1;
    Q8gSegArgs seg[3];
    int pair_rows = 16;   // epi 2: gate rows then up rows per block (16 or 32; the upload's interleave)
    int perm_hd = 0;      // epi 0: 0, or the head size of segments 0 and 1 stored in pair order (qk_column)
};
hipError_t launch_matmul_q8g(const Q8gArgs& a, hipStream_t s);
hipError_t launch_quantize_gs(const float* x, int8_t* q, float* sc, int gs, size_t n, hipStream_t s);
hipError_t launch_rope_cache(const float* cos_t, const float* sin_t, const StepState* st, int batch, float* q,
                             float* kc, int att, int kv, int hd, int kv_ld, int hf_pairs, hipStream_t s);
// One token through f16 weights with the chain fed from LDS (o % 16 == 0):
// norm_w non-null applies RMSNorm to x first; epi 0 store, 1 add, 2 SwiGLU
// of the 8-row gate/up pairs of each 16-row block -> out[o / 2].
// The F16 one-token QKV epilogue (epi 3): rows [q | k | v] rotated in
// pairs of adjacent rows (rope_gguf pairs, or util::rope pairs stored in pair
// order when hf: qk_column), q to q_out, k and v assigned into the caches at
// position st->pos (keys transposed [kv][kv_ld]).
struct F16Qkv {
    float* q_out = nullptr; float* k_cache = nullptr; float* v_cache = nullptr;
    const float* rope_cos = nullptr; const float* rope_sin = nullptr;   // [ctx][head/2]
    const StepState* st = nullptr;
    int att = 0, kv = 0, hd = 0, kv_ld = 0, hf = 0;
};
hipError_t launch_f16_gemv(const uint16_t* w, int n, int o, const float* x, const float* norm_w, float eps, int epi,
                           float* out, hipStream_t s,
                           const F16Qkv* qkv = nullptr);
// raw [batch][2 * hidden] in that pair layout -> h [batch][hidden]
hipError_t launch_swiglu_pairs(const float* raw, int hidden, int batch, float* h, hipStream_t s);
hipError_t launch_qkv_f16(const float* raw, const float* cos_t, const float* sin_t, const StepState* st, int batch,
                          float* sq, float* kc, float* vc, int att, int kv, int hd, int kv_ld, int hf_pairs,
                          hipStream_t s);
// Decode attention split over the context (tolerance mode): workgroups per
// kv head, scratch bytes (partials + one count per kv head, the counts zero
// before the first launch; each launch leaves them zero), and the launch.
int attn_split_parts(int n_kv_heads);
size_t attn_split_bytes(int n_heads, int n_kv_heads, int head_size);
bool attn_split_supported(int n_heads, int n_kv_heads, int head_size);
hipError_t launch_attn_split(const float* sq, const float* kc, const float* vc, const StepState* st, int kv_ld,
                             int n_heads, int n_kv_heads, int head_size, float scale, int qfmt, int8_t* aq, float* as,
                             float* att_f32, float* scratch, hipStream_t s);
hipError_t launch_serial_sum_selftest(const float* v, const uint32_t* offs, int cases, int seg, float* out,
                                      hipStream_t s);

// error reporting shared by the C ABI
void set_error(const std::string& msg);

}  // namespace yl
