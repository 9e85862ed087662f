// yl_attn.hip -- attention over the device KV cache (forward.rs:299-400).
//
// Arithmetic of fused_attention, per (query head, token):
//   score[t2] = reduce_add(8-lane partial q.k over head_size) * scale
//   max from -1e10; e = exp(score - max); sum_exp serial over t2;
//   p = e * (1/sum_exp);  out[d] = reduce_add(lane j sums p*v over t2 = 8c+j
//   in c order) + the seq_len % 8 tail in t2 order.
//
// k_attn_decode (one token): grid (n_heads, head_size/32), one workgroup
// per 32 output dimensions of a head, independent of every other
// workgroup.  k_attention (prompt batches) keeps one workgroup per
// (head, token) with the causal mask of the whole call's span.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kAttnThreads = 256;

template <int QF>
__device__ void quantize_head_output(const float* outl, int hd, int8_t* aq, float* as, size_t group0) {
    const int ng = hd / kGroup;
    for (int g = threadIdx.x; g < ng; g += blockDim.x) {
        const float* v = outl + g * kGroup;
        float amax = 0.0f;
        for (int k = 0; k < kGroup; k++) amax = fmaxf(amax, fabsf(v[k]));
        const float s = group_scale<QF>(amax);
        as[group0 + g] = s;
        for (int k = 0; k < kGroup; k++) aq[(group0 + g) * kGroup + k] = (int8_t)quant_one<QF>(v[k], s);
    }
}

// ---------------------------------------------------------------------------
// Decode (one token).  Workgroup (h, ds) owns query head h and the 32
// output dimensions [32*ds, 32*ds + 32) of it -- exactly one quantization
// group of the attention output -- and needs no other workgroup:
//   1. scores: thread t scores positions 4t..4t+3 (+ 4*512 per round); the
//      key cache is transposed ([kv_dim][kv_ld]), so one 16-byte load per
//      lane brings a key dimension of 4 positions, and the dimensions are
//      consumed in groups of 8 (the reference's lane partials) with the next
//      group's loads in flight; q is read as uniform (scalar) values;
//   2. max, exp, and the serial sum (segmented over wavefronts 0-3);
//   3. the P.V chains of its 32 dimensions over V tiles of 256 positions
//      that LDS DMA (16 bytes per lane) fills: up to 112 chunks (903
//      positions) with every tile resident, the DMA wavefronts copy their V
//      values into registers during the sum and run the chains with p from
//      registers; longer contexts refill the tiles up to 4 ahead and the
//      chains read V and p from LDS;
//   4. the 8-lane reduction + tail, and the quantized group.
// Only 16-byte loads per lane keep the CU's memory pipeline at full width
// (a 4-byte load per lane moves a quarter of the bytes per address cycle).
// Scores, exponentials and probabilities live in one transposed array,
// pt[j][c] = x[8c + j], the layout the chains read.
// LDS (floats): pt 8*PCS | V tiles n_vt*256*32 | partials 8*32 | out 32 |
// reduction 16
// ---------------------------------------------------------------------------
constexpr int kDecThreads = 512;
constexpr int kDecDims = 32;                   // output dims per workgroup
constexpr int kDecChains = 8 * kDecDims;       // P.V chains per workgroup
constexpr int kVTileRows = 256;                // V rows (positions) per LDS tile
constexpr int kVTileFloats = kVTileRows * kDecDims;
constexpr int kMaxVTiles = 4;                  // V tiles in flight
constexpr int kDecLdsBudget = 156 * 1024;      // LDS bytes one workgroup may use
constexpr int kBufFlags = 0x00020000;          // buffer descriptor word 3: raw 32-bit data
// wavefronts that run the softmax denominator of contexts up to
// kAttnSplitSeq (seg_serial_sum: 2 segments of the row each)
constexpr int kSumWaves = 4;
// seg_serial_sum's LDS scratch (floats): segment ends, bases, then the
// float64 segment sums
constexpr int kSumScratch = 2 * kSumWaves * 64 + 2 * kSumWaves + 2 * (2 * kSumWaves);
static_assert(kDecThreads / 64 == 2 * kSumWaves, "one sum segment per wavefront's exponentials");

// pt row stride: positions up to max_seq rounded to 64 (the serial sum
// reads zero padding to that length), + 4 floats to spread banks
__host__ __device__ inline int attn_pt_stride(int max_seq) { return ((max_seq + 63) & ~63) / 8 + 4; }
// contexts longer than this take the scores kernel + the decode kernel
constexpr int kAttnSplitSeq = 4096;
// + for contexts up to kAttnSplitSeq, the exponentials in position order for
// the serial sum (max_seq rounded up to 64) and the sum's scratch; longer
// ones sum from pt
__host__ __device__ inline size_t attn_fixed_lds_floats(int max_seq) {
    const size_t el = max_seq <= kAttnSplitSeq ? (size_t)((max_seq + 63) & ~63) + kSumScratch : 0;
    return 8 * (size_t)attn_pt_stride(max_seq) + 8 * kDecDims + kDecDims + 16 + el;
}
// V tile buffers that fit beside the fixed part (0: fewer than 2 fit)
__host__ __device__ inline int attn_v_tiles(int max_seq) {
    const long long free_b = kDecLdsBudget - (long long)attn_fixed_lds_floats(max_seq) * 4;
    const int n = free_b > 0 ? (int)(free_b / (kVTileFloats * 4)) : 0;
    return n >= 2 ? (n > kMaxVTiles ? kMaxVTiles : n) : 0;
}
__host__ __device__ inline size_t attn_decode_lds_floats(int max_seq) {
    return attn_fixed_lds_floats(max_seq) + (size_t)attn_v_tiles(max_seq) * kVTileFloats;
}

__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ vf4 buf_load_f32x4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(vf4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// LDS DMA of V rows [r0, r0 + kVTileRows) of 32 columns from col0 into an
// LDS tile [kVTileRows][32]: one instruction moves 8 rows (64 lanes x 16
// bytes).  Only the last kDmaWaves wavefronts issue them (kVTileDmaPerWave
// each per tile); they have no P.V chains and are idle while wavefront 0
// sums the softmax denominator.  Rows past `rows` re-read the last one
// (never used).
constexpr int kDmaWaves = 4;
constexpr int kDmaWave0 = kDecThreads / 64 - kDmaWaves;
constexpr int kVTileDmaPerWave = kVTileRows / 8 / kDmaWaves;
static_assert(kDecChains <= kDmaWave0 * 64, "the DMA wavefronts hold no P.V chain");
__device__ __forceinline__ void v_tile_dma(float* tile, const float* __restrict__ vc, int kv_dim, int col0, int r0,
                                           int rows) {
    const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) - kDmaWave0;
#pragma unroll
    for (int k = 0; k < kVTileDmaPerWave; k++) {
        const int g = w + k * kDmaWaves;
        const int row = min(r0 + g * 8 + (lane >> 3), rows - 1);
        __builtin_amdgcn_global_load_lds(vc + (size_t)row * kv_dim + col0 + (lane & 7) * 4, tile + g * 8 * kDecDims,
                                         16, 0, 0);
    }
}
// Waits until at most `later` tiles' DMA of this (DMA) wavefront is in flight.
__device__ __forceinline__ void wait_v_tiles(int later) {
    static_assert(kVTileDmaPerWave == 8, "wait counts below assume 8 DMA instructions per tile");
    switch (later) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    }
}

// e = exp(score - max) into pt and in position order into el for
// contexts up to kAttnSplitSeq: wavefront w takes positions [w L, w L + L)
// (L = seg_sum_len(seq, 8), 8 L = seq rounded up to 64), which is segment w
// of the serial sum, and stores their float64 sum in segsum[w]
template <int NV>
__device__ __forceinline__ void exp_segment(float* pt, float* el, int PCS, int L, int seq, float mx,
                                            double* segsum) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float ev[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int t2 = w * L + min(lane + 64 * i, L - 1);
        ev[i] = pt[(t2 & 7) * PCS + (t2 >> 3)];
    }
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int t2 = w * L + lane + 64 * i;
        const float e = t2 < seq ? expf_rn(ev[i] - mx) : 0.0f;
        if (lane + 64 * i < L) {
            pt[(t2 & 7) * PCS + (t2 >> 3)] = e;
            el[t2] = e;
            acc += (double)e;
        }
    }
    acc = wave_sum_f64(acc);
    if (lane == 0) segsum[w] = acc;
}

// e = exp(score - max) into pt and, with EL, in position order into el
template <int NV, bool EL>
__device__ __forceinline__ void exp_row(float* pt, float* el, int PCS, int b0, int seq, int pad, float mx) {
    float ev[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int t2 = min(b0 + (int)threadIdx.x + i * kDecThreads, pad - 1);
        ev[i] = pt[(t2 & 7) * PCS + (t2 >> 3)];
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int t2 = b0 + (int)threadIdx.x + i * kDecThreads;
        const float e = t2 < seq ? expf_rn(ev[i] - mx) : 0.0f;
        if (t2 < pad) {
            pt[(t2 & 7) * PCS + (t2 >> 3)] = e;
            if constexpr (EL) el[t2] = e;
        }
    }
}

constexpr int kScoreLoads = 32;   // 16-byte key loads in flight per lane (decode kernel)

// One round of the decode kernel's scores: wavefront `wave` = lane partial
// j computes partial j (key dimensions 8s + j, s in order) of NC chunks of
// 256 positions starting at r0 (4 positions per lane), every key load of
// the round issued before the first product; partials go to
// P.V from registers, for contexts of at most kPvRegChunks chunks whose V
// tiles all fit in LDS at once.  The DMA wavefronts hold the chains: while
// the others sum the softmax denominator they copy their V values
// v[8c + j][d] into registers (c in order, +0 past the last chunk), and once
// 1 / sum is known lane i of each 16-lane row (one lane partial j per row)
// holds p[8(16r + i) + j] = e * (1 / sum) in register r (+0 past the last
// chunk).  Each product p * v takes its p by DPP row broadcast, and the
// chain adds the products in c order with no LDS read inside it (each
// product rounded on its own, as in the reference).  The padded steps add
// +0 * +0 = +0, which
// leaves every sum unchanged: a chain that starts at +0 never holds -0
// (round-to-nearest gives +0 for an exact cancellation).
constexpr int kPvRegChunks = 112;   // 7 registers of 16 chunks (8 spill to scratch)
constexpr int kPvRegs = kPvRegChunks / 16;
// v[k] = p_k * v[k] for the 16 chunks of one register (p_k by DPP row
// broadcast from lane k of the row): the products go first, independent of
// the chain, so the chain is plain dependent adds (9.5 cycles per step
// measured, against 13 with each product between two adds)
template <int K = 0>
__device__ __forceinline__ void pv_dpp_products(float p, float (&v)[16]) {
    if constexpr (K < 16) {
        v[K] = fmul(row_bcast_lane<K>(p), v[K]);
        pv_dpp_products<K + 1>(p, v);
    }
}
// The chain over NR registers of products (one straight block, so the
// products of later registers are scheduled among the adds)
template <int NR>
__device__ __forceinline__ float pv_chain_regs(const float (&pr)[kPvRegs], float (&vr)[kPvRegs][16]) {
#pragma unroll
    for (int r = 0; r < NR; r++) pv_dpp_products(pr[r], vr[r]);
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc = fadd(acc, vr[r][i]);
    return acc;
}

// part[j][RP].  Quads past the row re-read its last quad (never used).
template <int HD, int NC>
__device__ __forceinline__ void score_loads(__amdgpu_buffer_rsrc_t krs, int r0, int n_quads, int lane, int wave,
                                            int row_step, vf4 (&k4)[NC][HD / 8]) {
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
        const int quad = min(r0 / 4 + ch * 64 + lane, n_quads - 1);
#pragma unroll
        for (int s = 0; s < HD / 8; s++) k4[ch][s] = buf_load_f32x4(krs, quad * 16, (8 * s + wave) * row_step);
    }
}
template <int HD, int NC>
__device__ __forceinline__ void score_products(const float* qp, const vf4 (&k4)[NC][HD / 8], int lane, int wave,
                                               float* part, int RP) {
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
        float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < HD / 8; s++) {
            const float qv = qp[8 * s];
            l[0] = fadd(l[0], fmul(qv, k4[ch][s].x));
            l[1] = fadd(l[1], fmul(qv, k4[ch][s].y));
            l[2] = fadd(l[2], fmul(qv, k4[ch][s].z));
            l[3] = fadd(l[3], fmul(qv, k4[ch][s].w));
        }
        *reinterpret_cast<vf4*>(part + wave * RP + ch * 256 + 4 * lane) = vf4{l[0], l[1], l[2], l[3]};
    }
}
template <int HD, int NC>
__device__ __forceinline__ void score_round(__amdgpu_buffer_rsrc_t krs, const float* qp, int r0, int n_quads,
                                            int lane, int wave, int row_step, float* part, int RP) {
    vf4 k4[NC][HD / 8];
    score_loads<HD, NC>(krs, r0, n_quads, lane, wave, row_step, k4);
    // (left free, the scheduler keeps a dozen loads in flight)
    __builtin_amdgcn_sched_barrier(0);
    score_products<HD, NC>(qp, k4, lane, wave, part, RP);
}
constexpr int kScoreRows = 256;   // positions per scores workgroup
constexpr int kLongQuads = 8;     // score quads per decode thread: max_seq <= 8 * 4 * kDecThreads

template <int HD>
__global__ __launch_bounds__(kDecThreads) void k_attn_scores(const float* __restrict__ sq,
                                                             const float* __restrict__ kc,
                                                             const StepState* __restrict__ st, int n_heads,
                                                             int n_kv_heads, float attn_scale, int kv_ld,
                                                             float* __restrict__ sc, int sc_ld) {
    extern __shared__ __align__(16) float lds[];
    const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int j = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int seq = st->pos + 1;
    const int p0 = blockIdx.y * kScoreRows;
    if (p0 >= seq) return;
    const int r = n_heads / n_kv_heads;
    // quads start at most at the last position and rows are kv_ld >= seq (a
    // multiple of 4) long, so every 16-byte read stays inside its row
    const int quad = min(p0 / 4 + lane, (seq + 3) / 4 - 1);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(kc + (size_t)g * HD * kv_ld), (short)0, HD * kv_ld * 4, kBufFlags);
    vf4 k4[HD / 8];
#pragma unroll
    for (int s = 0; s < HD / 8; s++) k4[s] = buf_load_f32x4(krs, quad * 16, (8 * s + j) * kv_ld * 4);
    for (int hh = 0; hh < r; hh++) {
        const float* qp = sq + (size_t)(g * r + hh) * HD + j;
        float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < HD / 8; s++) {
            const float qv = qp[8 * s];
            l[0] = fadd(l[0], fmul(qv, k4[s].x));
            l[1] = fadd(l[1], fmul(qv, k4[s].y));
            l[2] = fadd(l[2], fmul(qv, k4[s].z));
            l[3] = fadd(l[3], fmul(qv, k4[s].w));
        }
        *reinterpret_cast<vf4*>(lds + (hh * 8 + j) * kScoreRows + 4 * lane) = vf4{l[0], l[1], l[2], l[3]};
    }
    __syncthreads();
    const int n = min(kScoreRows, seq - p0);
    for (int i = tid; i < r * kScoreRows; i += kDecThreads) {
        const int hh = i / kScoreRows, p = i % kScoreRows;
        float lj[8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) lj[jj] = lds[(hh * 8 + jj) * kScoreRows + p];
        if (p < n) sc[(size_t)(g * r + hh) * sc_ld + p0 + p] = fmul(reduce_add8(lj), attn_scale);
    }
}

template <int QF, int HD, bool LONG>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_attn_decode(
    const float* __restrict__ sq, const float* __restrict__ kc, const float* __restrict__ vc,
    const StepState* __restrict__ st, int n_heads, int n_kv_heads, float attn_scale, int max_seq, int kv_ld,
    int n_vt, int8_t* __restrict__ aq, float* __restrict__ as, float* __restrict__ att_f32,
    const float* __restrict__ sc, int sc_ld, unsigned* __restrict__ fault) {
    extern __shared__ __align__(16) float lds[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroups are dealt to the 8 XCDs round-robin by index (each XCD has
    // its own L2).  Order the (kv head, dims, query head) tuples so that
    // each XCD receives a contiguous run of them: the query heads that read
    // the same keys and V columns then share one L2.
    const int r = n_heads / n_kv_heads, nb = gridDim.x;
    const int lg = (nb & 7) ? (int)blockIdx.x : (int)(blockIdx.x & 7) * (nb >> 3) + (int)(blockIdx.x >> 3);
    const int kvh = lg / (r * (HD / kDecDims));
    const int ds = (lg / r) % (HD / kDecDims);
    const int h = kvh * r + lg % r;
    const int kv_dim = n_kv_heads * HD;
    const int PCS = attn_pt_stride(max_seq);
    float* pt = lds;
    float* vt = pt + 8 * PCS;
    float* part = vt + n_vt * kVTileFloats;
    float* outl = part + kDecChains;
    float* red = outl + kDecDims;
    float* el = red + 16;   // exponentials in position order (!LONG)
    float* sx = el + ((max_seq + 63) & ~63);   // the serial sum's scratch (!LONG)
    int* sum_ctr = reinterpret_cast<int*>(red + 12);
    int* dma_ctr = reinterpret_cast<int*>(red + 13);   // DMA wavefronts whose V tiles landed
    if (tid == 0) {   // (seen after the score rounds' barriers)
        *sum_ctr = 0;
        *dma_ctr = 0;
    }
    const float* __restrict__ qh = sq + (size_t)h * HD;
    const int col0 = kvh * HD + ds * kDecDims;
    // keys of this kv head through a buffer descriptor: a per-lane 32-bit
    // offset (4 positions) and a uniform offset per key dimension, so no
    // load needs a 64-bit address register; quads start at most at the last
    // position, and rows are kv_ld >= max_seq (a multiple of 4) long, so
    // every 16-byte read stays inside its row
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(kc + (size_t)kvh * HD * kv_ld), (short)0, HD * kv_ld * 4, kBufFlags);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(vc), (short)0, max_seq * kv_dim * 4, kBufFlags);
    const int lane = tid & 63;

    // The key loads of the first score round go out before the step's
    // position is read (one dependent load later): they cover the first
    // positions of the context up to one round (clamped to max_seq), and
    // the scores of positions past seq are never used.
    constexpr int NCH = kScoreLoads / (HD / 8);   // chunks of 256 positions per round
    constexpr int RP = NCH * 256;
    // Chunk 0 (positions 0-255, always scored) goes out first; the chunks
    // of round 0 that hold positions follow once the position is read, the
    // others are not fetched (zero registers, their partials never read).
    vf4 k0[LONG ? 1 : NCH][HD / 8];
    const int q0 = (min(max_seq, RP) + 3) / 4;
    if constexpr (!LONG) {
#pragma unroll
        for (int s8 = 0; s8 < HD / 8; s8++)
            k0[0][s8] = buf_load_f32x4(krs, min(lane, q0 - 1) * 16, (8 * s8 + wave) * kv_ld * 4);
    }
    const int seq = st->pos + 1;
    const int n_chunks = seq / 8;
    if constexpr (!LONG) {
        const int live0 = min(NCH, (seq + 255) / 256);
#pragma unroll
        for (int ch = 1; ch < NCH; ch++) {
            const int quad = min(ch * 64 + lane, q0 - 1);
            if (ch < live0) {   // (uniform)
#pragma unroll
                for (int s8 = 0; s8 < HD / 8; s8++)
                    k0[ch][s8] = buf_load_f32x4(krs, quad * 16, (8 * s8 + wave) * kv_ld * 4);
            } else {
#pragma unroll
                for (int s8 = 0; s8 < HD / 8; s8++) k0[ch][s8] = vf4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }

    // the seq % 8 tail rows of V, for the output threads (tid < 32)
    float vtail[7];
#pragma unroll
    for (int i = 0; i < 7; i++)
        vtail[i] = buf_load_f32(vrs, (col0 + (tid & 31)) * 4, min(n_chunks * 8 + i, seq - 1) * kv_dim * 4);

    // 1. scores -> pt (transposed)
    const int n_quads = (seq + 3) / 4;
    float lmax = -1e10f;
    if constexpr (LONG) {
        // the scores kernel's row of this head (rows are sc_ld >= max_seq, a
        // multiple of 4, floats long)
        // every load is issued before the first is used (quads past the row
        // re-read its last quad)
        const float* __restrict__ sh = sc + (size_t)h * sc_ld;
        vf4 s4[kLongQuads];
#pragma unroll
        for (int i = 0; i < kLongQuads; i++)
            s4[i] = *reinterpret_cast<const vf4*>(sh + 4 * min(tid + i * kDecThreads, n_quads - 1));
#pragma unroll
        for (int i = 0; i < kLongQuads; i++)
#pragma unroll
            for (int pp = 0; pp < 4; pp++) {
                const int p = 4 * (tid + i * kDecThreads) + pp;
                const bool live = p < seq;
                *(live ? pt + (p & 7) * PCS + (p >> 3) : red + 15) = s4[i][pp];
                lmax = fmaxf(lmax, live ? s4[i][pp] : -1e10f);
            }
    } else {
        // wavefront j computes lane partial j (key dimensions 8s + j, s in
        // order) of every position, 4 per lane: a round takes NCH chunks of
        // 256 positions with all their key rows in flight (HD/8 16-byte
        // loads per chunk), and the partials meet in the V tile area
        // ([8][RP], free until the V DMA starts) for reduce_add8 and the scale
        // round 0 from the keys already in flight, then rounds of only the
        // chunks that hold positions (loads past the last one would all
        // re-read its last quad, still costing memory-pipe cycles), one
        // straight-line variant per chunk count
        static_assert(8 * RP <= 2 * kVTileFloats, "partials must fit two V tiles");
        float* part = vt;
        const float* qp = qh + wave;   // wave = j, uniform: scalar query loads
        const int row_step = kv_ld * 4;
        // the round's partials -> scaled scores in pt and the running max
        auto reduce_round = [&](int r0) {
            lds_barrier();
            const int nr = min(RP, seq - r0);
            for (int i = tid; i < nr; i += kDecThreads) {
                float lj[8];
#pragma unroll
                for (int jj = 0; jj < 8; jj++) lj[jj] = part[jj * RP + i];
                const int p = r0 + i;
                const float sv = fmul(reduce_add8(lj), attn_scale);
                const bool live = p < seq;
                *(live ? pt + (p & 7) * PCS + (p >> 3) : red + 15) = sv;
                lmax = fmaxf(lmax, live ? sv : -1e10f);
            }
            lds_barrier();   // part is rewritten by the next round, then by the V DMA
        };
        score_products<HD, NCH>(qp, k0, lane, wave, part, RP);
        reduce_round(0);
        for (int r0 = RP; r0 < seq; r0 += RP) {
            const int nlive = min(NCH, (n_quads - r0 / 4 + 63) / 64);
            auto round = [&](auto nc) {
                score_round<HD, decltype(nc)::value>(krs, qp, r0, n_quads, lane, wave, row_step, part, RP);
            };
            switch (nlive) {
            case 1: round(std::integral_constant<int, 1>{}); break;
            case 2: if constexpr (NCH >= 2) round(std::integral_constant<int, 2>{}); break;
            case 3: if constexpr (NCH >= 3) round(std::integral_constant<int, 3>{}); break;
            case 4: if constexpr (NCH >= 4) round(std::integral_constant<int, 4>{}); break;
            default: if constexpr (NCH >= 8) round(std::integral_constant<int, NCH>{}); break;
            }
            reduce_round(r0);
        }
    }
    const int n_tiles = (8 * n_chunks + kVTileRows - 1) / kVTileRows;
    const bool dma_wave = wave >= kDmaWave0;

    // 2. softmax: max from -1e10 (forward.rs:351-356), e = exp(s - max),
    // sum_exp serial in position order, p = e * (1 / sum_exp)
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) red[tid >> 6] = lmax;
    lds_barrier();   // the V tiles stay in flight
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < kDecThreads / 64; w++) mx = fmaxf(mx, red[w]);
    const int pad = (seq + 63) & ~63;
    double* segsum = reinterpret_cast<double*>(sx + 2 * kSumWaves * 65);
    if constexpr (LONG) {
        // up to 8 independent exponentials per thread and round (the
        // polynomial is a chain of dependent double-precision steps)
        const int nv = (pad + kDecThreads - 1) / kDecThreads;
        if (nv <= 1) exp_row<1, false>(pt, el, PCS, 0, seq, pad, mx);
        else if (nv == 2) exp_row<2, false>(pt, el, PCS, 0, seq, pad, mx);
        else if (nv <= 4) exp_row<4, false>(pt, el, PCS, 0, seq, pad, mx);
        else
            for (int b0 = 0; b0 < pad; b0 += 8 * kDecThreads) exp_row<8, false>(pt, el, PCS, b0, seq, pad, mx);
    } else {
        // wavefront w: segment w of the serial sum (L <= 512 positions)
        const int L = seg_sum_len(seq, 2 * kSumWaves);
        const int nv = (L + 63) / 64;
        if (nv <= 1) exp_segment<1>(pt, el, PCS, L, seq, mx, segsum);
        else if (nv == 2) exp_segment<2>(pt, el, PCS, L, seq, mx, segsum);
        else if (nv <= 4) exp_segment<4>(pt, el, PCS, L, seq, mx, segsum);
        else exp_segment<8>(pt, el, PCS, L, seq, mx, segsum);
    }
    lds_barrier();
    // the first V tiles start now, issued by the DMA wavefronts while
    // wavefront 0 sums
    const bool regpv = !LONG && n_chunks <= kPvRegChunks && n_tiles <= n_vt;   // (uniform)
    if (dma_wave)
        for (int t = 0; t < n_tiles && t < n_vt; t++)
            v_tile_dma(vt + t * kVTileFloats, vc, kv_dim, col0, t * kVTileRows, seq);
    // with regpv the DMA wavefronts hold the P.V chains: chain (j, d) of
    // thread rt = tid - 64 kDmaWave0, j = rt / 32, d = rt % 32
    const int rt = tid - 64 * kDmaWave0;
    const int rj = (rt >> 5) & 7, rd = rt & 31;
    float vr[kPvRegs][16];
    if (regpv && dma_wave) {
        // once every DMA wavefront's tiles have landed: V values into
        // registers while the denominator is summed
        wait_v_tiles(0);
        lds_arrive(dma_ctr);
        lds_wait_count(dma_ctr, kDmaWaves, fault);
        // (a chunk c of a live 16-group lies in tile c / 32 < n_tiles:
        // 16 ceil(n / 16) <= 32 ceil(n / 32); rows past seq repeat row
        // seq - 1, and the partial group's padding is set to +0)
        const float* vb = vt + rj * kDecDims + rd;
#pragma unroll
        for (int r = 0; r < kPvRegs; r++)
            if (16 * r < n_chunks) {   // (uniform)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    constexpr int kRowFloats = 8 * kDecDims;   // one chunk: 8 rows
                    const int c = 16 * r + i;
                    vr[r][i] = vb[(c / 32) * kVTileFloats + (c % 32) * kRowFloats];
                }
                if (16 * r + 16 > n_chunks) {   // (uniform)
#pragma unroll
                    for (int i = 0; i < 16; i++) vr[r][i] = 16 * r + i < n_chunks ? vr[r][i] : 0.0f;
                }
            }
    }
    if (LONG && tid < 64) {
        // one wavefront, from the transposed row
        const float sum = wave_serial_sum_at([pt, PCS](int i) { return pt[(i & 7) * PCS + (i >> 3)]; }, seq);
        if (tid == 0) red[8] = sum > 0.0f ? 1.0f / sum : 0.0f;
    } else if (!LONG && tid < 64 * kSumWaves) {
        // the exponentials in position order (zero-padded to 64) by the
        // wavefronts without V DMA
        static_assert(kSumWaves <= kDmaWave0, "the sum's wavefronts issue no DMA");
        const float sum = seg_serial_sum<kSumWaves>(el, seq, segsum, sx, sum_ctr, 0, fault);
        if (tid == 0) red[8] = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    lds_barrier();
    const float inv = red[8];

    // 3. P.V chains (forward.rs:372-395): lane j adds p*v over c in order.
    if (regpv) {
        if (dma_wave) {
            // p = e * (1 / sum) of this row's 16 chunks per register
            const float* pj = pt + rj * PCS;
            // (every read issued before the first is used: clamped
            // indexes, no branch)
            const int last = n_chunks - 1, i16 = tid & 15;
            float pr[kPvRegs];
#pragma unroll
            for (int r = 0; r < kPvRegs; r++) {
                const int c = 16 * r + i16;
                const float e = pj[max(min(c, last), 0)];
                pr[r] = c <= last ? fmul(e, inv) : 0.0f;
            }
            float acc = 0.0f;
            static_assert(kPvRegs == 7, "one case per register count");
            switch ((n_chunks + 15) / 16) {
            case 1: acc = pv_chain_regs<1>(pr, vr); break;
            case 2: acc = pv_chain_regs<2>(pr, vr); break;
            case 3: acc = pv_chain_regs<3>(pr, vr); break;
            case 4: acc = pv_chain_regs<4>(pr, vr); break;
            case 5: acc = pv_chain_regs<5>(pr, vr); break;
            case 6: acc = pv_chain_regs<6>(pr, vr); break;
            case 7: acc = pv_chain_regs<7>(pr, vr); break;
            default: break;   // no whole chunk
            }
            part[rj * kDecDims + rd] = acc;
        }
    } else {
        for (int t2 = tid; t2 < seq; t2 += kDecThreads) {
            float* e = pt + (t2 & 7) * PCS + (t2 >> 3);
            *e = fmul(*e, inv);
        }
        // Chain (j, d) of thread tid < kDecChains: j = tid / 32, d = tid % 32,
        // V from LDS tiles refilled by the DMA wavefronts.
        const int cj = (tid >> 5) & 7, cd = tid & 31;
        float acc = 0.0f;
        for (int t = 0; t < n_tiles; t++) {
            // this wavefront's DMA into tile t; the later tiles already issued
            // may stay in flight
            if (dma_wave) wait_v_tiles(min(n_vt - 1, n_tiles - 1 - t));
            lds_barrier();    // the DMA of tile t (and, for t = 0, the p row)
            const float* tile = vt + (t % n_vt) * kVTileFloats;
            if (tid < kDecChains) {
                const int c0 = t * (kVTileRows / 8);
                const int steps = min(kVTileRows / 8, n_chunks - c0);
                const float* pj = pt + cj * PCS + c0;
                float vv[kVTileRows / 8];
#pragma unroll
                for (int i = 0; i < kVTileRows / 8; i++) vv[i] = tile[(8 * i + cj) * kDecDims + cd];
                if (steps == kVTileRows / 8) {
                    // a whole tile: no per-step bound
#pragma unroll
                    for (int i = 0; i < kVTileRows / 8; i += 4) {
                        const vf4 p4 = *reinterpret_cast<const vf4*>(pj + i);
                        acc = fadd(acc, fmul(p4.x, vv[i + 0]));
                        acc = fadd(acc, fmul(p4.y, vv[i + 1]));
                        acc = fadd(acc, fmul(p4.z, vv[i + 2]));
                        acc = fadd(acc, fmul(p4.w, vv[i + 3]));
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < kVTileRows / 8; i += 4) {
                        const vf4 p4 = *reinterpret_cast<const vf4*>(pj + i);
                        if (i + 0 < steps) acc = fadd(acc, fmul(p4.x, vv[i + 0]));
                        if (i + 1 < steps) acc = fadd(acc, fmul(p4.y, vv[i + 1]));
                        if (i + 2 < steps) acc = fadd(acc, fmul(p4.z, vv[i + 2]));
                        if (i + 3 < steps) acc = fadd(acc, fmul(p4.w, vv[i + 3]));
                    }
                }
            }
            if (t + n_vt < n_tiles) {
                lds_barrier();    // tile t consumed before it is refilled
                if (dma_wave) v_tile_dma(vt + (t % n_vt) * kVTileFloats, vc, kv_dim, col0, (t + n_vt) * kVTileRows, seq);
            }
        }
        if (tid < kDecChains) part[cj * kDecDims + cd] = acc;
    }
    __syncthreads();

    // 4. out[d] = reduce_add(8 lane chains) + the seq % 8 tail in order,
    // then the 32-group quantization of the output projection's input
    if (tid < kDecDims) {
        float lj[8];
#pragma unroll
        for (int j = 0; j < 8; j++) lj[j] = part[j * kDecDims + tid];
        // the tail's p values, all read before the first is used (pt rows
        // have PCS > n_chunks entries; p is normalized in place only on the
        // tile path)
        float pe[7];
#pragma unroll
        for (int i = 0; i < 7; i++) pe[i] = pt[i * PCS + n_chunks];
        float out = reduce_add8(lj);
#pragma unroll
        for (int i = 0; i < 7; i++) {
            const float sum = fadd(out, fmul(regpv ? fmul(pe[i], inv) : pe[i], vtail[i]));
            out = n_chunks * 8 + i < seq ? sum : out;
        }
        const size_t col = (size_t)h * HD + (size_t)ds * kDecDims + tid;
        if (att_f32) att_f32[col] = out;
        if constexpr (QF >= 0) {
            // (fmaxf keeps the larger non-NaN operand, so the order of the
            // 32-lane reduction does not matter)
            float am = group_max(fabsf(out), 32);
            am = fmaxf(am, 0.0f);
            const float s = group_scale<QF>(am);
            aq[col] = (int8_t)quant_one<QF>(out, s);
            if (tid == 0) as[col / kGroup] = s;
        }
    }
}

// ---------------------------------------------------------------------------
// Long contexts, head sizes 64 and 128, 2/4/8 query heads per kv head: the
// softmax and the P.V chains as three more kernels after k_attn_scores.
// Scratch after the scores: p transposed [n_heads][8][pcs] (p[8c + j] at
// (h*8 + j)*pcs + c, pcs = sc_ld / 8), then the lane partials
// [n_heads][HD][8].
// ---------------------------------------------------------------------------
constexpr int kPvRows = 64;     // V rows (one lane j) per LDS slot
constexpr int kPvSlots = 8;     // slots in flight

// Waits until at most n of this wavefront's vector memory operations are
// in flight (n < 64; the immediate must be a constant).
// Softmax of one head: max from -1e10, e = exp(score - max) into LDS (+0
// from seq to the next multiple of 64), the serial sum by the segmented sum
// of all 8 wavefronts (seg_serial_sum_wide), p = e * (1 / sum) written
// transposed for the P.V kernel.  LDS: el (attn_softmax_el_floats) | the
// sum's scratch.
__host__ __device__ inline int attn_softmax_el_floats(int sc_ld) { return ((sc_ld + 63) & ~63) + 64; }
constexpr int kSoftSumScratch = 16 * 64 + 8 + 2 * 8 + 4;   // ends, bases, float64 segment sums, counter
__global__ __launch_bounds__(kDecThreads) void k_attn_softmax(const StepState* __restrict__ st, int sc_ld,
                                                              int n_heads, float* __restrict__ scratch,
                                                              unsigned* __restrict__ fault) {
    extern __shared__ __align__(16) float el[];
    __shared__ float red[16];
    const int h = blockIdx.x, tid = threadIdx.x;
    float* sx = el + attn_softmax_el_floats(sc_ld);
    double* segsum = reinterpret_cast<double*>(sx + 16 * 64 + 8);
    int* sum_ctr = reinterpret_cast<int*>(segsum + 8);
    if (tid == 0) *sum_ctr = 0;   // (seen after the first barrier)
    const int seq = st->pos + 1, n_quads = (seq + 3) / 4;
    const float* __restrict__ sh = scratch + (size_t)h * sc_ld;
    float* __restrict__ pt = scratch + (size_t)n_heads * sc_ld + (size_t)h * sc_ld;   // [8][pcs] of this head
    const int pcs = sc_ld / 8;
    vf4 s4[kLongQuads];
#pragma unroll
    for (int i = 0; i < kLongQuads; i++) s4[i] = *reinterpret_cast<const vf4*>(sh + 4 * min(tid + i * kDecThreads, n_quads - 1));
    float lmax = -1e10f;
#pragma unroll
    for (int i = 0; i < kLongQuads; i++)
#pragma unroll
        for (int pp = 0; pp < 4; pp++)
            lmax = fmaxf(lmax, 4 * (tid + i * kDecThreads) + pp < seq ? s4[i][pp] : -1e10f);
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) red[tid >> 6] = lmax;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < kDecThreads / 64; w++) mx = fmaxf(mx, red[w]);
#pragma unroll
    for (int i = 0; i < kLongQuads; i++)
#pragma unroll
        for (int pp = 0; pp < 4; pp++) {
            const int p = 4 * (tid + i * kDecThreads) + pp;
            if (p < seq) el[p] = expf_rn(s4[i][pp] - mx);
        }
    for (int p = seq + tid; p < ((seq + 63) & ~63); p += kDecThreads) el[p] = 0.0f;
    __syncthreads();
    seg_sums_f64_wide<kDecThreads / 64>(el, seq, segsum);
    __syncthreads();
    {
        const float sum = seg_serial_sum_wide<kDecThreads / 64>(el, seq, segsum, sx, sum_ctr, 0, fault);
        if (tid == 0) red[8] = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = red[8];
    for (int p = tid; p < seq; p += kDecThreads) pt[(p & 7) * pcs + (p >> 3)] = fmul(el[p], inv);
}

// The same softmax for rows longer than LDS holds (contexts beyond 16384):
// the max over the scores row in global memory, e = exp(score - max) back
// into the row, the serial sum in segments of kSoftSeg values staged into
// LDS (double-buffered: the next segment is copied while wavefront 0 sums the
// current one, each segment continuing from the previous segment's sum),
// then p = e * (1 / sum) transposed as above.
constexpr int kSoftSeg = 6144;
__global__ __launch_bounds__(kDecThreads) void k_attn_softmax_long(const StepState* __restrict__ st, int sc_ld,
                                                                   int n_heads, float* __restrict__ scratch,
                                                                   unsigned* __restrict__ fault) {
    extern __shared__ __align__(16) float seg[];   // [2][kSoftSeg]
    __shared__ float red[16];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int seq = st->pos + 1;
    float* __restrict__ sh = scratch + (size_t)h * sc_ld;
    float* __restrict__ pt = scratch + (size_t)n_heads * sc_ld + (size_t)h * sc_ld;
    const int pcs = sc_ld / 8;
    float lmax = -1e10f;
    for (int p = tid; p < seq; p += kDecThreads) lmax = fmaxf(lmax, sh[p]);
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) red[tid >> 6] = lmax;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < kDecThreads / 64; w++) mx = fmaxf(mx, red[w]);
    for (int p = tid; p < seq; p += kDecThreads) sh[p] = expf_rn(sh[p] - mx);
    __syncthreads();   // (the row's e values, written by every wavefront)
    const int nseg = (seq + kSoftSeg - 1) / kSoftSeg;
    auto stage = [&](int k) {
        float* d = seg + (k & 1) * kSoftSeg;
        const int b = k * kSoftSeg, n = min(kSoftSeg, seq - b);
        for (int i = tid; i < n; i += kDecThreads) d[i] = sh[b + i];
    };
    stage(0);
    __syncthreads();
    float sum = 0.0f;
    for (int k = 0; k < nseg; k++) {
        if (k + 1 < nseg) stage(k + 1);
        if (tid < 64) {
            const float* d = seg + (k & 1) * kSoftSeg;
            sum = wave_serial_sum(d, min(kSoftSeg, seq - k * kSoftSeg), sum);
        }
        __syncthreads();   // segment k summed and segment k + 1 staged
    }
    if (tid == 0) red[8] = sum > 0.0f ? 1.0f / sum : 0.0f;
    __syncthreads();
    const float inv = red[8];
    for (int p = tid; p < seq; p += kDecThreads) pt[(p & 7) * pcs + (p >> 3)] = fmul(sh[p], inv);
}

// P.V chains of one lane j: workgroup (kv head g, 64-dimension part, j),
// wavefront w = query head g*r + w, lane = dimension.  p[8c + j] is the same
// for the whole wavefront (scalar loads); V rows 8c + j (256 bytes of the
// part) stream through an LDS ring of kPvSlots slots of kPvRows rows, every
// wavefront issuing 16/r of each slot's 16 DMA instructions.
template <int HD, int R>
__global__ __launch_bounds__(64 * R) void k_attn_pv_j(const float* __restrict__ vc, const StepState* __restrict__ st,
                                                      int n_heads, int n_kv_heads, int sc_ld,
                                                      float* __restrict__ scratch) {
    extern __shared__ __align__(16) float ring[];   // [kPvSlots][kPvRows][64] V, then [kPvSlots][R][64] p
    static_assert(kPvRows == 64 && kPvSlots == 8 && 16 % R == 0, "one p per lane and slot");
    constexpr int NP = HD / 64;
    constexpr int DPW = 16 / R + 1;   // DMA instructions per wavefront and slot: V rows, then p
    const int g = blockIdx.x / NP, part = blockIdx.x % NP, j = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = g * R + wave;
    const int kv_dim = n_kv_heads * HD;
    const int seq = st->pos + 1, n_chunks = seq / 8;
    const int pcs = sc_ld / 8;
    const float* __restrict__ ph = scratch + (size_t)n_heads * sc_ld + ((size_t)h * 8 + j) * pcs;
    const float* __restrict__ vcol = vc + (size_t)g * HD + part * 64;
    float* __restrict__ pring = ring + kPvSlots * kPvRows * 64;
    const int n_slots = (n_chunks + kPvRows - 1) / kPvRows;
    // slot sl: V rows c = sl*kPvRows + 4*k + (lane >> 4), k = wave + R*i, 16-byte
    // piece lane & 15; p of chunk sl*kPvRows + lane for this wavefront's head
    auto dma = [&](int sl) {
        float* dst = ring + (sl % kPvSlots) * kPvRows * 64;
#pragma unroll
        for (int i = 0; i < 16 / R; i++) {
            const int k = wave + R * i;
            const int c = min(sl * kPvRows + 4 * k + (lane >> 4), n_chunks - 1);
            __builtin_amdgcn_global_load_lds(vcol + (size_t)(8 * c + j) * kv_dim + (lane & 15) * 4,
                                             dst + k * 4 * 64, 16, 0, 0);
        }
        __builtin_amdgcn_global_load_lds(ph + min(sl * kPvRows + lane, n_chunks - 1),
                                         pring + ((sl % kPvSlots) * R + wave) * 64, 4, 0, 0);
    };
    for (int sl = 0; sl < n_slots && sl < kPvSlots; sl++) dma(sl);
    float acc = 0.0f;
    for (int sl = 0; sl < n_slots; sl++) {
        wait_vm_slots<DPW>(min(kPvSlots - 1, n_slots - 1 - sl));
        lds_barrier();   // every wavefront's DMA of slot sl
        const float* tile = ring + (sl % kPvSlots) * kPvRows * 64;
        const float* prow = pring + ((sl % kPvSlots) * R + wave) * 64;
        const int steps = min(kPvRows, n_chunks - sl * kPvRows);
        if (steps == kPvRows) {
            // groups of 8 steps: the next group's V (4 two-row reads) and p
            // (2 broadcast reads) are issued before this group's 16 VALU ops,
            // so each LDS latency hides under the previous group.  The reads
            // are inline assembly with explicit waits: the compiler counts
            // the LDS DMA above as a pending flat access and would otherwise
            // wait for every LDS read at each use.
            const unsigned va = lds_addr(tile + lane), pa = lds_addr(prow);
            vf2 vr[2][4];
            vf4 pr[2][2];
#define YL_PV_LOAD(gi, b)                                                                                       \
            vr[b][0] = lds_read2st64<8 * (gi)>(va); vr[b][1] = lds_read2st64<8 * (gi) + 2>(va);                 \
            vr[b][2] = lds_read2st64<8 * (gi) + 4>(va); vr[b][3] = lds_read2st64<8 * (gi) + 6>(va);             \
            pr[b][0] = lds_read_b128<32 * (gi)>(pa); pr[b][1] = lds_read_b128<32 * (gi) + 16>(pa);
#define YL_PV_STEP(gi, n)                                                                                       \
            {                                                                                                   \
                constexpr int b = (gi) & 1;                                                                     \
                lgkm_wait_tie<n>(vr[b][0], vr[b][1], vr[b][2], vr[b][3], pr[b][0], pr[b][1]);                   \
                _Pragma("unroll") for (int k = 0; k < 8; k++)                                                   \
                    acc = fadd(acc, fmul(pr[b][k >> 2][k & 3], vr[b][k >> 1][k & 1]));                          \
            }
            YL_PV_LOAD(0, 0)
            YL_PV_LOAD(1, 1) YL_PV_STEP(0, 6)
            YL_PV_LOAD(2, 0) YL_PV_STEP(1, 6)
            YL_PV_LOAD(3, 1) YL_PV_STEP(2, 6)
            YL_PV_LOAD(4, 0) YL_PV_STEP(3, 6)
            YL_PV_LOAD(5, 1) YL_PV_STEP(4, 6)
            YL_PV_LOAD(6, 0) YL_PV_STEP(5, 6)
            YL_PV_LOAD(7, 1) YL_PV_STEP(6, 6)
            YL_PV_STEP(7, 0)
#undef YL_PV_LOAD
#undef YL_PV_STEP
            static_assert(kPvRows == 64, "8 groups of 8 rows");
        } else {
            for (int i = 0; i < steps; i++) acc = fadd(acc, fmul(prow[i], tile[i * 64 + lane]));
        }
        if (sl + kPvSlots < n_slots) {
            lds_barrier();   // slot consumed before it is refilled
            dma(sl + kPvSlots);
        }
    }
    float* __restrict__ lp = scratch + (size_t)n_heads * sc_ld * 2;
    lp[((size_t)h * HD + part * 64 + lane) * 8 + j] = acc;
}

// out[d] = reduce_add8(lane partials) + the seq % 8 tail in order, then the
// 32-group quantization of the output projection's input.
template <int QF, int HD>
__global__ __launch_bounds__(HD) void k_attn_pv_out(const float* __restrict__ vc, const StepState* __restrict__ st,
                                                    int n_heads, int n_kv_heads, int sc_ld,
                                                    const float* __restrict__ scratch, int8_t* __restrict__ aq,
                                                    float* __restrict__ as, float* __restrict__ att_f32) {
    const int h = blockIdx.x, d = threadIdx.x;
    const int kvh = h / (n_heads / n_kv_heads), kv_dim = n_kv_heads * HD;
    const int seq = st->pos + 1, n_chunks = seq / 8, pcs = sc_ld / 8;
    const float* __restrict__ lp = scratch + (size_t)n_heads * sc_ld * 2 + ((size_t)h * HD + d) * 8;
    float lj[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) lj[jj] = lp[jj];
    float out = reduce_add8(lj);
    const float* __restrict__ pt = scratch + (size_t)n_heads * sc_ld + (size_t)h * 8 * pcs;
    for (int i = 0; n_chunks * 8 + i < seq; i++)
        out = fadd(out, fmul(pt[i * pcs + n_chunks], vc[(size_t)(n_chunks * 8 + i) * kv_dim + kvh * HD + d]));
    const size_t col = (size_t)h * HD + d;
    if (att_f32) att_f32[col] = out;
    if constexpr (QF >= 0) {
        float am = fabsf(out);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 32));
        am = fmaxf(am, 0.0f);
        const float sc = group_scale<QF>(am);
        aq[col] = (int8_t)quant_one<QF>(out, sc);
        if ((d & 31) == 0) as[col / kGroup] = sc;
    }
}

// ---------------------------------------------------------------------------
// Prompt batches: one workgroup per (query head, token); seq_len = pos +
// batch, the token's own position pos + t, later positions masked to -1e10.
// LDS: scores seq_len | q head_size | partials 8*head_size | out head_size.
// ---------------------------------------------------------------------------
template <int QF>
__global__ __launch_bounds__(kAttnThreads) void k_attention(const float* __restrict__ sq,
                                                            const float* __restrict__ kc,
                                                            const float* __restrict__ vc,
                                                            const StepState* __restrict__ st, int batch,
                                                            int kv_ld, int n_heads, int n_kv_heads, int hd,
                                                            float attn_scale, int8_t* __restrict__ aq,
                                                            float* __restrict__ as,
                                                            float* __restrict__ att_f32) {
    extern __shared__ __align__(16) float lds_f[];
    __shared__ float red[8];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int pos0 = st->pos;
    const int seq_len = pos0 + batch;
    const int abs_pos = pos0 + t;
    const int max_t2 = abs_pos < seq_len - 1 ? abs_pos : seq_len - 1;
    const int kvh = h / (n_heads / n_kv_heads);
    const int kv_dim = n_kv_heads * hd;
    const int att_dim = n_heads * hd;
    float* sc = lds_f;
    float* ql = sc + ((seq_len + 3) & ~3);
    float* part = ql + hd;
    float* outl = part + 8 * hd;

    for (int i = tid; i < hd; i += kAttnThreads) ql[i] = sq[(size_t)t * att_dim + (size_t)h * hd + i];
    __syncthreads();
    float lmax = -1e10f;
    const int n_simd = hd / 8;
    for (int t2 = tid; t2 <= max_t2; t2 += kAttnThreads) {
        // keys transposed: dimension i of position t2 at kt[i * kv_ld]
        const float* kt = kc + (size_t)kvh * hd * kv_ld + t2;
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int s = 0; s < n_simd; s++) {
            const float* q = ql + s * 8;
#pragma unroll
            for (int j = 0; j < 8; j++) l[j] = fadd(l[j], fmul(q[j], kt[(size_t)(8 * s + j) * kv_ld]));
        }
        const float sv = fmul(reduce_add8(l), attn_scale);
        sc[t2] = sv;
        lmax = fmaxf(lmax, sv);
    }
    for (int t2 = max_t2 + 1 + tid; t2 < seq_len; t2 += kAttnThreads) sc[t2] = -1e10f;
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) red[tid >> 6] = lmax;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < kAttnThreads / 64; w++) mx = fmaxf(mx, red[w]);
    for (int t2 = tid; t2 < seq_len; t2 += kAttnThreads) sc[t2] = expf_rn(sc[t2] - mx);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        int t2 = 0;
        for (; t2 + 4 <= seq_len; t2 += 4) {
            const float4 e4 = *reinterpret_cast<const float4*>(sc + t2);
            sum = fadd(sum, e4.x);
            sum = fadd(sum, e4.y);
            sum = fadd(sum, e4.z);
            sum = fadd(sum, e4.w);
        }
        for (; t2 < seq_len; t2++) sum = fadd(sum, sc[t2]);
        red[4] = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = red[4];
    for (int t2 = tid; t2 < seq_len; t2 += kAttnThreads) sc[t2] = fmul(sc[t2], inv);
    __syncthreads();
    const int n_chunks = seq_len / 8;
    const float* vbase = vc + (size_t)kvh * hd;
    for (int ch = tid; ch < 8 * hd; ch += kAttnThreads) {
        const int d = ch % hd, j = ch / hd;
        float l = 0.0f;
        const float* vp = vbase + (size_t)j * kv_dim + d;
#pragma unroll 8
        for (int cc = 0; cc < n_chunks; cc++) l = fadd(l, fmul(sc[8 * cc + j], vp[(size_t)(8 * cc) * kv_dim]));
        part[j * hd + d] = l;
    }
    __syncthreads();
    for (int d = tid; d < hd; d += kAttnThreads) {
        float l[8];
#pragma unroll
        for (int j = 0; j < 8; j++) l[j] = part[j * hd + d];
        float sum = reduce_add8(l);
        for (int t2 = n_chunks * 8; t2 < seq_len; t2++)
            sum = fadd(sum, fmul(sc[t2], vbase[(size_t)t2 * kv_dim + d]));
        outl[d] = sum;
        if (att_f32) att_f32[(size_t)t * att_dim + (size_t)h * hd + d] = sum;
    }
    __syncthreads();
    if constexpr (QF >= 0)
        quantize_head_output<QF>(outl, hd, aq, as, (size_t)t * (att_dim / kGroup) + ((size_t)h * hd) / kGroup);
}

static size_t attention_lds_bytes(int seq_len, int head_size) {
    return ((size_t)((seq_len + 3) & ~3) + 10 * (size_t)head_size) * sizeof(float);
}
bool attention_row_fits(int seq_len, int head_size) { return attention_lds_bytes(seq_len, head_size) <= 60 * 1024; }

hipError_t launch_attention(const float* sq, const float* kc, const float* vc, const StepState* st, int batch,
                            int max_seq, int kv_ld, int n_heads, int n_kv_heads, int head_size, float scale, int qfmt,
                            int8_t* aq, float* as, float* att_f32, hipStream_t s) {
    // max_seq: the seq_len of this call (LDS holds its score row)
    if (!attention_row_fits(max_seq, head_size)) return hipErrorInvalidValue;
    const size_t smem = attention_lds_bytes(max_seq, head_size);
    const dim3 grid(n_heads, batch);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_attention<kQ8>), grid, dim3(kAttnThreads), smem, s, sq, kc, vc, st, batch, kv_ld,
                           n_heads, n_kv_heads, head_size, scale, aq, as, att_f32);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_attention<kQ4>), grid, dim3(kAttnThreads), smem, s, sq, kc, vc, st, batch, kv_ld,
                           n_heads, n_kv_heads, head_size, scale, aq, as, att_f32);
    else
        hipLaunchKernelGGL((k_attention<-1>), grid, dim3(kAttnThreads), smem, s, sq, kc, vc, st, batch, kv_ld,
                           n_heads, n_kv_heads, head_size, scale, aq, as, att_f32);
    return hipGetLastError();
}

size_t attn_decode_lds_bytes(int max_seq) { return attn_decode_lds_floats(max_seq) * sizeof(float); }

bool attn_decode_split(int max_seq) { return max_seq > kAttnSplitSeq; }
// Head size 64 or 128 with 2, 4 or 8 query heads per kv head runs the
// four-kernel path, whose softmax streams rows of any length; every other
// layout keeps the scores row of the decode kernel in LDS (16384 positions).
int attn_decode_limit(int n_heads, int n_kv_heads, int head_size) {
    const int r = n_kv_heads > 0 ? n_heads / n_kv_heads : 0;
    if ((head_size == 64 || head_size == 128) && (r == 2 || r == 4 || r == 8)) return 0x7fffffff;
    return kLongQuads * 4 * kDecThreads;
}
bool attn_decode_fits(int max_seq, int n_heads, int n_kv_heads, int head_size) {
    return attn_v_tiles(max_seq < kAttnSplitSeq ? max_seq : kAttnSplitSeq) >= 2 &&
           max_seq <= attn_decode_limit(n_heads, n_kv_heads, head_size);
}
static int attn_scores_ld(int max_seq) { return (max_seq + 127) & ~127; }
// scores [n_heads][sc_ld], p [n_heads][8][sc_ld / 8], lane partials
// [n_heads][128][8]
size_t attn_scores_bytes(int n_heads, int max_seq) {
    return attn_decode_split(max_seq)
               ? (size_t)n_heads * (2 * (size_t)attn_scores_ld(max_seq) + 128 * 8) * sizeof(float)
               : 0;
}

template <class K>
static hipError_t opt_in_lds(K* kern, size_t smem) {
    if (smem <= 60 * 1024) return hipSuccess;
    // more than the default 64 KiB of LDS with the static part
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)smem);
}

template <int QF, int HD>
static hipError_t launch_attn_decode_k(const float* sq, const float* kc, const float* vc, const StepState* st,
                                       int max_seq, int kv_ld, int n_heads, int n_kv_heads, float scale, int8_t* aq,
                                       float* as, float* att_f32, float* sc, hipStream_t s) {
    const dim3 grid(n_heads * (HD / kDecDims));
    if (max_seq > attn_decode_limit(n_heads, n_kv_heads, HD)) return hipErrorInvalidValue;
    if (attn_decode_split(max_seq)) {
        if (!sc) return hipErrorInvalidValue;   // the scores scratch of long contexts
        const int r = n_heads / n_kv_heads;
        const size_t smem_s = (size_t)r * 8 * kScoreRows * sizeof(float);
        if (smem_s > kDecLdsBudget) return hipErrorInvalidValue;
        const int sc_ld = attn_scores_ld(max_seq);
        hipError_t e = opt_in_lds(&k_attn_scores<HD>, smem_s);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((k_attn_scores<HD>), dim3(n_kv_heads, (max_seq + kScoreRows - 1) / kScoreRows),
                           dim3(kDecThreads), smem_s, s, sq, kc, st, n_heads, n_kv_heads, scale, kv_ld, sc, sc_ld);
        if constexpr (HD >= 64) if (r == 2 || r == 4 || r == 8) {
            // softmax, P.V by lane j, output
            // (rows up to 16384 positions are held in LDS whole)
            const bool long_row = max_seq > kLongQuads * 4 * kDecThreads;
            const size_t smem_e = long_row ? 2 * (size_t)kSoftSeg * sizeof(float)
                                           : ((size_t)attn_softmax_el_floats(sc_ld) + kSoftSumScratch) * sizeof(float);
            const size_t smem_r = (size_t)kPvSlots * (kPvRows + r) * 64 * sizeof(float);
            auto pv = r == 2 ? &k_attn_pv_j<HD, 2> : r == 4 ? &k_attn_pv_j<HD, 4> : &k_attn_pv_j<HD, 8>;
            auto softmax = long_row ? &k_attn_softmax_long : &k_attn_softmax;
            e = opt_in_lds(softmax, smem_e);
            if (e == hipSuccess) e = opt_in_lds(pv, smem_r);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL(softmax, dim3(n_heads), dim3(kDecThreads), smem_e, s, st, sc_ld, n_heads, sc,
                               wait_fault_word(false));
            hipLaunchKernelGGL(pv, dim3(n_kv_heads * (HD / 64), 8), dim3(64 * r), smem_r, s, vc, st, n_heads,
                               n_kv_heads, sc_ld, sc);
            hipLaunchKernelGGL((k_attn_pv_out<QF, HD>), dim3(n_heads), dim3(HD), 0, s, vc, st, n_heads, n_kv_heads,
                               sc_ld, sc, aq, as, att_f32);
            return hipGetLastError();
        }
        // other layouts: the decode kernel reads the scores row back into LDS
        const int n_vt = attn_v_tiles(max_seq);
        if (n_vt < 2) return hipErrorInvalidValue;
        const size_t smem = attn_decode_lds_bytes(max_seq);
        e = opt_in_lds(&k_attn_decode<QF, HD, true>, smem);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((k_attn_decode<QF, HD, true>), grid, dim3(kDecThreads), smem, s, sq, kc, vc, st, n_heads,
                           n_kv_heads, scale, max_seq, kv_ld, n_vt, aq, as, att_f32, sc, sc_ld, nullptr);
        return hipGetLastError();
    }
    const int n_vt = attn_v_tiles(max_seq);
    if (n_vt < 2) return hipErrorInvalidValue;
    const size_t smem = attn_decode_lds_bytes(max_seq);
    const hipError_t e = opt_in_lds(&k_attn_decode<QF, HD, false>, smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_attn_decode<QF, HD, false>), grid, dim3(kDecThreads), smem, s, sq, kc, vc, st, n_heads,
                       n_kv_heads, scale, max_seq, kv_ld, n_vt, aq, as, att_f32, nullptr, 0, wait_fault_word(false));
    return hipGetLastError();
}

template <int QF>
static hipError_t launch_attn_decode_q(const float* sq, const float* kc, const float* vc, const StepState* st,
                                       int max_seq, int kv_ld, int n_heads, int n_kv_heads, int hd, float scale,
                                       int8_t* aq, float* as, float* att_f32, float* sc, hipStream_t s) {
    switch (hd) {
    case 32: return launch_attn_decode_k<QF, 32>(sq, kc, vc, st, max_seq, kv_ld, n_heads, n_kv_heads, scale, aq, as, att_f32, sc, s);
    case 64: return launch_attn_decode_k<QF, 64>(sq, kc, vc, st, max_seq, kv_ld, n_heads, n_kv_heads, scale, aq, as, att_f32, sc, s);
    case 128: return launch_attn_decode_k<QF, 128>(sq, kc, vc, st, max_seq, kv_ld, n_heads, n_kv_heads, scale, aq, as, att_f32, sc, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_decode(const float* sq, const float* kc, const float* vc, const StepState* st, int max_seq,
                              int kv_ld, int n_heads, int n_kv_heads, int head_size, float scale, int qfmt, int8_t* aq,
                              float* as, float* att_f32, float* sc, hipStream_t s) {
    if (kv_ld % 4 || kv_ld < max_seq) return hipErrorInvalidValue;
    if (qfmt == kQ8)
        return launch_attn_decode_q<kQ8>(sq, kc, vc, st, max_seq, kv_ld, n_heads, n_kv_heads, head_size, scale, aq,
                                         as, att_f32, sc, s);
    if (qfmt == kQ4)
        return launch_attn_decode_q<kQ4>(sq, kc, vc, st, max_seq, kv_ld, n_heads, n_kv_heads, head_size, scale, aq,
                                         as, att_f32, sc, s);
    return launch_attn_decode_q<-1>(sq, kc, vc, st, max_seq, kv_ld, n_heads, n_kv_heads, head_size, scale, aq, as,
                                    att_f32, sc, s);
}

}  // namespace yl
