// yl_gemv.hip -- quantized GEMV / batched matvec (weight_type.rs:122-226)
// with the neighbouring elementwise work of forward.rs fused in.
//
// Workgroup layout: wavefronts 0..NA-1 are activation wavefronts (NA = 4
// with an RMSNorm prologue, else 1); the rest are weight wavefronts.  Each
// weight wavefront owns RW consecutive
// output rows of one batch row (blockIdx.y) and every block of them:
//   lane l works on row r = l / LPR, blocks b = k*LPR + l % LPR for slots
//   k = 0..PPL-1 (LPR lanes per row, RW = 64/LPR rows per wavefront),
// so slot k covers the same block range [k*LPR, (k+1)*LPR) of every row.
//
// 1. The activation wavefronts issue their loads first; after one barrier
//    each weight wavefront issues the loads of its first LA slots (two
//    16-byte loads per Q8_0 block or one per Q4_0 block, plus the f16 scale,
//    through buffer descriptors: one VGPR offset per lane, slot offsets in
//    scalar registers) and waits for the activation row.
// 2. The activation wavefronts (no weight loads) stage the row in LDS:
//    either the already quantized row (LDS DMA), or -- for the QKV and
//    gate/up matmuls -- RMSNorm + quantize of the f32 residual stream (in
//    layer 0, of the token's embedding row), shared by four wavefronts.
//    They also stage the values the rows' sums start from (K/V cache entries
//    for the `+=` columns) and the RoPE angles, then count themselves done
//    in an LDS counter.  No further workgroup barrier is involved: a barrier
//    would complete only once every wavefront has issued its loads, which
//    under full HBM load is most of the kernel.
// 3. Per slot, as its loads land: each lane's exact int32 block dot
//    (v_dot4_i32_i8) becomes the f32 term ((float)isum * w_scale) * x_scale,
//    and the row's first lane adds the slot's terms of its row in block
//    order onto the row's accumulator, reading lane j's term through DPP
//    (row_shl:j), or by readlane when a row spans the wavefront -- the
//    reference's `xout += term` sequence, so every output is bit-identical
//    to matmul_q8_slices.  The sums advance while later
//    slots are in flight; the loads of slot k + LA go out after slot k.
// 4. Epilogues: residual add (WO, W2), RoPE + K/V cache (QKV), SwiGLU +
//    quantize of h (gate/up; the only cross-wavefront step, after one
//    workgroup barrier at the end), or a plain store.
//
// Q4_0 weights keep the reference nibble order (low nibble of byte j is
// element 2j, high nibble 2j+1, unsigned 0..15); the activation row is
// staged with each 8-group reordered to (even, odd) elements so that
// (w & 0x0f0f0f0f) and ((w >> 4) & 0x0f0f0f0f) dot against it directly.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

__device__ __forceinline__ uint2 q4_reorder8(uint2 v) {
    const uint32_t ev = (v.x & 0xffu) | ((v.x >> 8) & 0xff00u) | ((v.y & 0xffu) << 16) |
                        ((v.y << 8) & 0xff000000u);
    const uint32_t od = ((v.x >> 8) & 0xffu) | ((v.x >> 16) & 0xff00u) | ((v.y << 8) & 0xff0000u) |
                        (v.y & 0xff000000u);
    return make_uint2(ev, od);
}

template <int WF>
struct WBlock;
template <>
struct WBlock<kQ8> { uint4 a, b; };
template <>
struct WBlock<kQ4> { uint4 a; };
template <>
struct WBlock<kQ8S> { uint4 a, b; };
template <>
struct WBlock<kQ8S64> { uint4 a, b; };
template <>
struct WBlock<kQ8S128> { uint4 a, b; };

// 32-blocks per scale group of a weight format
template <int WF>
constexpr int blocks_per_group() { return WF == kQ8S64 ? 2 : (WF == kQ8S128 ? 4 : 1); }

// The activation format of a weight format (Q8 rows with f32 block scales
// dot against the same 32-groups as Q8_0).
template <int WF>
constexpr int act_fmt() { return WF == kQ4 ? kQ4 : kQ8; }

// Block scales: f16 words (Q8_0, Q4_0) or f32 (kQ8S).
template <int WF>
struct ScaleWord { using type = uint16_t; };
template <>
struct ScaleWord<kQ8S> { using type = float; };
template <>
struct ScaleWord<kQ8S64> { using type = float; };
template <>
struct ScaleWord<kQ8S128> { using type = float; };

constexpr int kBufRaw = 0x00020000;   // buffer descriptor word 3: raw 32-bit data

// A buffer descriptor built from values the compiler must keep in scalar
// registers (a descriptor in vector registers turns every load into a
// readfirstlane loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, int bytes) {
    const uint64_t p = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    void* q = (void*)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(q, (short)0, __builtin_amdgcn_readfirstlane(bytes), kBufRaw);
}

// Weights are read once per token, so they are loaded non-temporally
// (cache policy `nt`): a decode step streams over a gigabyte of weights, and
// loads that allocate normally would evict from the L2s and the 256 MiB
// Infinity Cache the small data every kernel waits on -- its kernel
// arguments, the step state, the activation rows, the KV cache.
constexpr int kPolStream = 2;   // buffer load aux bit 1: nt

__device__ __forceinline__ uint4 buf_u4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kPolStream));
}

// The 16-byte pieces of a lane's slot: for 32-byte blocks, at voff and
// voff + HB.  The weight wavefronts use HB = 16 * LPR: the LPR lanes of a
// row then read 16 * LPR contiguous bytes per instruction (whole cache
// lines), each lane one half of two blocks (see half_dot).
template <int WF, int HB>
__device__ __forceinline__ void load_block(WBlock<WF>& w, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
    if constexpr (WF != kQ4) {
        w.a = buf_u4(r, voff, soff);
        w.b = buf_u4(r, voff + HB, soff);
    } else {
        w.a = buf_u4(r, voff, soff);
    }
}

// Exact int32 dot of one 16-byte half block with its 16 activations.
__device__ __forceinline__ int half_dot(uint4 w, const int32_t* xw) {
    int a = __builtin_amdgcn_sdot4((int)w.x, xw[0], 0, false);
    a = __builtin_amdgcn_sdot4((int)w.y, xw[1], a, false);
    a = __builtin_amdgcn_sdot4((int)w.z, xw[2], a, false);
    return __builtin_amdgcn_sdot4((int)w.w, xw[3], a, false);
}

// Exact int32 dot of one block (|sum| < 2^24, integer adds in any order):
// two independent v_dot4 chains of four, then one add.
template <int WF>
__device__ __forceinline__ int block_dot(const WBlock<WF>& w, const int32_t* xw) {
    int a0 = 0, a1 = 0;
    if constexpr (WF != kQ4) {
        a0 = __builtin_amdgcn_sdot4((int)w.a.x, xw[0], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)w.b.x, xw[4], a1, false);
        a0 = __builtin_amdgcn_sdot4((int)w.a.y, xw[1], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)w.b.y, xw[5], a1, false);
        a0 = __builtin_amdgcn_sdot4((int)w.a.z, xw[2], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)w.b.z, xw[6], a1, false);
        a0 = __builtin_amdgcn_sdot4((int)w.a.w, xw[3], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)w.b.w, xw[7], a1, false);
    } else {
        const uint32_t m = 0x0f0f0f0fu;
        a0 = __builtin_amdgcn_sdot4((int)(w.a.x & m), xw[0], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)(w.a.z & m), xw[4], a1, false);
        a0 = __builtin_amdgcn_sdot4((int)((w.a.x >> 4) & m), xw[1], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)((w.a.z >> 4) & m), xw[5], a1, false);
        a0 = __builtin_amdgcn_sdot4((int)(w.a.y & m), xw[2], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)(w.a.w & m), xw[6], a1, false);
        a0 = __builtin_amdgcn_sdot4((int)((w.a.y >> 4) & m), xw[3], a0, false);
        a1 = __builtin_amdgcn_sdot4((int)((w.a.w >> 4) & m), xw[7], a1, false);
    }
    return a0 + a1;
}

constexpr int kMaxWeightWaves = 8;
constexpr int kNormWaves = 4;         // activation wavefronts of the RMSNorm kernels
constexpr int kGemvMaxThreads = 64 * (kMaxWeightWaves + kNormWaves);

// ----------------------------------------------------------- LDS layout ----
// act row   : n bytes (int8, Q4 8-groups reordered), rounded up to 1 KiB
//             (whole LDS DMA rows)
// act scales: nb floats, rounded up to 1 KiB
// sync      : 4 ints (counters of the activation wavefronts, ss)
// init      : R floats (the value each row's sum starts from)
// outs      : R floats (finished sums, for the SwiGLU step)
// rope      : 2R floats + 4 (the QKV epilogue's angles and position)
// norm      : 8 transposed chain rows of squares (RMSNorm kernels only)
struct GemvLds {
    size_t act, scales, sync, init, outs, rope, norm, total;
};
__host__ __device__ inline GemvLds gemv_lds(int n, int nb, int R, bool norm) {
    GemvLds l{};
    size_t o = 0;
    l.act = o;
    o += ((size_t)n + 1023) & ~(size_t)1023;
    l.scales = o;
    o += ((size_t)nb * 4 + 1023) & ~(size_t)1023;
    l.sync = o;
    o += 16;
    l.init = o;
    o += (size_t)R * 4;
    l.outs = o;
    o += (size_t)R * 4;
    l.rope = o;
    o += (size_t)R * 8 + 16;
    o = (o + 15) & ~(size_t)15;
    l.norm = o;
    if (norm) o += (size_t)8 * rowq_stride(n) * 4;
    l.total = o;
    return l;
}

// `bytes` bytes from global memory into LDS by LDS DMA: EB bytes per lane
// (16 or 4), 64*EB bytes per instruction.  `bytes` is a multiple of EB and
// src is EB-aligned; lanes past the end re-read the last EB bytes into the
// padding of the region (rounded up to 64*EB).  No registers hold the data,
// so no wait is implied; the caller waits (wait_vm_all) before reading it.
template <int EB>
__device__ __forceinline__ void dma_bytes(void* dst, const void* src, int bytes) {
    const int lane = threadIdx.x & 63;
    const uint8_t* s8 = reinterpret_cast<const uint8_t*>(src);
    uint8_t* d8 = reinterpret_cast<uint8_t*>(dst);
    for (int j = 0; j * 64 * EB < bytes; j++) {
        const int e = min(j * 64 * EB + lane * EB, bytes - EB);
        if constexpr (EB == 16) __builtin_amdgcn_global_load_lds(s8 + e, d8 + j * 64 * EB, 16, 0, 0);
        else __builtin_amdgcn_global_load_lds(s8 + e, d8 + j * 64 * EB, 4, 0, 0);
    }
}

// acc + v with v taken from lane (this lane + I) of the same 16-lane row.
template <int I>
__device__ __forceinline__ float add_from_lane_plus(float acc, float v) {
    if constexpr (I == 0) return fadd(acc, v);
    else return fadd(acc, dpp_zero<0x100 + I, 0xF>(v));   // row_shl:I
}

// The lane (of a row's LPR) that holds the term of the slot's block I: lane
// I, or with split halves (SPLIT) lane 2I for the slot's first LPR/2 blocks
// and lane 2(I - LPR/2) + 1 for the others.
template <int LPR, bool SPLIT, int I>
constexpr int term_lane() {
    return !SPLIT ? I : (I < LPR / 2 ? 2 * I : 2 * (I - LPR / 2) + 1);
}

// Chain step of one slot (LPR <= 16): the row's first lane adds the slot's
// terms of its row in block order, reading block I's term by
// row_shl:term_lane(I).
template <int LPR, bool SPLIT, int I = 0>
__device__ __forceinline__ float chain_slot_full(float acc, float term) {
    if constexpr (I < LPR)
        return chain_slot_full<LPR, SPLIT, I + 1>(add_from_lane_plus<term_lane<LPR, SPLIT, I>()>(acc, term), term);
    else return acc;
}
// The same for the row's last, partial slot: `valid` (< LPR) terms.
template <int LPR, bool SPLIT, int I = 0>
__device__ __forceinline__ float chain_slot_part(float acc, float term, int valid) {
    if constexpr (I < LPR) {
        if (I >= valid) return acc;
        return chain_slot_part<LPR, SPLIT, I + 1>(add_from_lane_plus<term_lane<LPR, SPLIT, I>()>(acc, term), term,
                                                  valid);
    } else {
        return acc;
    }
}
template <int LPR, bool SPLIT>
__device__ __forceinline__ float chain_slot_dpp(float acc, float term, int first_block, int nb) {
    const int valid = nb - first_block;   // uniform
    if (valid >= LPR) return chain_slot_full<LPR, SPLIT>(acc, term);
    if (valid <= 0) return acc;
    return chain_slot_part<LPR, SPLIT>(acc, term, valid);
}
// The same for groups of G blocks: a group's term sits on the lane of its
// first block, so the chain reads the lanes of blocks 0, G, 2G, ...
// (`valid` counts blocks; nb is a multiple of G).
template <int LPR, bool SPLIT, int G, int I = 0>
__device__ __forceinline__ float chain_slot_fullg(float acc, float term) {
    if constexpr (I < LPR)
        return chain_slot_fullg<LPR, SPLIT, G, I + G>(add_from_lane_plus<term_lane<LPR, SPLIT, I>()>(acc, term),
                                                      term);
    else return acc;
}
template <int LPR, bool SPLIT, int G, int I = 0>
__device__ __forceinline__ float chain_slot_partg(float acc, float term, int valid) {
    if constexpr (I < LPR) {
        if (I >= valid) return acc;
        return chain_slot_partg<LPR, SPLIT, G, I + G>(add_from_lane_plus<term_lane<LPR, SPLIT, I>()>(acc, term),
                                                      term, valid);
    } else {
        return acc;
    }
}
template <int LPR, bool SPLIT, int G>
__device__ __forceinline__ float chain_slot_dppg(float acc, float term, int first_block, int nb) {
    const int valid = nb - first_block;   // uniform
    if (valid >= LPR) return chain_slot_fullg<LPR, SPLIT, G>(acc, term);
    if (valid <= 0) return acc;
    return chain_slot_partg<LPR, SPLIT, G>(acc, term, valid);
}

// Chain step of one slot when a row spans the whole wavefront (LPR = 64):
// each term in block order by readlane, added in every lane (the row's sum
// is the same in all 64).  valid (uniform) terms of a partial slot.
__device__ __forceinline__ float lane_term(float term, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, term), l));
}
// (the scheduler issues each term's readlane two adds ahead of its use)
template <bool SPLIT, int B, int I = 0>
__device__ __forceinline__ void wave_terms16_at(float (&v)[16], float term) {
    if constexpr (I < 16) {
        v[I] = lane_term(term, term_lane<64, SPLIT, B + I>());
        wave_terms16_at<SPLIT, B, I + 1>(v, term);
    }
}
template <bool SPLIT, int G = 0>
__device__ __forceinline__ float chain_wave_full(float acc, float term) {
    if constexpr (G < 4) {
        float v[16];
        wave_terms16_at<SPLIT, 16 * G>(v, term);
#pragma unroll
        for (int i = 0; i < 16; i++) acc = fadd(acc, v[i]);
        return chain_wave_full<SPLIT, G + 1>(acc, term);
    } else {
        return acc;
    }
}
template <bool SPLIT>
__device__ __forceinline__ float chain_slot_wave(float acc, float term, int first_block, int nb) {
    const int valid = nb - first_block;   // uniform
    if (valid >= 64) return chain_wave_full<SPLIT>(acc, term);
    for (int i = 0; i < valid; i++) acc = fadd(acc, lane_term(term, SPLIT ? (i < 32 ? 2 * i : 2 * (i - 32) + 1) : i));
    return acc;
}

// Few wavefronts per SIMD: registers go to loads in flight rather than to
// occupancy.
template <int WF, int EPI, bool EMB, int LPR, int PPL>
__global__ __launch_bounds__(kGemvMaxThreads) __attribute__((amdgpu_waves_per_eu(1, 3))) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    // a row's lanes share one 16-lane DPP row, or a row spans the wavefront
    // (one scale per block, the residual and plain-store epilogues)
    static_assert(LPR == 8 || LPR == 16 ||
                      (LPR == 64 && blocks_per_group<WF>() == 1 && (EPI == kEpiResid || EPI == kEpiStore)),
                  "lanes per row");
    constexpr int RW = 64 / LPR;          // rows per weight wavefront
    constexpr bool kNorm = EPI == kEpiQkvRope || EPI == kEpiSwiglu;
    constexpr bool kQPro = EPI == kEpiResidQ;   // an f32 input row, quantized here (no RMSNorm)
    constexpr bool kStage = kNorm || kQPro;     // the activation row is made by NA wavefronts
    constexpr int NA = kStage ? kNormWaves : 1;   // activation wavefronts
    constexpr int GSZ = 32 * blocks_per_group<WF>();   // activation (and weight scale) group
    const int n = a.n, nb = a.nb, o = a.o;
    const int nww = (int)(blockDim.x >> 6) - NA;
    const int R = RW * nww;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = blockIdx.y;
    const int row0 = blockIdx.x * R;
    const GemvLds L = gemv_lds(n, nb, R, kNorm);
    int8_t* xl = reinterpret_cast<int8_t*>(smem + L.act);
    float* xsl = reinterpret_cast<float*>(smem + L.scales);
    int* ctr_sq = reinterpret_cast<int*>(smem + L.sync);       // squares written
    int* ctr_row = ctr_sq + 2;                                   // activation row ready
    float* initl = reinterpret_cast<float*>(smem + L.init);
    float* outl = reinterpret_cast<float*>(smem + L.outs);

    // The activation wavefronts issue their loads before this barrier and
    // the weight wavefronts theirs after it, so the row reaches the CU ahead
    // of the weights.  The counters start at zero (LDS holds whatever the
    // previous workgroup left).
    if (tid < 3) __hip_atomic_store(ctr_sq + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

    if (wave < NA) {
        // ---------------------------------------------- activation wavefronts
        if constexpr (kStage) {
            // RMSNorm (util.rs:389-426) + quantize of the residual row (or,
            // kQPro, quantize of the f32 input row), shared by the NA
            // wavefronts: member i of the team holds the 8 elements from
            // 8*(p*team + i) in pass p
            constexpr int MP = kQPro ? 4 : 2;   // dim <= 8192 (kQPro) or 4096: passes of 256 x 8
            const int dim = n;
            const RowTeam tm{tid, 64 * NA};
            const int passes = rowq_passes(dim, 64 * NA);
            vf4 xv[2 * MP], wv_n[kNorm ? 2 * MP : 1];
            EmbRegs<EMB ? MP : 1> er_;
            bool in_vocab = true;
            // the position of the QKV epilogue, loaded first (the RoPE angles
            // and the cache entries the K/V sums start from depend on it)
            int pos = 0;
            if constexpr (EPI == kEpiQkvRope)
                if (wave == NA - 1) pos = a.state->pos + t;
            if constexpr (EMB) {
                const uint32_t tok = a.tokens[t];
                in_vocab = tok < (uint32_t)a.emb.vocab;
                rowq_load_emb<MP>(tm, er_, a.emb, tok, passes);
            } else if constexpr (kQPro) {
                rowq_load_f32<MP>(tm, xv, a.xf + (size_t)t * dim, dim, passes);
            } else {
                rowq_load_f32<MP>(tm, xv, a.x + (size_t)t * dim, dim, passes);
            }
            if constexpr (kNorm) rowq_load_f32<MP>(tm, wv_n, a.norm_w, dim, passes);
            __syncthreads();
            if constexpr (EMB) {
                // the residual stream starts as the embedding row
                // (transformer_llama_gguf.rs:459-473, base_transformer.rs:143-161)
                rowq_embed_values<MP>(xv, er_, in_vocab, passes);
                if (blockIdx.x == 0) {
#pragma unroll
                    for (int p = 0; p < MP; p++)
                        if (p < passes && rowq_live(tm, p, dim)) {
                            vf4* xo = reinterpret_cast<vf4*>(a.x + (size_t)t * dim + rowq_elem(tm, p, dim));
                            xo[0] = xv[2 * p];
                            xo[1] = xv[2 * p + 1];
                        }
                }
            }
            // squares -> the 8 transposed chain rows (zero padded)
            float* sq = reinterpret_cast<float*>(smem + L.norm);
            const int S = rowq_stride(dim);
            if constexpr (kNorm) {
#pragma unroll
            for (int p = 0; p < MP; p++)
                if (p < passes && rowq_live(tm, p, dim)) {
                    const int i = rowq_elem(tm, p, dim) >> 3;
                    const vf4 u = xv[2 * p], v = xv[2 * p + 1];
                    sq[0 * S + i] = fmul(u.x, u.x);
                    sq[1 * S + i] = fmul(u.y, u.y);
                    sq[2 * S + i] = fmul(u.z, u.z);
                    sq[3 * S + i] = fmul(u.w, u.w);
                    sq[4 * S + i] = fmul(v.x, v.x);
                    sq[5 * S + i] = fmul(v.y, v.y);
                    sq[6 * S + i] = fmul(v.z, v.z);
                    sq[7 * S + i] = fmul(v.w, v.w);
                }
            {
                const int n8 = dim / 8, pad = rowq_chain_len(dim) - n8;
                for (int i = tid; i < 8 * pad; i += 64 * NA) sq[(i / pad) * S + n8 + i % pad] = 0.0f;
            }
            // the chain may start: it waits for the squares only
            lds_arrive(ctr_sq);
            }
            // initial values of the rows' sums: the K/V `+=` columns start
            // from the cache (forward.rs:166-169, weight_type.rs:190-201),
            // and (QKV) the epilogue's position and the RoPE angles of the
            // rows (util.rs:653-718; the table row of the position), loaded
            // by the last activation wavefront into registers before the
            // chain and staged after it (lane i: row i, R <= 64), published
            // with the activation row (ctr_row)
            static_assert(64 / LPR * kMaxWeightWaves <= 64, "one lane per row of the workgroup");
            float ini = 0.0f, rcos = 0.0f, rsin = 0.0f;
            if (wave == NA - 1 && lane < R) {
                if constexpr (EPI == kEpiQkvRope) {
                    const int att = a.att_dim, kv = a.kv_dim, hd = a.head_size;
                    const int row = min(row0 + lane, o - 1);
                    const int col = row < att ? row : (row < att + kv ? row - att : row - att - kv);
                    const int pair = (col % hd) >> 1;
                    rcos = a.rope_cos[(size_t)pos * (hd >> 1) + pair];
                    rsin = a.rope_sin[(size_t)pos * (hd >> 1) + pair];
                    const bool is_k = row >= att && row < att + kv, is_v = row >= att + kv;
                    const int c = is_v ? row - att - kv : (is_k ? qk_column(row - att, a.head_size, a.hf_rows) : 0);
                    if ((is_k || is_v) && c < (kv / 4) * 4)
                        ini = is_v ? a.v_cache[(size_t)pos * kv + c] : a.k_cache[(size_t)c * a.kv_ld + pos];
                }
            }
            // the serial sum of squares -> ss: every activation wavefront
            // runs the 8 chains itself (lanes 0-7), so none waits for
            // another's result
            float ss = 1.0f;
            if constexpr (kNorm) {
                lds_wait_count(ctr_sq, NA, a.fault);
                ss = rowq_chain(dim, a.eps, sq);
            }
            if (wave == NA - 1) {
                if (lane < R) initl[lane] = ini;
                if constexpr (EPI == kEpiQkvRope) {
                    float* ropel = reinterpret_cast<float*>(smem + L.rope);
                    if (lane < R) {
                        ropel[2 * lane] = rcos;
                        ropel[2 * lane + 1] = rsin;
                    }
                    if (lane == 0) reinterpret_cast<int*>(ropel)[2 * R] = pos;
                }
            }
            // o = w * (ss * x) and the GSZ-group quantization of the
            // member's slices (the 4 lanes of a quad hold one 32-group, 8
            // consecutive lanes one 64-group)
#pragma unroll
            for (int p = 0; p < MP; p++)
                if (p < passes && rowq_live(tm, p, dim)) {
                    const int e = rowq_elem(tm, p, dim);
                    const vf4 x0 = xv[2 * p], x1 = xv[2 * p + 1];
                    float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    float am = 0.0f;
                    if constexpr (kNorm) {
                        const vf4 w0 = wv_n[2 * p], w1 = wv_n[2 * p + 1];
                        const float w8[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                        for (int k = 0; k < 8; k++) v[k] = fmul(w8[k], fmul(ss, v[k]));
                    }
#pragma unroll
                    for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(v[k]));
                    am = fmaxf(am, dpp_mov<0xB1>(am));   // quad_perm [1,0,3,2]
                    am = fmaxf(am, dpp_mov<0x4E>(am));   // quad_perm [2,3,0,1]
                    if constexpr (GSZ >= 64) am = fmaxf(am, __shfl_xor(am, 4, 64));
                    if constexpr (GSZ >= 128) am = fmaxf(am, __shfl_xor(am, 8, 64));
                    const float sc = group_scale<act_fmt<WF>()>(am);
                    int q[8];
                    quant8<act_fmt<WF>()>(v, sc, q);
                    *reinterpret_cast<uint2*>(xl + e) =
                        WF == kQ4 ? make_uint2(pack4(q[0], q[2], q[4], q[6]), pack4(q[1], q[3], q[5], q[7]))
                                  : make_uint2(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]));
                    if ((tid & (GSZ / 8 - 1)) == 0) xsl[e / GSZ] = sc;
                }
            lds_arrive(ctr_row);
        } else {
            // the quantized row and its scales by LDS DMA and, for the plain
            // store, the initial values of the `+=` columns
            // (int8 rows: n % 32 == 0, so 16-byte pieces; scale rows start at
            // any 4-byte boundary)
            dma_bytes<16>(xl, a.xq + (size_t)t * n, n);
            dma_bytes<4>(xsl, a.xs + (size_t)t * nb, nb * 4);
            float iv = 0.0f;
            if constexpr (EPI == kEpiStore) {
                const int row = min(row0 + lane, o - 1);
                iv = row < a.accumulate_cols ? a.out[(size_t)t * o + row] : 0.0f;
            }
            __syncthreads();
            wait_vm_all();
            if constexpr (WF == kQ4) {
                // Q4_0: each 8-group reordered to (even, odd) elements, in place
                uint2* xd = reinterpret_cast<uint2*>(xl);
                for (int i = lane; i < n / 8; i += 64) xd[i] = q4_reorder8(xd[i]);
            }
            if (lane < R) initl[lane] = iv;   // R <= 64
            lds_arrive(ctr_row);
        }
    } else {
        // -------------------------------------------------- weight wavefronts
        __syncthreads();
        const int w = wave - NA;
        const int wrow0 = row0 + w * RW;                    // this wavefront's first row
        const int r = lane / LPR, j = lane - (lane / LPR) * LPR;
        const int rows_here = max(0, min(RW, o - wrow0));
        const size_t row_bytes = WF != kQ4 ? (size_t)n : (size_t)n / 2;
        constexpr int kBlockBytes = WF != kQ4 ? 32 : 16;
        using SW = typename ScaleWord<WF>::type;
        constexpr int kScaleBytes = (int)sizeof(SW);
        // descriptors over this wavefront's rows: rows past the matrix read 0
        const __amdgpu_buffer_rsrc_t qr =
            uniform_rsrc(a.qs + (size_t)min(wrow0, o - 1) * row_bytes, (int)(rows_here * row_bytes));
        // scales per row: one per block, or one per group of 2 or 4 blocks
        constexpr int kBlocksPerScale = blocks_per_group<WF>();
        const int nsc = nb / kBlocksPerScale;
        constexpr bool kF32Scales = WF == kQ8S || WF == kQ8S64 || WF == kQ8S128;
        const void* scale_rows = kF32Scales ? (const void*)(a.sf + (size_t)min(wrow0, o - 1) * nsc)
                                            : (const void*)(a.d + (size_t)min(wrow0, o - 1) * nb);
        const __amdgpu_buffer_rsrc_t dr = uniform_rsrc(scale_rows, rows_here * nsc * kScaleBytes);
        // 32-byte blocks are read in split halves: in a slot's 32*LPR bytes of
        // a row, lane j reads the 16 bytes at 16j (half j%2 of block j/2) and
        // those at 16(LPR + j) (the same half of block LPR/2 + j/2), so each
        // load instruction covers whole lines.  The pair of lanes (2m, 2m+1)
        // then holds blocks m and LPR/2 + m whole; lane 2m takes the term of
        // block m, lane 2m+1 that of block LPR/2 + m (term_lane).
        constexpr bool kSplit = WF != kQ4;
        const int jb = kSplit ? ((j & 1) ? LPR / 2 + (j >> 1) : (j >> 1)) : j;   // the block of this lane's term
        const int qv = (int)(r * row_bytes) + (kSplit ? j * 16 : j * kBlockBytes);
        const int dv_off = (r * nsc + jb / kBlocksPerScale) * kScaleBytes;
        // Slot by slot (loads complete in issue order, so slot k's wait
        // leaves the later slots in flight; the scheduling barriers keep the
        // compiler from regrouping them).  LA slots go out first, then slot
        // k + LA right after slot k is consumed, into the registers slot k
        // used: under full HBM load a load waits for queue space, and a
        // wavefront that issued everything up front would start its first
        // slot only when most data had arrived.  Measured on the 1B shapes:
        // 4 slots ahead for 8-slot rows (2, 3 and 6 are slower), 6 for
        // 16-slot rows (down matmul 6.5 -> 6.3 us; 4 and 8 are slower).
        constexpr int LA = PPL <= 4 ? PPL : PPL == 16 ? 6 : (PPL / 2 < 8 ? PPL / 2 : 8);
        WBlock<WF> wv[LA];
        SW dv[LA];
        auto issue = [&](int k) {
            load_block<WF, 16 * LPR>(wv[k % LA], qr, qv, k * LPR * kBlockBytes);
            if constexpr (kF32Scales)
                dv[k % LA] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(dr, dv_off, k * (LPR / kBlocksPerScale) * kScaleBytes,
                                                                kPolStream));
            else
                dv[k % LA] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(dr, dv_off, k * LPR * 2, kPolStream);
            __builtin_amdgcn_sched_barrier(0);
        };
#pragma unroll
        for (int k = 0; k < LA; k++) issue(k);
        // the row's first lane holds its sum
        const int my_r = r;
        const bool chain_lane = j == 0;
        const int my_row = wrow0 + my_r;
        // epilogue operand of the residual add (needed only at the end)
        float resid = 0.0f;
        if constexpr (EPI == kEpiResid || EPI == kEpiResidQ) resid = a.x[(size_t)t * o + min(my_row, o - 1)];
        __builtin_amdgcn_sched_barrier(0);

        lds_wait_count(ctr_row, NA, a.fault);
        float acc = initl[min(w * RW + my_r, R - 1)];
#pragma unroll
        for (int k = 0; k < PPL; k++) {
            // exact block dot -> f32 term (lanes past nb compute a term the
            // chain never reads)
            const int b = k * LPR + jb;
            const int bb = b < nb ? b : nb - 1;
            int isum;
            if constexpr (kSplit) {
                const int h = (j & 1) * 16;
                const int b0 = min(k * LPR + (j >> 1), nb - 1), b1 = min(k * LPR + LPR / 2 + (j >> 1), nb - 1);
                int s0 = half_dot(wv[k % LA].a, reinterpret_cast<const int32_t*>(xl + b0 * 32 + h));
                int s1 = half_dot(wv[k % LA].b, reinterpret_cast<const int32_t*>(xl + b1 * 32 + h));
                // whole-block dots from the pair's two halves (quad_perm [1,0,3,2])
                s0 += __builtin_amdgcn_update_dpp(0, s0, 0xB1, 0xF, 0xF, false);
                s1 += __builtin_amdgcn_update_dpp(0, s1, 0xB1, 0xF, 0xF, false);
                isum = (j & 1) ? s1 : s0;
            } else {
                isum = block_dot<WF>(wv[k % LA], reinterpret_cast<const int32_t*>(xl + bb * 32));
            }
            float ws;
            if constexpr (kF32Scales) ws = dv[k % LA];
            else ws = f16_to_f32(dv[k % LA]);
            if constexpr (kBlocksPerScale > 1) {
                // the group's exact int32 dot: this block's plus the next
                // blocks' (their lanes are 1 apart, or 2 with split halves:
                // row_shl, then twice that for 4 blocks; the lane of the
                // group's first block owns it), then its one term
                // ((float)isum * w_scale) * x_scale
                constexpr int kMate = kSplit ? 2 : 1;
                isum += __builtin_amdgcn_update_dpp(0, isum, 0x100 + kMate, 0xF, 0xF, true);
                if constexpr (kBlocksPerScale == 4)
                    isum += __builtin_amdgcn_update_dpp(0, isum, 0x100 + 2 * kMate, 0xF, 0xF, true);
                const float term = fmul(fmul((float)isum, ws), xsl[bb / kBlocksPerScale]);
                acc = chain_slot_dppg<LPR, kSplit, kBlocksPerScale>(acc, term, k * LPR, nb);
            } else {
                const float term = fmul(fmul((float)isum, ws), xsl[bb]);
                if constexpr (LPR == 64) acc = chain_slot_wave<kSplit>(acc, term, k * LPR, nb);
                else acc = chain_slot_dpp<LPR, kSplit>(acc, term, k * LPR, nb);
            }
            if (k + LA < PPL) issue(k + LA);
        }

        // epilogues on the finished sums (chain lanes hold row my_row)
        const bool live = chain_lane && my_row < o;
        if constexpr (EPI == kEpiStore) {
            if (live) a.out[(size_t)t * o + my_row] = acc;
        } else if constexpr (EPI == kEpiResid || EPI == kEpiResidQ) {
            // residual add (forward.rs:196-204 / 245-253)
            if (live) a.x[(size_t)t * o + my_row] = fadd(resid, acc);
        } else if constexpr (EPI == kEpiQkvRope) {
            // rope_gguf (util.rs:653-718): pair (2i, 2i+1) of a head rotated
            // by the angle table row `pos`; v rows are stored as summed.
            // The rows of a pair are in this wavefront (RW even).  With
            // hf_rows the stored pair (2j, 2j+1) is util::rope's pair
            // (j, j + head/2) (util.rs:589-635), the same rotation, written
            // to those columns.
            const float other = __shfl_xor(acc, LPR, 64);
            if (live) {
                const float* ropel = reinterpret_cast<const float*>(smem + L.rope);
                const int pos = reinterpret_cast<const int*>(ropel)[2 * R];
                const int att = a.att_dim, kv = a.kv_dim;
                const bool odd = my_row & 1;
                if (my_row >= att + kv) {
                    a.v_cache[(size_t)pos * kv + (my_row - att - kv)] = acc;
                } else {
                    const int col = qk_column(my_row < att ? my_row : my_row - att, a.head_size, a.hf_rows);
                    const int li = w * RW + my_r;
                    const float c = ropel[2 * li];
                    const float s = ropel[2 * li + 1];
                    const float v0 = odd ? other : acc, v1 = odd ? acc : other;
                    const float rr = odd ? fadd(fmul(v0, s), fmul(v1, c)) : fmul(v0, c) - fmul(v1, s);
                    if (my_row < att) a.q_out[(size_t)t * att + col] = rr;
                    else a.k_cache[(size_t)col * a.kv_ld + pos] = rr;
                }
            }
        } else if constexpr (EPI == kEpiSwiglu) {
            if (chain_lane) outl[w * RW + my_r] = acc;
        }
    }

    if constexpr (EPI == kEpiSwiglu) {
        // SwiGLU (forward.rs:220-237) of the workgroup's 32 outputs: rows
        // [32 gate | 32 up] of one 64-row group, h = (g / (1 + exp(-g))) * u,
        // then this 32-group of h is quantized for the down projection.
        __syncthreads();
        if (wave == 0 && lane < 32) {
            const float g = outl[lane];
            const float u = outl[32 + lane];
            const float den = fadd(1.0f, expf_rn(-g));
            const float h = fmul(g / den, u);
            const int grp = blockIdx.x;
            const size_t base = (size_t)t * a.hidden + (size_t)grp * kGroup;
            if (a.h_f32) a.h_f32[base + lane] = h;
            if (!a.hq) return;   // f32 h only (the down projection quantizes it in 64-groups)
            float am = group_max(fabsf(h), 32);   // lanes 0-31 (rows 0 and 1) all active
            am = fmaxf(am, 0.0f);
            const float sc = a.h_fmt == kQ4 ? group_scale<kQ4>(am) : group_scale<kQ8>(am);
            const int q = a.h_fmt == kQ4 ? quant_one<kQ4>(h, sc) : quant_one<kQ8>(h, sc);
            a.hq[base + lane] = (int8_t)q;
            if (lane == 0) a.hs[(size_t)t * (a.hidden / kGroup) + grp] = sc;
        }
    }
}

// ------------------------------------------------------------ dispatch ----

// Lanes per row and slots per lane for a row of nb blocks: 8 lanes per row
// (8 rows per wavefront) up to 32 blocks, 16 lanes (4 rows) with 4 slots up
// to 64, then 16 lanes with 8, 16 or 32 slots.  A row's lanes stay inside one 16-lane DPP row, where the
// row sums gather the terms.  The gate/up matmul needs 64 rows per
// workgroup (8 weight wavefronts of 8 rows), so it keeps 8 lanes per row and
// takes 16 slots up to 128 blocks.  Residual and plain-store matmuls of 128
// to 512 blocks, at most 2048 rows and at most 2048 x 256 row-blocks, in
// formats with one scale per block, give each row a whole wavefront (64
// lanes, 2, 4 or 8 slots, 8 rows per workgroup): with few rows (the 1B down
// projection's 2048) that keeps 8 weight wavefronts per CU streaming
// instead of 2.  Its chain advances one row per instruction (a DPP chain
// advances four), so beyond those bounds the chain's VALU work outgrows the
// stream (Llama-3-8B's down projection, 4096 x 448 blocks: 13.8 us against
// 10.1 on 16-lane rows).
struct GemvPlan {
    int lpr, ppl, nww;
};
static bool plan_gemv(int o, int nb, int epi, bool wave_rows, GemvPlan* p) {
    if (nb <= 0) return false;
    if (wave_rows && (epi == kEpiResid || epi == kEpiStore) && nb >= 128 && nb <= 512 && o <= 2048 &&
        o * nb <= 2048 * 256) {
        p->lpr = 64;
        p->ppl = nb <= 128 ? 2 : nb <= 256 ? 4 : 8;
        p->nww = kMaxWeightWaves;
        return true;
    }
    if (epi == kEpiSwiglu) {
        if (o % 64 || nb > 128) return false;
        p->lpr = 8;
        p->ppl = nb <= 8 ? 1 : nb <= 16 ? 2 : nb <= 32 ? 4 : nb <= 64 ? 8 : 16;
        p->nww = 8;
        return true;
    }
    if (nb > 32 && nb <= 64) {
        // 16 lanes per row, all 4 slots of a row in flight at once, and as
        // many weight wavefronts (4 rows each, not only powers of two) as
        // keep the grid within one round of 256 workgroups: more independent
        // load streams per CU for the small projections
        p->lpr = 16;
        p->ppl = 4;
        p->nww = 1;
        while (p->nww < kMaxWeightWaves && (o + 4 * p->nww - 1) / (4 * p->nww) > 256) p->nww++;
        return true;
    }
    if (nb <= 64) {
        p->lpr = 8;
        p->ppl = nb <= 8 ? 1 : nb <= 16 ? 2 : nb <= 32 ? 4 : 8;
    } else {
        p->lpr = 16;
        p->ppl = nb <= 128 ? 8 : nb <= 256 ? 16 : nb <= 512 ? 32 : 0;
        if (!p->ppl) return false;
    }
    // one round of workgroups on the 256 CUs: the fewest weight wavefronts
    // per workgroup that keep the grid within 256 workgroups
    const int rw = 64 / p->lpr;
    p->nww = 1;
    while (p->nww < kMaxWeightWaves && (o + rw * p->nww - 1) / (rw * p->nww) > 256) p->nww *= 2;
    return true;
}

template <int WF, int EPI, bool EMB, int LPR, int PPL>
static hipError_t launch_k(const GemvArgs& a, int nww, int batch, hipStream_t st) {
    constexpr bool kNorm = EPI == kEpiQkvRope || EPI == kEpiSwiglu;
    constexpr int NA = kNorm || EPI == kEpiResidQ ? kNormWaves : 1;
    const int R = (64 / LPR) * nww;
    const GemvLds L = gemv_lds(a.n, a.nb, R, kNorm);
    if (L.total > 160 * 1024) return hipErrorInvalidValue;
    if (L.total > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv<WF, EPI, EMB, LPR, PPL>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((a.o + R - 1) / R, batch);
    hipLaunchKernelGGL((k_gemv<WF, EPI, EMB, LPR, PPL>), grid, dim3(64 * (nww + NA)), L.total, st, a);
    return hipGetLastError();
}

template <int WF, int EPI, bool EMB>
static hipError_t launch_plan(const GemvArgs& a, const GemvPlan& p, int batch, hipStream_t st) {
    if (p.lpr == 8) {
        switch (p.ppl) {
        case 1: return launch_k<WF, EPI, EMB, 8, 1>(a, p.nww, batch, st);
        case 2: return launch_k<WF, EPI, EMB, 8, 2>(a, p.nww, batch, st);
        case 4: return launch_k<WF, EPI, EMB, 8, 4>(a, p.nww, batch, st);
        case 8: return launch_k<WF, EPI, EMB, 8, 8>(a, p.nww, batch, st);
        case 16:
            if constexpr (EPI == kEpiSwiglu) return launch_k<WF, EPI, EMB, 8, 16>(a, p.nww, batch, st);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
        }
    }
    if constexpr (blocks_per_group<WF>() == 1 && (EPI == kEpiResid || EPI == kEpiStore)) {
        if (p.lpr == 64) {
            switch (p.ppl) {
            case 2: return launch_k<WF, EPI, EMB, 64, 2>(a, p.nww, batch, st);
            case 4: return launch_k<WF, EPI, EMB, 64, 4>(a, p.nww, batch, st);
            case 8: return launch_k<WF, EPI, EMB, 64, 8>(a, p.nww, batch, st);
            default: return hipErrorInvalidValue;
            }
        }
    }
    if constexpr (EPI != kEpiSwiglu) {
        if (p.lpr == 16) {
            switch (p.ppl) {
            case 4: return launch_k<WF, EPI, EMB, 16, 4>(a, p.nww, batch, st);
            case 8: return launch_k<WF, EPI, EMB, 16, 8>(a, p.nww, batch, st);
            case 16: return launch_k<WF, EPI, EMB, 16, 16>(a, p.nww, batch, st);
            case 32: return launch_k<WF, EPI, EMB, 16, 32>(a, p.nww, batch, st);
            default: return hipErrorInvalidValue;
            }
        }
    }
    return hipErrorInvalidValue;
}

template <int WF>
static hipError_t launch_wf(const GemvArgs& a, int epi, int batch, hipStream_t st) {
    GemvPlan p{};
    if (!plan_gemv(a.o, a.nb, epi, blocks_per_group<WF>() == 1, &p)) return hipErrorInvalidValue;
    switch (epi) {
    case kEpiStore: return launch_plan<WF, kEpiStore, false>(a, p, batch, st);
    case kEpiQkvRope:
        if (a.emb.q) return launch_plan<WF, kEpiQkvRope, true>(a, p, batch, st);
        return launch_plan<WF, kEpiQkvRope, false>(a, p, batch, st);
    case kEpiResid: return launch_plan<WF, kEpiResid, false>(a, p, batch, st);
    case kEpiSwiglu: return launch_plan<WF, kEpiSwiglu, false>(a, p, batch, st);
    case kEpiResidQ:
        if constexpr (WF == kQ8S64 || WF == kQ8S128) return launch_plan<WF, kEpiResidQ, false>(a, p, batch, st);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const GemvArgs& args, int wfmt, int epi, int batch, hipStream_t s) {
    if ((epi == kEpiQkvRope || epi == kEpiSwiglu) && (args.n % 32 || args.n > 4096)) return hipErrorInvalidValue;
    if (epi == kEpiResidQ && (args.n > 8192 || !args.xf)) return hipErrorInvalidValue;
    // kQ8S64 / kQ8S128 activations are quantized in 64 / 128-groups by the kernel's own prologue
    if ((wfmt == kQ8S64 || wfmt == kQ8S128) &&
        (args.n % (wfmt == kQ8S64 ? 64 : 128) || args.nb != args.n / 32 || epi == kEpiResid || epi == kEpiStore))
        return hipErrorInvalidValue;
    if (args.n % 32 || args.n > 16384 || args.o <= 0) return hipErrorInvalidValue;
    GemvArgs a = args;
    a.fault = wait_fault_word(false);
    if (wfmt == kQ8) return launch_wf<kQ8>(a, epi, batch, s);
    if (wfmt == kQ4) return launch_wf<kQ4>(a, epi, batch, s);
    if (wfmt == kQ8S) return launch_wf<kQ8S>(a, epi, batch, s);
    if (wfmt == kQ8S64) return launch_wf<kQ8S64>(a, epi, batch, s);
    if (wfmt == kQ8S128) return launch_wf<kQ8S128>(a, epi, batch, s);
    return hipErrorInvalidValue;
}

size_t gemv_bytes_per_row_block(int wfmt) { return wfmt == kQ8 ? 34 : 18; }

bool gemv_launch_shape(int o, int nb, int epi, int wfmt, int* grid, int* threads) {
    GemvPlan p{};
    if (!plan_gemv(o, nb, epi, wfmt == kQ8 || wfmt == kQ4 || wfmt == kQ8S, &p)) return false;
    const int na = epi == kEpiQkvRope || epi == kEpiSwiglu || epi == kEpiResidQ ? kNormWaves : 1;
    const int R = (64 / p.lpr) * p.nww;
    *grid = (o + R - 1) / R;
    *threads = 64 * (p.nww + na);
    return true;
}

}  // namespace yl
