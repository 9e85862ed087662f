// yl_gemv.hip -- quantized GEMV / batched matvec (weight_type.rs:122-226)
// with the neighbouring elementwise work of forward.rs fused in.
//
// A workgroup owns R consecutive output rows of one batch row (blockIdx.y).
// Its threads split the R*nb (row, block) pairs.  Every thread first issues
// the loads of all its pairs' weights (two 16-byte loads per Q8_0 block, one
// per Q4_0 block, plus the f16 scale) into registers, right after its share
// of the activation row; the workgroup then prepares the activation row in
// LDS -- either staging an already quantized row, or (QKV and gate/up
// matmuls) computing RMSNorm + quantize of the f32 residual stream itself --
// while the weights are in flight.
//
// Each pair's exact int32 block dot (v_dot4_i32_i8) becomes the f32 term
//     ((float)isum * w_scale) * x_scale
// in LDS, and thread r sums row r's terms in block order from the row's
// initial value: the reference's `xout += term` sequence, so every output is
// bit-identical to matmul_q8_slices for any grid shape.
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

template <int WF>
__device__ __forceinline__ void load_block(WBlock<WF>& w, const uint8_t* __restrict__ p) {
    if constexpr (WF == kQ8) {
        const uint4* q = reinterpret_cast<const uint4*>(p);
        w.a = q[0];
        w.b = q[1];
    } else {
        w.a = *reinterpret_cast<const uint4*>(p);
    }
}

template <int WF>
__device__ __forceinline__ int block_dot(const WBlock<WF>& w, const int32_t* xw) {
    int acc = 0;
    if constexpr (WF == kQ8) {
        acc = __builtin_amdgcn_sdot4((int)w.a.x, xw[0], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.a.y, xw[1], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.a.z, xw[2], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.a.w, xw[3], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.x, xw[4], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.y, xw[5], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.z, xw[6], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.w, xw[7], acc, false);
    } else {
        const uint32_t m = 0x0f0f0f0fu;
        acc = __builtin_amdgcn_sdot4((int)(w.a.x & m), xw[0], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.x >> 4) & m), xw[1], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.a.y & m), xw[2], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.y >> 4) & m), xw[3], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.a.z & m), xw[4], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.z >> 4) & m), xw[5], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.a.w & m), xw[6], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.w >> 4) & m), xw[7], acc, false);
    }
    return acc;
}

// terms row stride (floats): float4-aligned rows for the ordered sums
__host__ __device__ inline int terms_stride(int nb) { return ((nb + 3) & ~3) + 4; }

static size_t gemv_smem(int n, int nb, int R, int epi, int dim) {
    size_t s = (size_t)n + (size_t)nb * 4;
    s = (s + 15) & ~(size_t)15;
    s += (size_t)R * terms_stride(nb) * 4 + 64 * 4;
    if (epi == kEpiQkvRope || epi == kEpiSwiglu) s += (size_t)8 * rowq_stride(dim) * 4;   // chain rows
    return s;
}

// Block terms of one row added in block order onto acc (the reference's
// `xout += term` sequence).
__device__ __forceinline__ float ordered_row_sum(const float* tr, int nb, float acc) {
    const vf4* t4 = reinterpret_cast<const vf4*>(tr);
    const int nq = nb >> 2, nfull = nq >> 3;   // whole batches of 8 float4s
    acc = lds_serial_sum(t4, nfull, acc);
    for (int q = nfull * 8; q < nq; q++) {
        const vf4 v = t4[q];
        acc = fadd(acc, v.x);
        acc = fadd(acc, v.y);
        acc = fadd(acc, v.z);
        acc = fadd(acc, v.w);
    }
    for (int b = nq * 4; b < nb; b++) acc = fadd(acc, tr[b]);
    return acc;
}

// Few wavefronts per SIMD: a decode launch has 1-2 workgroups per CU, so
// registers go to loads in flight rather than to occupancy.
template <int WF, int R, int TPB, int PMAX, int EPI, bool EMB>
__global__ __launch_bounds__(TPB) __attribute__((amdgpu_waves_per_eu(1, TPB > 512 ? 3 : 2))) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int n = a.n, nb = a.nb, o = a.o;
    const int tid = threadIdx.x;
    const int t = blockIdx.y;
    const int row0 = blockIdx.x * R;
    const int TS = terms_stride(nb);
    int8_t* xl = reinterpret_cast<int8_t*>(smem);
    float* xsl = reinterpret_cast<float*>(smem + n);
    float* terms = reinterpret_cast<float*>(smem + (((size_t)n + (size_t)nb * 4 + 15) & ~(size_t)15));
    float* accs = terms + R * TS;
    float* xt = accs + 64;
    constexpr bool kNorm = EPI == kEpiQkvRope || EPI == kEpiSwiglu;

    // Global loads are issued in the order they are needed: activation
    // inputs (recently written, cache-hot) before weights, weights before
    // what only the epilogue reads.  Vector-memory loads retire in order, so
    // waiting for the activations leaves the weights in flight.
    // With an RMSNorm prologue every thread loads its slices of the row
    // first, so they land early; the squares, the serial sum (one wavefront)
    // and the quantization then run while the weights stream in.
    // All loads are unconditional (out-of-range indices are clamped and their
    // data ignored): a load under a divergent branch makes the compiler wait
    // for it at the branch join, which would serialize the HBM round trips.
    const int dim = n;
    constexpr int WT = TPB;                      // threads that load weights
    const int tw = tid;                          // weight-thread index
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int total = R * nb;
    WBlock<WF> wv[PMAX];
    uint16_t dv[PMAX];
    float ep0 = 0.0f, ep1 = 1.0f, ep2 = 0.0f;
    bool ep_acc = false;
    int pos = 0;

    auto load_weights = [&]() {
        const size_t row_bytes = WF == kQ8 ? (size_t)n : (size_t)n / 2;
        const int dr = WT / nb, db = WT % nb;
        int r = tw / nb, b = tw - (tw / nb) * nb;
#pragma unroll
        for (int k = 0; k < PMAX; k++) {
            const bool ok = tw + k * WT < total && row0 + r < o;
            const size_t row = ok ? (size_t)(row0 + r) : 0;
            load_block<WF>(wv[k], a.qs + row * row_bytes + (size_t)b * (WF == kQ8 ? 32 : 16));
            dv[k] = a.d[row * nb + b];
            r += dr;
            b += db;
            if (b >= nb) { b -= nb; r += 1; }
        }
    };
    // values the epilogue reads (cache initial values and RoPE angles at the
    // decode position, the residual row, the accumulate-into output); row r
    // of the workgroup is finished by weight thread r (R <= 64: one
    // wavefront), which issues these loads right after its weight loads
    auto load_epilogue = [&]() {
        pos = (EPI == kEpiQkvRope) ? a.state->pos + t : 0;
        const int er = min(row0 + (tw >= 0 && tw < R ? tw : 0), o - 1);
        if constexpr (EPI == kEpiQkvRope) {
            // K/V rows accumulate into the cache (forward.rs:166-169)
            const int att = a.att_dim, kv = a.kv_dim, hd = a.head_size;
            const bool is_k = er >= att && er < att + kv, is_v = er >= att + kv;
            const int c = is_v ? er - att - kv : (is_k ? er - att : 0);
            ep_acc = (is_k || is_v) && c < (kv / 4) * 4;
            ep0 = is_v ? a.v_cache[(size_t)pos * kv + c] : a.k_cache[(size_t)c * a.kv_ld + pos];
            const int col = er < att ? er : c;
            const int pair = (col % hd) >> 1;
            ep1 = a.rope_cos[(size_t)pos * (hd >> 1) + pair];
            ep2 = a.rope_sin[(size_t)pos * (hd >> 1) + pair];
        } else if constexpr (EPI == kEpiResid) {
            ep0 = a.x[(size_t)t * o + er];
        } else if constexpr (EPI == kEpiStore) {
            ep_acc = er < a.accumulate_cols;
            ep0 = a.out[(size_t)t * o + er];
        }
    };

    if constexpr (kNorm) {
        // 1. every thread: its 8-element groups of the residual row (or, in
        // layer 0, of the token's embedding row) and of the norm weights,
        // then the epilogue values and its weight pairs, all issued before
        // any wait.  Loads retire in order, so the row groups arrive first
        // while the weights stream on.
        constexpr int MP = (4096 / 8 + TPB - 1) / TPB;   // dim <= 4096
        const int ng = dim / 8;
        vf4 xg[2 * MP], wg[2 * MP];
        uint2 eq[EMB ? MP : 1];
        uint16_t ed[EMB ? MP : 1];
        uint32_t tok = 0;
        bool in_vocab = true;
        if constexpr (EMB) {
            tok = a.tokens[t];
            in_vocab = tok < (uint32_t)a.emb.vocab;
        }
#pragma unroll
        for (int p = 0; p < MP; p++) {
            if (p * TPB >= ng) break;
            const int e = 8 * min(tid + p * TPB, ng - 1);
            if constexpr (EMB) {
                // interleaved Q8_0 table: bytes q+128 at [vocab/64][dim/16][64][16],
                // f16 scales at [vocab/64][dim/32][64]; ids outside the vocabulary
                // read row 0 and become zeros below
                const size_t tile = in_vocab ? tok >> 6 : 0;
                const int ln = (int)(tok & 63u);
                const uint8_t* q = reinterpret_cast<const uint8_t*>(a.emb.q);
                eq[p] = *reinterpret_cast<const uint2*>(q + ((tile * (dim / 16) + (e >> 4)) * 64 + ln) * 16 + (e & 15));
                ed[p] = a.emb.d[(tile * (dim / 32) + (e >> 5)) * 64 + ln];
            } else {
                const vf4* x4 = reinterpret_cast<const vf4*>(a.x + (size_t)t * dim + e);
                xg[2 * p] = x4[0];
                xg[2 * p + 1] = x4[1];
            }
            const vf4* w4 = reinterpret_cast<const vf4*>(a.norm_w + e);
            wg[2 * p] = w4[0];
            wg[2 * p + 1] = w4[1];
        }
        if (wave == 0) load_epilogue();
        load_weights();
        // (nothing below may be scheduled before the weight loads are issued)
        __builtin_amdgcn_sched_barrier(0);

        // 2. squares -> the 8 transposed chain rows in LDS (zero padded)
        const int S = rowq_stride(dim);
        float* sq = xt;
#pragma unroll
        for (int p = 0; p < MP; p++) {
            const int g = tid + p * TPB;
            if (p * TPB >= ng || g >= ng) break;
            if constexpr (EMB) {
                // the residual stream starts as the embedding row
                // (transformer_llama_gguf.rs:459-473, base_transformer.rs:143-161)
                const float sc = f16_to_f32(ed[p]);
                float v[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t w = k < 4 ? eq[p].x : eq[p].y;
                    const int u = (int)((w >> (8 * (k & 3))) & 0xffu);
                    v[k] = in_vocab ? fmul((float)(u - 128), sc) : 0.0f;
                }
                xg[2 * p] = vf4{v[0], v[1], v[2], v[3]};
                xg[2 * p + 1] = vf4{v[4], v[5], v[6], v[7]};
                if (blockIdx.x == 0) {
                    vf4* xo = reinterpret_cast<vf4*>(a.x + (size_t)t * dim + 8 * g);
                    xo[0] = xg[2 * p];
                    xo[1] = xg[2 * p + 1];
                }
            }
            const vf4 x0 = xg[2 * p], x1 = xg[2 * p + 1];
            sq[0 * S + g] = fmul(x0.x, x0.x);
            sq[1 * S + g] = fmul(x0.y, x0.y);
            sq[2 * S + g] = fmul(x0.z, x0.z);
            sq[3 * S + g] = fmul(x0.w, x0.w);
            sq[4 * S + g] = fmul(x1.x, x1.x);
            sq[5 * S + g] = fmul(x1.y, x1.y);
            sq[6 * S + g] = fmul(x1.z, x1.z);
            sq[7 * S + g] = fmul(x1.w, x1.w);
        }
        {
            const int pad = rowq_chain_len(dim) - ng;
            for (int i = tid; i < 8 * pad; i += TPB) sq[(i / pad) * S + ng + i % pad] = 0.0f;
        }
        __syncthreads();

        // 3. the serial sum of squares (wavefront 0, lanes 0-7) -> ss
        if (wave == 0) {
            const float ss = rowq_chain(dim, a.eps, sq);
            if (tid == 0) accs[0] = ss;
        }
        __syncthreads();

        // 4. o = w * (ss * x) and the 32-group quantization, each thread on
        // its own groups (the 4 threads of a quad hold one 32-group)
        const float ss = accs[0];
#pragma unroll
        for (int p = 0; p < MP; p++) {
            if (p * TPB >= ng) break;
            const int g = tid + p * TPB;
            const bool live = g < ng;
            const vf4 x0 = xg[2 * p], x1 = xg[2 * p + 1], w0 = wg[2 * p], w1 = wg[2 * p + 1];
            float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            float am = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                v[k] = fmul(w[k], fmul(ss, v[k]));
                am = fmaxf(am, fabsf(v[k]));
            }
            am = fmaxf(am, dpp_mov<0xB1>(am));   // quad_perm [1,0,3,2]
            am = fmaxf(am, dpp_mov<0x4E>(am));   // quad_perm [2,3,0,1]
            const float sc = group_scale<WF>(am);
            int q[8];
            quant8<WF>(v, sc, q);
            if (live) {
                *reinterpret_cast<uint2*>(xl + 8 * g) =
                    WF == kQ4 ? make_uint2(pack4(q[0], q[2], q[4], q[6]), pack4(q[1], q[3], q[5], q[7]))
                              : make_uint2(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]));
                if ((g & 3) == 0) xsl[g >> 2] = sc;
            }
        }
        __syncthreads();
    } else {
        // 1a. quantized activation row -> registers
        constexpr int kMaxStage = 16384 / 8 / TPB;   // staged int8 rows: n <= 16384
        constexpr int kMaxScale = (512 + TPB - 1) / TPB;
        uint2 qv[kMaxStage];
        float sv[kMaxScale];
        const uint2* __restrict__ xg = reinterpret_cast<const uint2*>(a.xq + (size_t)t * n);
        const float* __restrict__ xsg = a.xs + (size_t)t * nb;
#pragma unroll
        for (int k = 0; k < kMaxStage; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < n / 8) qv[k] = xg[i < n / 8 ? i : 0];
        }
#pragma unroll
        for (int k = 0; k < kMaxScale; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < nb) sv[k] = xsg[i < nb ? i : 0];
        }
        // 1b. epilogue values, weights -> registers
        load_epilogue();
        load_weights();
        // 2. activation row -> LDS (int8 values + f32 group scales)
        uint2* xd = reinterpret_cast<uint2*>(xl);
#pragma unroll
        for (int k = 0; k < kMaxStage; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < n / 8 && i < n / 8) {
                uint2 v = qv[k];
                if constexpr (WF == kQ4) v = q4_reorder8(v);
                xd[i] = v;
            }
        }
#pragma unroll
        for (int k = 0; k < kMaxScale; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < nb && i < nb) xsl[i] = sv[k];
        }
        __syncthreads();
    }

    // 3. exact block dots -> f32 terms in LDS
    {
        const int dr = WT / nb, db = WT % nb;
        int r = tw / nb, b = tw - (tw / nb) * nb;
        if (db == 0) {
            // every pair of this thread uses the same activation block
            int32_t xw[8];
#pragma unroll
            for (int j = 0; j < 8; j++) xw[j] = reinterpret_cast<const int32_t*>(xl + b * 32)[j];
            const float xs_b = xsl[b];
#pragma unroll
            for (int k = 0; k < PMAX; k++) {
                if (tw + k * WT < total) {
                    float term = 0.0f;
                    if (row0 + r < o) term = fmul(fmul((float)block_dot<WF>(wv[k], xw), f16_to_f32(dv[k])), xs_b);
                    terms[r * TS + b] = term;
                }
                r += dr;
            }
        } else {
#pragma unroll
            for (int k = 0; k < PMAX; k++) {
                if (tw + k * WT < total) {
                    float term = 0.0f;
                    if (row0 + r < o) {
                        const int isum = block_dot<WF>(wv[k], reinterpret_cast<const int32_t*>(xl + b * 32));
                        term = fmul(fmul((float)isum, f16_to_f32(dv[k])), xsl[b]);
                    }
                    terms[r * TS + b] = term;
                }
                r += dr;
                b += db;
                if (b >= nb) { b -= nb; r += 1; }
            }
        }
    }
    __syncthreads();

    // 4. ordered per-row sums
    if (tw >= 0 && tw < R) {
        const int row = row0 + tw;
        if (row < o) {
            const float acc = ordered_row_sum(terms + tw * TS, nb, ep_acc ? ep0 : 0.0f);
            accs[tw] = acc;
            if constexpr (EPI == kEpiStore) a.out[(size_t)t * o + row] = acc;
            if constexpr (EPI == kEpiResid) {
                // residual add (forward.rs:196-204 / 245-253)
                a.x[(size_t)t * o + row] = fadd(ep0, acc);
            }
        }
    }
    if constexpr (EPI == kEpiStore || EPI == kEpiResid) return;
    __syncthreads();

    // 5. epilogues over neighbouring rows
    if constexpr (EPI == kEpiQkvRope) {
        // rope_gguf (util.rs:653-718): pair (2i, 2i+1) of a head rotated by the
        // angle table row `pos`; v rows are stored as summed.
        if (tw >= 0 && tw < R) {
            const int row = row0 + tw;
            if (row < o) {
                const int att = a.att_dim, kv = a.kv_dim, hd = a.head_size;
                const float v = accs[tw];
                if (row >= att + kv) {
                    a.v_cache[(size_t)pos * kv + (row - att - kv)] = v;
                } else {
                    const int col = row < att ? row : row - att;
                    const float c = ep1, s = ep2;
                    const float v0 = accs[tw & ~1], v1 = accs[tw | 1];
                    const float r = (tw & 1) ? fadd(fmul(v0, s), fmul(v1, c)) : fmul(v0, c) - fmul(v1, s);
                    if (row < att) a.q_out[(size_t)t * att + col] = r;
                    else a.k_cache[(size_t)col * a.kv_ld + pos] = r;
                }
            }
        }
    } else if constexpr (EPI == kEpiSwiglu) {
        // SwiGLU (forward.rs:220-237): h = (g / (1 + exp(-g))) * u, then this
        // 32-group of h is quantized for the down projection.
        if (tw >= 0 && tw < 32) {
            const float g = accs[tw];
            const float u = accs[32 + tw];
            const float den = fadd(1.0f, expf_rn(-g));
            const float h = fmul(g / den, u);
            const int grp = blockIdx.x;
            const size_t base = (size_t)t * a.hidden + (size_t)grp * kGroup;
            if (a.h_f32) a.h_f32[base + tw] = h;
            float am = group_max(fabsf(h), 32);   // lanes 0-31 (rows 0 and 1) all active
            am = fmaxf(am, 0.0f);
            const float sc = a.h_fmt == kQ4 ? group_scale<kQ4>(am) : group_scale<kQ8>(am);
            const int q = a.h_fmt == kQ4 ? quant_one<kQ4>(h, sc) : quant_one<kQ8>(h, sc);
            a.hq[base + tw] = (int8_t)q;
            if (tw == 0) a.hs[(size_t)t * (a.hidden / kGroup) + grp] = sc;
        }
    }
}

// ------------------------------------------------------------ dispatch ----

struct GemvShape {
    int R, WT, PMAX;   // rows per workgroup, weight-loading threads, pairs per thread
};

// Rows per workgroup and threads: enough workgroups to cover the 256 CUs,
// 32-128 KiB of weights in flight per CU, and every pair of a thread loaded
// before its first use.  Kernels with an RMSNorm prologue launch one more
// wavefront (the normalizing one) than WT.
static GemvShape pick_shape(int o, int nb, int epi) {
    GemvShape s;
    s.WT = epi == kEpiSwiglu ? 512 : 256;
    if (epi == kEpiSwiglu) s.R = 64;
    else if (nb >= 192) s.R = 4;
    else if (o >= 8192) s.R = 16;
    else s.R = 8;
    const int p = (s.R * nb + s.WT - 1) / s.WT;
    s.PMAX = p <= 1 ? 1 : p <= 2 ? 2 : p <= 4 ? 4 : p <= 8 ? 8 : p <= 16 ? 16 : 0;
    return s;
}

template <int WF, int R, int TPB, int PMAX, int EPI, bool EMB>
static hipError_t launch_k(const GemvArgs& a, dim3 grid, size_t smem, hipStream_t st) {
    if (smem > 65536) {
        // rows longer than 4096 need more than the default 64 KiB of LDS
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv<WF, R, TPB, PMAX, EPI, EMB>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_gemv<WF, R, TPB, PMAX, EPI, EMB>), grid, dim3(TPB), smem, st, a);
    return hipGetLastError();
}

template <int WF, int R, int TPB, int EPI, bool EMB>
static hipError_t launch_r2(const GemvArgs& a, int pmax, int batch, hipStream_t st) {
    const size_t smem = gemv_smem(a.n, a.nb, R, EPI, a.n);
    const dim3 grid((a.o + R - 1) / R, batch);
    switch (pmax) {
    case 1: return launch_k<WF, R, TPB, 1, EPI, EMB>(a, grid, smem, st);
    case 2: return launch_k<WF, R, TPB, 2, EPI, EMB>(a, grid, smem, st);
    case 4: return launch_k<WF, R, TPB, 4, EPI, EMB>(a, grid, smem, st);
    case 8: return launch_k<WF, R, TPB, 8, EPI, EMB>(a, grid, smem, st);
    case 16: return launch_k<WF, R, TPB, 16, EPI, EMB>(a, grid, smem, st);
    default: return hipErrorInvalidValue;
    }
}

template <int WF, int R, int TPB, int EPI>
static hipError_t launch_r(const GemvArgs& a, int pmax, int batch, hipStream_t st) {
    if constexpr (EPI == kEpiQkvRope) {
        if (a.emb.q) return launch_r2<WF, R, TPB, EPI, true>(a, pmax, batch, st);
    }
    return launch_r2<WF, R, TPB, EPI, false>(a, pmax, batch, st);
}

template <int WF, int EPI>
static hipError_t launch_epi(const GemvArgs& a, int batch, hipStream_t st) {
    const GemvShape s = pick_shape(a.o, a.nb, EPI);
    if (s.PMAX == 0) return hipErrorInvalidValue;
    if constexpr (EPI == kEpiSwiglu) {
        return launch_r<WF, 64, 512, EPI>(a, s.PMAX, batch, st);
    } else {
        constexpr int T = 256;
        if (s.R == 4) return launch_r<WF, 4, T, EPI>(a, s.PMAX, batch, st);
        if (s.R == 16) return launch_r<WF, 16, T, EPI>(a, s.PMAX, batch, st);
        return launch_r<WF, 8, T, EPI>(a, s.PMAX, batch, st);
    }
}

template <int WF>
static hipError_t launch_wf(const GemvArgs& a, int epi, int batch, hipStream_t st) {
    switch (epi) {
    case kEpiStore: return launch_epi<WF, kEpiStore>(a, batch, st);
    case kEpiQkvRope: return launch_epi<WF, kEpiQkvRope>(a, batch, st);
    case kEpiResid: return launch_epi<WF, kEpiResid>(a, batch, st);
    case kEpiSwiglu: return launch_epi<WF, kEpiSwiglu>(a, batch, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const GemvArgs& a, int wfmt, int epi, int batch, hipStream_t s) {
    if ((epi == kEpiQkvRope || epi == kEpiSwiglu) && (a.n % 32 || a.n > 4096)) return hipErrorInvalidValue;
    if (a.n % 32 || a.n > 16384) return hipErrorInvalidValue;
    if (wfmt == kQ8) return launch_wf<kQ8>(a, epi, batch, s);
    if (wfmt == kQ4) return launch_wf<kQ4>(a, epi, batch, s);
    return hipErrorInvalidValue;
}

size_t gemv_bytes_per_row_block(int wfmt) { return wfmt == kQ8 ? 34 : 18; }

}  // namespace yl
