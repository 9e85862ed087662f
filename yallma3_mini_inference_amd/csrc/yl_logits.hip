// yl_logits.hip -- final RMSNorm + tied-embedding logits (forward.rs:256-279)
// + greedy argmax (sampler.rs:67-79) + end-of-step bookkeeping.
//
// Every workgroup normalizes the last token's residual row itself (util.rs
// rmsnorm, f32 result in LDS) while its first embedding loads are in flight,
// then each wavefront takes 64 consecutive vocabulary rows (lane = row).  A
// lane keeps the 8 f32x8 lane partials of its row and walks the row in
// 16-element chunks (two f32x8 steps each), so every partial sees its terms
// in the reference's order.  The embedding value is the exact f32 product
// q * scale of the Q8_0 table (transformer_llama_gguf.rs:465-470).
// Each workgroup writes the maximum of its rows as a packed 64-bit key
// (larger value, then smaller index) into a device-scope atomic max and
// counts itself done; the last workgroup to finish turns the winner into
// the next token, appends it to the output ring and advances the position.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

// The embedding table is streamed once per token: non-temporal loads keep it
// from evicting the data the next step's kernels wait on (see yl_gemv.hip).
typedef int vi4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 load_stream(const int4* p) {
    const vi4_t v = __builtin_nontemporal_load(reinterpret_cast<const vi4_t*>(p));
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t load_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }

constexpr int kLogitThreads = 256;
constexpr int kLogitGroups = 2;   // groups of 4 chunks (16 bytes per lane each) in flight

// EF = 0: Q8_0 table (u8 chunks of 16 + f16 scale pairs); EF = 1: f16 table
// (32-byte chunks of 16 values), whose values are exactly the reference's f32
// table (load_f16_tensor, transformer_llama_gguf.rs:412-421,487); EF = 3:
// int8 chunks of 16 with an f32 scale per group of gs (lm.rs and safetensors
// Q8 embeddings): the reference dequantizes these into an f32 table
// (transformer_llama_lmrs.rs:176-181, transformer_llama_st.rs:236-250) whose
// values are exactly q * scale, recomputed here for a quarter of the bytes.
template <int EF>
__global__ __launch_bounds__(kLogitThreads) void k_logits(EmbQ8 e, const float* __restrict__ x,
                                                          const float* __restrict__ norm_w, float eps,
                                                          float* __restrict__ logits,
                                                          StepState* st, uint32_t* __restrict__ ring,
                                                          uint32_t ring_cap, int advance) {
    extern __shared__ __align__(16) float lds[];
    __shared__ unsigned long long wkey[kLogitThreads / 64];
    constexpr int MP = 8192 / 8 / kLogitThreads;   // dim <= 8192
    constexpr int NG = kLogitGroups;
    constexpr int CI = EF == 1 ? 2 : 1;   // int4 loads per 16-value chunk
    const int dim = e.dim, tid = threadIdx.x;
    float* xn = lds;             // the normalized row, zero over the padding
    float* sq = lds + e.dimp;
    const int wave = tid >> 6, lane = tid & 63;
    const int tile = blockIdx.x * (kLogitThreads / 64) + wave;
    const bool live = tile < e.tiles;
    const int ng = e.dimp / 64;   // groups: 4 chunks, one block pair
    // chunk k of this row at qp[k * cs], the scales of block pair g at dp[g * cs]
    const size_t cs = (size_t)e.tiles * 64;
    // (F16 and F32: each chunk is CI int4, chunk k of this row at qp[CI * k * cs + i])
    const int4* qp = reinterpret_cast<const int4*>(e.q) + (size_t)(live ? tile : 0) * 64 * CI + lane * CI;
    const uint32_t* dp = reinterpret_cast<const uint32_t*>(e.d) + (size_t)(live ? tile : 0) * 64 + lane;
    // (EF 3: the scale of chunk k's group at sp[(16 * k / gs) * cs])
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(e.d32) + (size_t)(live ? tile : 0) * 64 + lane;
    for (int i = dim + tid; i < e.dimp; i += kLogitThreads) xn[i] = 0.0f;

    // the residual row and norm weights first (every wavefront's loads issued
    // before the barrier), then the first embedding groups, which stay in
    // flight while the row is normalized (loads retire in issue order)
    const RowTeam tm = team_workgroup();
    const int passes = rowq_passes(dim, kLogitThreads);
    vf4 xv[2 * MP], wv[2 * MP];
    rowq_load_f32<MP>(tm, xv, x, dim, passes);
    rowq_load_f32<MP>(tm, wv, norm_w, dim, passes);
    __syncthreads();
    // a ring of NG groups: each group's scale word, then its 4 chunks
    int4 qv[NG][4 * CI];
    uint32_t sv[NG];
    uint32_t s4[NG][4];
    auto load_group = [&](int gg, int g) {
        if constexpr (EF == 0) {
            sv[gg] = load_stream(dp + (size_t)g * cs);
#pragma unroll
            for (int c = 0; c < 4; c++) qv[gg][c] = load_stream(qp + (size_t)(4 * g + c) * cs);
        } else if constexpr (EF == 3) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                s4[gg][c] = load_stream(sp + (size_t)((16 * (4 * g + c)) / e.gs) * cs);
                qv[gg][c] = load_stream(qp + (size_t)(4 * g + c) * cs);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int i = 0; i < CI; i++) qv[gg][CI * c + i] = load_stream(qp + (size_t)(4 * g + c) * cs * CI + i);
        }
    };
#pragma unroll
    for (int gg = 0; gg < NG; gg++) load_group(gg, min(gg, ng - 1));
    rowq_stage<MP>(tm, xv, wv, dim, passes, sq);
    rowq_norm_quant<-1, false>(dim, eps, sq, nullptr, nullptr, xn);

    unsigned long long kk = 0ull;
    if (live) {
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int g0 = 0; g0 < ng; g0 += NG) {
#pragma unroll
            for (int gg = 0; gg < NG; gg++) {
                const int g = g0 + gg;
                if (NG > 1 && g >= ng) break;
                const uint32_t sw = EF == 0 ? sv[gg] : 0u;
                uint32_t sc4[4];
#pragma unroll
                for (int c = 0; c < 4; c++) sc4[c] = EF == 3 ? s4[gg][c] : 0u;
                int4 q4[4 * CI];
#pragma unroll
                for (int c = 0; c < 4 * CI; c++) q4[c] = qv[gg][c];
                // refill with group g + NG (clamped re-reads past the row are
                // never used)
                load_group(gg, min(g + NG, ng - 1));
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (EF == 3) {
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float scv = __builtin_bit_cast(float, sc4[c]);
                        const float* xk = xn + (4 * g + c) * 16;
                        const uint32_t w[4] = {(uint32_t)q4[c].x, (uint32_t)q4[c].y, (uint32_t)q4[c].z,
                                               (uint32_t)q4[c].w};
#pragma unroll
                        for (int ei = 0; ei < 16; ei++) {
                            const int qv8 = (int)(int8_t)((w[ei >> 2] >> (8 * (ei & 3))) & 0xffu);
                            l[ei & 7] = fadd(l[ei & 7], fmul(xk[ei], fmul((float)qv8, scv)));
                        }
                    }
                    continue;
                }
                if constexpr (EF == 1) {
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float* xk = xn + (4 * g + c) * 16;
                        const uint32_t w[8] = {(uint32_t)q4[2 * c].x, (uint32_t)q4[2 * c].y, (uint32_t)q4[2 * c].z,
                                               (uint32_t)q4[2 * c].w, (uint32_t)q4[2 * c + 1].x,
                                               (uint32_t)q4[2 * c + 1].y, (uint32_t)q4[2 * c + 1].z,
                                               (uint32_t)q4[2 * c + 1].w};
#pragma unroll
                        for (int ei = 0; ei < 16; ei++) {
                            const float ev = f16_to_f32((uint16_t)(w[ei >> 1] >> (16 * (ei & 1))));
                            l[ei & 7] = fadd(l[ei & 7], fmul(xk[ei], ev));
                        }
                    }
                    continue;
                }
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float scv = f16_to_f32((uint16_t)(c < 2 ? sw & 0xffffu : sw >> 16));
                    const float nsc = -128.0f * scv;   // exact: power-of-two multiple
                    const float* xk = xn + (4 * g + c) * 16;
                    const uint32_t w[4] = {(uint32_t)q4[c].x, (uint32_t)q4[c].y, (uint32_t)q4[c].z,
                                           (uint32_t)q4[c].w};
#pragma unroll
                    for (int m = 0; m < 4; m++) {
#pragma unroll
                        for (int bb = 0; bb < 4; bb++) {
                            const int ei = m * 4 + bb;
                            // table bytes hold u = q + 128; u*scale - 128*scale is
                            // exactly q*scale (at most 19 significant bits), so the
                            // single rounding of the fma is no rounding at all
                            const float uf = (float)((w[m] >> (8 * bb)) & 0xffu);
                            const float e2 = __builtin_fmaf(uf, scv, nsc);
                            l[ei & 7] = fadd(l[ei & 7], fmul(xk[ei], e2));
                        }
                    }
                }
            }
        }
        const float logit = reduce_add8(l);
        const int row = tile * 64 + lane;
        if (row < e.vocab) {
            if (logits) logits[row] = logit;
            kk = argmax_key(logit, (uint32_t)row);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o2 = __shfl_xor(kk, off, 64);
        kk = o2 > kk ? o2 : kk;
    }
    if (lane == 0) wkey[wave] = kk;
    __syncthreads();
    if (tid != 0) return;
    unsigned long long m = wkey[0];
    for (int w = 1; w < kLogitThreads / 64; w++) m = wkey[w] > m ? wkey[w] : m;
    // The step's key is the maximum over the workgroups' keys, kept by a
    // device-scope atomic max in the step state; then this workgroup counts
    // itself done.  The count's increment depends on the value the max
    // returned, so it is performed after the max; the workgroup that
    // counts last sees every workgroup's max.
    unsigned long long prev = __hip_atomic_fetch_max(&st->argmax, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t one = 1u;
    asm volatile("" : "+v"(one) : "v"(prev));
    const uint32_t done = __hip_atomic_fetch_add(&st->logits_done, one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done != gridDim.x - 1) return;
    // Greedy step end: the winner -> next token, appended to the output ring,
    // position advanced; the key and the count return to zero for the next
    // step.
    m = __hip_atomic_load(&st->argmax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // (every key is nonzero: a row's key is zero only for a NaN past row 0,
    // and row 0's key is never zero)
    const uint32_t tok = m ? 0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull) : 0u;
    st->token = tok;
    if (ring && st->n_out < ring_cap) ring[st->n_out] = tok;
    st->n_out += 1;
    st->pos += advance;
    __hip_atomic_store(&st->argmax, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&st->logits_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t logits_lds_bytes(int dim) { return ((size_t)((dim + 63) & ~63) + rowq_lds_floats(dim)) * sizeof(float); }
static int logits_blocks(const EmbQ8& e) { return (e.tiles + kLogitThreads / 64 - 1) / (kLogitThreads / 64); }

hipError_t launch_logits(const EmbQ8& e, const float* x, const float* norm_w, float eps, float* logits,
                         StepState* st, uint32_t* ring, uint32_t ring_cap, int advance,
                         hipStream_t s) {
    const int nblk = logits_blocks(e);
    if (e.dim % 32 || e.dim > 8192) return hipErrorInvalidValue;
    if (e.fmt == 3 && (e.gs <= 0 || e.gs % 16)) return hipErrorInvalidValue;
    auto kern = e.fmt == 3 ? k_logits<3> : (e.fmt == 1 ? k_logits<1> : k_logits<0>);
    if (logits_lds_bytes(e.dim) > 65536) {
        const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)logits_lds_bytes(e.dim));
        if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL(kern, dim3(nblk), dim3(kLogitThreads), logits_lds_bytes(e.dim), s, e, x, norm_w, eps,
                       logits, st, ring, ring_cap, advance);
    return hipGetLastError();
}

}  // namespace yl
