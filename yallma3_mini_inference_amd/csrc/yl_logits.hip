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
// (larger value, then smaller index); k_finalize reduces the keys, turns the
// winner into the next token, appends it to the output ring and advances
// the position.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kLogitThreads = 256;
constexpr int kLogitChunks = 8;   // 16-byte chunks in flight per lane

__global__ __launch_bounds__(kLogitThreads) void k_logits(EmbQ8 e, const float* __restrict__ x,
                                                          const float* __restrict__ norm_w, float eps,
                                                          float* __restrict__ logits,
                                                          unsigned long long* __restrict__ keys) {
    extern __shared__ __align__(16) float lds[];
    __shared__ unsigned long long wkey[kLogitThreads / 64];
    constexpr int MP = 8192 / 8 / kLogitThreads;   // dim <= 8192
    const int dim = e.dim, tid = threadIdx.x;
    float* xn = lds;
    float* sq = lds + dim;
    const int wave = tid >> 6, lane = tid & 63;
    const int tile = blockIdx.x * (kLogitThreads / 64) + wave;
    const bool live = tile < e.tiles;
    const int k16n = dim / 16, nbE = dim / kGroup;
    const int4* qp = reinterpret_cast<const int4*>(e.q) + (size_t)(live ? tile : 0) * k16n * 64 + lane;
    const uint16_t* dp = e.d + (size_t)(live ? tile : 0) * nbE * 64 + lane;

    // the residual row and norm weights first (every wavefront's loads issued
    // before the barrier), then the first embedding chunks, which stay in
    // flight while the row is normalized (loads retire in issue order)
    const RowTeam tm = team_workgroup();
    const int passes = rowq_passes(dim, kLogitThreads);
    vf4 xv[2 * MP], wv[2 * MP];
    rowq_load_f32<MP>(tm, xv, x, dim, passes);
    rowq_load_f32<MP>(tm, wv, norm_w, dim, passes);
    __syncthreads();
    // embedding chunks (16 bytes per lane) and their f16 block scales (one
    // per two chunks) in one ring, each scale issued right behind its chunks:
    // loads retire in issue order, so a scale loaded just in time would wait
    // for every chunk prefetched before it
    int4 qv[kLogitChunks];
    uint16_t sv[kLogitChunks / 2];
#pragma unroll
    for (int k = 0; k < kLogitChunks; k++) {
        qv[k] = qp[(size_t)min(k, k16n - 1) * 64];
        if (k & 1) sv[k >> 1] = dp[(size_t)min(k >> 1, nbE - 1) * 64];
    }
    rowq_stage<MP>(tm, xv, wv, dim, passes, sq);
    rowq_norm_quant<-1, false>(dim, eps, sq, nullptr, nullptr, xn);

    unsigned long long kk = 0ull;
    if (live) {
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int k0 = 0; k0 < k16n; k0 += kLogitChunks) {
#pragma unroll
            for (int kk2 = 0; kk2 < kLogitChunks; kk2++) {
                const int k = k0 + kk2;
                if (k < k16n) {
                    const int4 q4 = qv[kk2];
                    const float scv = f16_to_f32(sv[kk2 >> 1]);
                    // refill: chunk k + kLogitChunks, and after an odd chunk
                    // the scale of the block kLogitChunks/2 ahead (clamped
                    // reads past the row are never used)
                    qv[kk2] = qp[(size_t)min(k + kLogitChunks, k16n - 1) * 64];
                    if (kk2 & 1) sv[kk2 >> 1] = dp[(size_t)min((k + kLogitChunks) >> 1, nbE - 1) * 64];
                    const float nsc = -128.0f * scv;   // exact: power-of-two multiple
                    const float* xk = xn + k * 16;
                    const uint32_t w[4] = {(uint32_t)q4.x, (uint32_t)q4.y, (uint32_t)q4.z, (uint32_t)q4.w};
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
    if (tid == 0) {
        unsigned long long m = wkey[0];
        for (int w = 1; w < kLogitThreads / 64; w++) m = wkey[w] > m ? wkey[w] : m;
        keys[blockIdx.x] = m;
    }
}

// Greedy step end: maximum of the per-workgroup keys -> next token, appended
// to the output ring, position advanced.
__global__ __launch_bounds__(512) void k_finalize(const unsigned long long* __restrict__ keys, int n, StepState* st,
                                                  uint32_t* __restrict__ ring, uint32_t ring_cap, int advance) {
    __shared__ unsigned long long wk[8];
    unsigned long long m = 0ull;
    for (int i = threadIdx.x; i < n; i += 512) m = keys[i] > m ? keys[i] : m;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o2 = __shfl_xor(m, off, 64);
        m = o2 > m ? o2 : m;
    }
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x != 0) return;
    m = wk[0];
    for (int w = 1; w < 8; w++) m = wk[w] > m ? wk[w] : m;
    const uint32_t tok = 0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull);
    st->token = tok;
    if (ring && st->n_out < ring_cap) ring[st->n_out] = tok;
    st->n_out += 1;
    st->pos += advance;
}

size_t logits_lds_bytes(int dim) { return ((size_t)dim + rowq_lds_floats(dim)) * sizeof(float); }
int logits_blocks(const EmbQ8& e) { return (e.tiles + kLogitThreads / 64 - 1) / (kLogitThreads / 64); }

hipError_t launch_logits(const EmbQ8& e, const float* x, const float* norm_w, float eps, float* logits,
                         unsigned long long* keys, StepState* st, uint32_t* ring, uint32_t ring_cap, int advance,
                         hipStream_t s) {
    const int nblk = logits_blocks(e);
    if (e.dim % 32 || e.dim > 8192) return hipErrorInvalidValue;
    if (logits_lds_bytes(e.dim) > 65536) {
        const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(k_logits),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)logits_lds_bytes(e.dim));
        if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL(k_logits, dim3(nblk), dim3(kLogitThreads), logits_lds_bytes(e.dim), s, e, x, norm_w, eps,
                       logits, keys);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_finalize, dim3(1), dim3(512), 0, s, keys, nblk, st, ring, ring_cap, advance);
    return hipGetLastError();
}

}  // namespace yl
