// yl_attn.hip -- attention over the device KV cache (forward.rs:299-400).
//
// Arithmetic of fused_attention, per (query head, token):
//   score[t2] = reduce_add(8-lane partial q.k over head_size) * scale
//   max from -1e10; e = exp(score - max); sum_exp serial over t2;
//   p = e * (1/sum_exp);  out[d] = reduce_add(lane j sums p*v over t2 = 8c+j
//   in c order) + the seq_len % 8 tail in t2 order.
//
// k_attn_decode (one token): grid (n_heads, C).  Workgroup (h, c) computes
// the scores of positions [c*chunk, (c+1)*chunk) for head h into a scratch
// row; the last of the C workgroups of head h to finish (atomic counter, the
// pattern of a split reduction) runs the softmax and P.V for the head from
// the complete row and quantizes its output groups for the output
// projection.  k_attention (prompt batches) keeps one workgroup per
// (head, token) with the causal mask of the whole call's span.
#include <hip/hip_runtime.h>

#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kAttnThreads = 256;
constexpr int kAttnTile = 64;   // positions per LDS K tile

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

// LDS (floats): q hd | K tile kAttnTile*(hd+4) in phase 1, reused for the
// scores max_seq(+pad) in phase 2 | transposed p 8*PCS | partials 8*hd |
// out hd | reduction 16
__host__ __device__ inline size_t attn_decode_region(int max_seq, int hd) {
    const size_t a = (size_t)kAttnTile * (hd + 4), b = ((size_t)max_seq + 3) & ~(size_t)3;
    return a > b ? a : b;
}
__host__ __device__ inline int attn_pt_stride(int max_seq) { return ((max_seq / 8 + 1 + 3) & ~3) + 4; }
__host__ __device__ inline size_t attn_decode_lds_floats(int max_seq, int hd) {
    return (size_t)hd + attn_decode_region(max_seq, hd) + 8 * (size_t)attn_pt_stride(max_seq) + 9 * (size_t)hd + 16;
}

// Decode kernel: 512 threads.  Phase 2 keeps each thread's P.V chains'
// V values for up to kVChunk chain steps (and the seq_len % 8 tail rows) in
// registers, loaded before the softmax so their HBM latency overlaps the
// max / exp / serial sum.
constexpr int kDecThreads = 512;

template <int QF, int HD>
__global__ __launch_bounds__(kDecThreads) void k_attn_decode(const float* __restrict__ sq,
                                                             const float* __restrict__ kc,
                                                             const float* __restrict__ vc,
                                                             const StepState* __restrict__ st, int n_heads,
                                                             int n_kv_heads, float attn_scale, int max_seq,
                                                             float* __restrict__ scores,
                                                             unsigned* __restrict__ counters,
                                                             int8_t* __restrict__ aq, float* __restrict__ as,
                                                             float* __restrict__ att_f32) {
    constexpr int hd = HD;
    constexpr int CPT = (8 * HD + kDecThreads - 1) / kDecThreads;   // P.V chains per thread
    constexpr int kVChunk = 128 / CPT;                               // chain steps held in registers
    extern __shared__ __align__(16) float lds[];
    __shared__ int is_last;
    const int h = blockIdx.x, c = blockIdx.y, C = gridDim.y, tid = threadIdx.x;
    const int kvh = h / (n_heads / n_kv_heads);
    const int kv_dim = n_kv_heads * hd;
    const int seq = st->pos + 1;
    const int chunk = (seq + C - 1) / C;
    const int p0 = c * chunk;
    const int p1 = min(seq, p0 + chunk);
    constexpr int KS = hd + 4;
    float* ql = lds;
    float* kt = ql + hd;
    float* sc = kt;
    float* pt = kt + attn_decode_region(max_seq, hd);
    float* part = pt + 8 * attn_pt_stride(max_seq);
    float* outl = part + 8 * hd;
    float* red = outl + hd;
    float* srow = scores + (size_t)h * max_seq;

    for (int i = tid; i < hd; i += kDecThreads) ql[i] = sq[(size_t)h * hd + i];
    // phase 1: scores of this workgroup's positions
    for (int base = p0; base < p1; base += kAttnTile) {
        const int cnt = min(kAttnTile, p1 - base);
        __syncthreads();
        constexpr int h4 = hd / 4;
        for (int e = tid; e < cnt * h4; e += kDecThreads) {
            const int r = e / h4, q4 = e - r * h4;
            const float4 v = *reinterpret_cast<const float4*>(kc + (size_t)(base + r) * kv_dim + (size_t)kvh * hd + q4 * 4);
            *reinterpret_cast<float4*>(kt + r * KS + q4 * 4) = v;
        }
        __syncthreads();
        if (tid < cnt) {
            const float* kr = kt + tid * KS;
            float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < hd / 8; s++) {
#pragma unroll
                for (int j = 0; j < 8; j++) l[j] = fadd(l[j], fmul(ql[s * 8 + j], kr[s * 8 + j]));
            }
            srow[base + tid] = fmul(reduce_add8(l), attn_scale);
        }
    }
    // last arriver of this head runs phase 2 (the barrier orders every
    // thread's score stores before thread 0's release fence and count)
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const unsigned prev = atomicAdd(counters + h, 1u);
        is_last = prev == (unsigned)(C - 1) ? 1 : 0;
        if (is_last) {
            __threadfence();
            counters[h] = 0u;
        }
    }
    __syncthreads();
    if (!is_last) return;

    // softmax: max from -1e10, exp, serial sum, p = e * (1/sum)
    float lmax = -1e10f;
    for (int t2 = tid; t2 < seq; t2 += kDecThreads) {
        const float v = __hip_atomic_load(srow + t2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sc[t2] = v;
        lmax = fmaxf(lmax, v);
    }

    // V values of this thread's chains (d, j) for the first kVChunk steps,
    // issued now so they arrive during the softmax (clamped, unconditional
    // loads: a divergent branch would make the compiler wait at its join)
    const int n_chunks = seq / 8;
    const float* vbase = vc + (size_t)kvh * hd;
    float vtail[7];
    {
        const int d = tid < hd ? tid : 0;
#pragma unroll
        for (int i = 0; i < 7; i++) vtail[i] = vbase[(size_t)min(n_chunks * 8 + i, seq - 1) * kv_dim + d];
    }
    float vbuf[CPT][kVChunk];
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int ch = min(tid + k * kDecThreads, 8 * hd - 1);
        const int j = (ch / hd) & 7, d = ch % hd;
#pragma unroll
        for (int i = 0; i < kVChunk; i++) {
            const int row = min(8 * i + j, seq - 1);
            vbuf[k][i] = vbase[(size_t)row * kv_dim + d];
        }
    }
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) red[tid >> 6] = lmax;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < kDecThreads / 64; w++) mx = fmaxf(mx, red[w]);
    for (int t2 = tid; t2 < seq; t2 += kDecThreads) sc[t2] = expf_rn(sc[t2] - mx);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        int t2 = 0;
        const float4* s4 = reinterpret_cast<const float4*>(sc);
#pragma unroll 8
        for (; t2 + 4 <= seq; t2 += 4) {
            const float4 e4 = s4[t2 >> 2];
            sum = fadd(sum, e4.x);
            sum = fadd(sum, e4.y);
            sum = fadd(sum, e4.z);
            sum = fadd(sum, e4.w);
        }
        for (; t2 < seq; t2++) sum = fadd(sum, sc[t2]);
        red[8] = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = red[8];
    // p = e * inv, kept in sc and also transposed into pt[j][c] = p[8c+j] so
    // a chain reads its probabilities as consecutive floats
    const int PCS = attn_pt_stride(max_seq);
    for (int t2 = tid; t2 < seq; t2 += kDecThreads) {
        const float p = fmul(sc[t2], inv);
        sc[t2] = p;
        pt[(t2 & 7) * PCS + (t2 >> 3)] = p;
    }
    __syncthreads();

    // P.V chains: lane j of position group c, in c order
    float l[CPT];
#pragma unroll
    for (int k = 0; k < CPT; k++) l[k] = 0.0f;
    for (int r0 = 0; r0 < n_chunks; r0 += kVChunk) {
        if (r0 > 0) {
#pragma unroll
            for (int k = 0; k < CPT; k++) {
                const int ch = min(tid + k * kDecThreads, 8 * hd - 1);
                const int j = (ch / hd) & 7, d = ch % hd;
#pragma unroll
                for (int i = 0; i < kVChunk; i++) {
                    const int row = min(8 * (r0 + i) + j, seq - 1);
                    vbuf[k][i] = vbase[(size_t)row * kv_dim + d];
                }
            }
        }
        const int steps = min(kVChunk, n_chunks - r0);
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int ch = tid + k * kDecThreads;
            const float* pj = pt + ((ch / hd) & 7) * PCS + r0;
            float acc = l[k];
#pragma unroll
            for (int i = 0; i < kVChunk; i++)
                if (i < steps) acc = fadd(acc, fmul(pj[i], vbuf[k][i]));
            if (ch < 8 * hd) l[k] = acc;
        }
    }
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int ch = tid + k * kDecThreads;
        if (ch < 8 * hd) part[(ch / hd) * hd + (ch % hd)] = l[k];
    }
    __syncthreads();
    for (int d = tid; d < hd; d += kDecThreads) {
        float lj[8];
#pragma unroll
        for (int j = 0; j < 8; j++) lj[j] = part[j * hd + d];
        float sum = reduce_add8(lj);
#pragma unroll
        for (int i = 0; i < 7; i++)
            if (n_chunks * 8 + i < seq) sum = fadd(sum, fmul(sc[n_chunks * 8 + i], vtail[i]));
        outl[d] = sum;
        if (att_f32) att_f32[(size_t)h * hd + d] = sum;
    }
    __syncthreads();
    if constexpr (QF >= 0) quantize_head_output<QF>(outl, hd, aq, as, ((size_t)h * hd) / kGroup);
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
                                                            int n_heads, int n_kv_heads, int hd,
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
        const float4* kr = reinterpret_cast<const float4*>(kc + (size_t)t2 * kv_dim + (size_t)kvh * hd);
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int s = 0; s < n_simd; s++) {
            const float4 k0 = kr[2 * s], k1 = kr[2 * s + 1];
            const float* q = ql + s * 8;
            l[0] = fadd(l[0], fmul(q[0], k0.x));
            l[1] = fadd(l[1], fmul(q[1], k0.y));
            l[2] = fadd(l[2], fmul(q[2], k0.z));
            l[3] = fadd(l[3], fmul(q[3], k0.w));
            l[4] = fadd(l[4], fmul(q[4], k1.x));
            l[5] = fadd(l[5], fmul(q[5], k1.y));
            l[6] = fadd(l[6], fmul(q[6], k1.z));
            l[7] = fadd(l[7], fmul(q[7], k1.w));
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

hipError_t launch_attention(const float* sq, const float* kc, const float* vc, const StepState* st, int batch,
                            int max_seq, int n_heads, int n_kv_heads, int head_size, float scale, int qfmt,
                            int8_t* aq, float* as, float* att_f32, hipStream_t s) {
    const size_t smem = ((size_t)((max_seq + 3) & ~3) + 10 * (size_t)head_size) * sizeof(float);
    const dim3 grid(n_heads, batch);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_attention<kQ8>), grid, dim3(kAttnThreads), smem, s, sq, kc, vc, st, batch, n_heads,
                           n_kv_heads, head_size, scale, aq, as, att_f32);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_attention<kQ4>), grid, dim3(kAttnThreads), smem, s, sq, kc, vc, st, batch, n_heads,
                           n_kv_heads, head_size, scale, aq, as, att_f32);
    else
        hipLaunchKernelGGL((k_attention<-1>), grid, dim3(kAttnThreads), smem, s, sq, kc, vc, st, batch, n_heads,
                           n_kv_heads, head_size, scale, aq, as, att_f32);
    return hipGetLastError();
}

int attn_decode_splits(int max_seq) {
    // enough workgroups per head to spread the K reads, few enough that the
    // per-head counter sees little contention
    int c = (max_seq + 255) / 256;
    return c < 4 ? 4 : (c > 16 ? 16 : c);
}

size_t attn_decode_lds_bytes(int max_seq, int hd) { return attn_decode_lds_floats(max_seq, hd) * sizeof(float); }

template <int QF>
static hipError_t launch_attn_decode_q(const float* sq, const float* kc, const float* vc, const StepState* st,
                                       int max_seq, int n_heads, int n_kv_heads, int hd, float scale, float* scores,
                                       unsigned* counters, int8_t* aq, float* as, float* att_f32, hipStream_t s) {
    const size_t smem = attn_decode_lds_bytes(max_seq, hd);
    const dim3 grid(n_heads, attn_decode_splits(max_seq));
    if (smem > 65536) {
        // long contexts: opt in to more than the default 64 KiB of LDS
        hipError_t e = hipSuccess;
        if (hd == 32) e = hipFuncSetAttribute((const void*)&k_attn_decode<QF, 32>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (hd == 64) e = hipFuncSetAttribute((const void*)&k_attn_decode<QF, 64>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (hd == 128) e = hipFuncSetAttribute((const void*)&k_attn_decode<QF, 128>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
    }
    switch (hd) {
    case 32:
        hipLaunchKernelGGL((k_attn_decode<QF, 32>), grid, dim3(kDecThreads), smem, s, sq, kc, vc, st, n_heads,
                           n_kv_heads, scale, max_seq, scores, counters, aq, as, att_f32);
        break;
    case 64:
        hipLaunchKernelGGL((k_attn_decode<QF, 64>), grid, dim3(kDecThreads), smem, s, sq, kc, vc, st, n_heads,
                           n_kv_heads, scale, max_seq, scores, counters, aq, as, att_f32);
        break;
    case 128:
        hipLaunchKernelGGL((k_attn_decode<QF, 128>), grid, dim3(kDecThreads), smem, s, sq, kc, vc, st, n_heads,
                           n_kv_heads, scale, max_seq, scores, counters, aq, as, att_f32);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attn_decode(const float* sq, const float* kc, const float* vc, const StepState* st, int max_seq,
                              int n_heads, int n_kv_heads, int head_size, float scale, int qfmt, float* scores,
                              unsigned* counters, int8_t* aq, float* as, float* att_f32, hipStream_t s) {
    if (qfmt == kQ8)
        return launch_attn_decode_q<kQ8>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, head_size, scale, scores,
                                         counters, aq, as, att_f32, s);
    if (qfmt == kQ4)
        return launch_attn_decode_q<kQ4>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, head_size, scale, scores,
                                         counters, aq, as, att_f32, s);
    return launch_attn_decode_q<-1>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, head_size, scale, scores, counters,
                                    aq, as, att_f32, s);
}

}  // namespace yl
