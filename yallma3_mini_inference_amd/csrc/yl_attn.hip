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
//   1. scores of all seq positions, one position per thread per round, the K
//      row loaded straight into registers and q read as uniform (scalar)
//      values; every workgroup of the head recomputes them (K is read from
//      L2 after the first);
//   2. max, exp, and the serial sum (one lane, LDS reads kept in flight);
//   3. the P.V chains of its 32 dimensions, V prefetched into registers
//      while the softmax runs;
//   4. the 8-lane reduction + tail, and the quantized group.
// LDS (floats): e/p row kDecScLen | transposed p 8*PCS | partials 8*32 |
// out 32 | reduction 16
// ---------------------------------------------------------------------------
constexpr int kDecThreads = 512;
constexpr int kDecDims = 32;                   // output dims per workgroup
constexpr int kDecChains = 8 * kDecDims;       // P.V chains per workgroup
constexpr int kDecVSteps = 64;                 // chain steps of V held in registers

__host__ __device__ inline int attn_sc_len(int max_seq) { return (max_seq + 63) & ~63; }
__host__ __device__ inline int attn_pt_stride(int max_seq) { return ((max_seq / 8 + 1 + 3) & ~3) + 4; }
__host__ __device__ inline size_t attn_decode_lds_floats(int max_seq) {
    return (size_t)attn_sc_len(max_seq) + 8 * (size_t)attn_pt_stride(max_seq) + 8 * kDecDims + kDecDims + 16;
}

template <int QF, int HD>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_attn_decode(
    const float* __restrict__ sq, const float* __restrict__ kc, const float* __restrict__ vc,
    const StepState* __restrict__ st, int n_heads, int n_kv_heads, float attn_scale, int max_seq,
    int8_t* __restrict__ aq, float* __restrict__ as, float* __restrict__ att_f32) {
    constexpr int RB = HD == 128 ? 1 : (HD == 64 ? 2 : 4);   // score rounds per load batch
    extern __shared__ __align__(16) float lds[];
    const int h = blockIdx.x, ds = blockIdx.y, tid = threadIdx.x;
    const int kvh = h / (n_heads / n_kv_heads);
    const int kv_dim = n_kv_heads * HD;
    const int seq = st->pos + 1;
    const int n_chunks = seq / 8;
    const int PCS = attn_pt_stride(max_seq);
    float* sc = lds;
    float* pt = sc + attn_sc_len(max_seq);
    float* part = pt + 8 * PCS;
    float* outl = part + kDecChains;
    float* red = outl + kDecDims;
    const float* __restrict__ qh = sq + (size_t)h * HD;
    const float* kbase = kc + (size_t)kvh * HD;
    // chain (j, d) of this thread (tid < kDecChains): lane j of position
    // group c, output dimension d of this workgroup's slice
    const int cj = (tid >> 5) & 7, cd = tid & 31;
    const float* vcol = vc + (size_t)kvh * HD + ds * kDecDims + cd;

    // 1. scores; the V values of the first kDecVSteps chain steps are issued
    // after the first K batch (loads retire in order: waiting for K does
    // not wait for V)
    float vbuf[kDecVSteps];
    float vtail[7];
    float lmax = -1e10f;
    for (int r0 = 0; r0 * kDecThreads < seq; r0 += RB) {
        vf4 kr[RB][HD / 4];
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const int p = min((r0 + r) * kDecThreads + tid, seq - 1);
            const vf4* k4 = reinterpret_cast<const vf4*>(kbase + (size_t)p * kv_dim);
#pragma unroll
            for (int i = 0; i < HD / 4; i++) kr[r][i] = k4[i];
        }
        if (r0 == 0) {
#pragma unroll
            for (int i = 0; i < kDecVSteps; i++) vbuf[i] = vcol[(size_t)min(8 * i + cj, seq - 1) * kv_dim];
#pragma unroll
            for (int i = 0; i < 7; i++) vtail[i] = vcol[(size_t)min(n_chunks * 8 + i, seq - 1) * kv_dim];
        }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const int p = (r0 + r) * kDecThreads + tid;
            float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < HD / 8; s++) {
                const vf4 a = kr[r][2 * s], b = kr[r][2 * s + 1];
                l[0] = fadd(l[0], fmul(qh[8 * s + 0], a.x));
                l[1] = fadd(l[1], fmul(qh[8 * s + 1], a.y));
                l[2] = fadd(l[2], fmul(qh[8 * s + 2], a.z));
                l[3] = fadd(l[3], fmul(qh[8 * s + 3], a.w));
                l[4] = fadd(l[4], fmul(qh[8 * s + 4], b.x));
                l[5] = fadd(l[5], fmul(qh[8 * s + 5], b.y));
                l[6] = fadd(l[6], fmul(qh[8 * s + 6], b.z));
                l[7] = fadd(l[7], fmul(qh[8 * s + 7], b.w));
            }
            const float sv = fmul(reduce_add8(l), attn_scale);
            // unconditional store (positions past seq go to a spare slot):
            // a conditional one would let the compiler sink the K loads
            // into a divergent branch and wait for them at its end
            const bool live = p < seq;
            *(live ? sc + p : red + 15) = sv;
            lmax = fmaxf(lmax, live ? sv : -1e10f);
        }
    }

    // 2. softmax: max from -1e10 (forward.rs:351-356), e = exp(s - max),
    // sum_exp serial in position order, p = e * (1 / sum_exp)
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) red[tid >> 6] = lmax;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < kDecThreads / 64; w++) mx = fmaxf(mx, red[w]);
    const int sc_pad = (seq + 63) & ~63;
    for (int t2 = tid; t2 < sc_pad; t2 += kDecThreads) sc[t2] = t2 < seq ? expf_rn(sc[t2] - mx) : 0.0f;
    __syncthreads();
    if (tid == 0) {
        // blocks of 8 vf4s, the next block read before the current one is
        // added; the zero padding past seq adds nothing
        const vf4* s4 = reinterpret_cast<const vf4*>(sc);
        const int nblk = sc_pad / 32;
        float sum = 0.0f;
        vf4 va[8], vb[8];
#pragma unroll
        for (int k = 0; k < 8; k++) va[k] = s4[k];
        for (int b = 0; b < nblk; b += 2) {
            const int b1 = b + 1 < nblk ? b + 1 : b;
#pragma unroll
            for (int k = 0; k < 8; k++) vb[k] = s4[b1 * 8 + k];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                sum = fadd(sum, va[k].x);
                sum = fadd(sum, va[k].y);
                sum = fadd(sum, va[k].z);
                sum = fadd(sum, va[k].w);
            }
            const int b2 = b + 2 < nblk ? b + 2 : b;
#pragma unroll
            for (int k = 0; k < 8; k++) va[k] = s4[b2 * 8 + k];
            if (b + 1 < nblk) {
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    sum = fadd(sum, vb[k].x);
                    sum = fadd(sum, vb[k].y);
                    sum = fadd(sum, vb[k].z);
                    sum = fadd(sum, vb[k].w);
                }
            }
        }
        red[8] = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = red[8];
    // p kept in sc (for the tail) and transposed, pt[j][c] = p[8c + j], so a
    // chain reads its probabilities as consecutive floats
    for (int t2 = tid; t2 < seq; t2 += kDecThreads) {
        const float p = fmul(sc[t2], inv);
        sc[t2] = p;
        pt[(t2 & 7) * PCS + (t2 >> 3)] = p;
    }
    __syncthreads();

    // 3. P.V chains (forward.rs:372-395): lane j adds p*v over c in order
    if (tid < kDecChains) {
        float acc = 0.0f;
        const float* pj = pt + cj * PCS;
        for (int c0 = 0; c0 < n_chunks; c0 += kDecVSteps) {
            if (c0 > 0) {
#pragma unroll
                for (int i = 0; i < kDecVSteps; i++)
                    vbuf[i] = vcol[(size_t)min(8 * (c0 + i) + cj, seq - 1) * kv_dim];
            }
            const int steps = min(kDecVSteps, n_chunks - c0);
#pragma unroll
            for (int i = 0; i < kDecVSteps; i += 4) {
                const vf4 p4 = *reinterpret_cast<const vf4*>(pj + c0 + i);
                if (i + 0 < steps) acc = fadd(acc, fmul(p4.x, vbuf[i + 0]));
                if (i + 1 < steps) acc = fadd(acc, fmul(p4.y, vbuf[i + 1]));
                if (i + 2 < steps) acc = fadd(acc, fmul(p4.z, vbuf[i + 2]));
                if (i + 3 < steps) acc = fadd(acc, fmul(p4.w, vbuf[i + 3]));
            }
        }
        part[cj * kDecDims + cd] = acc;
    }
    __syncthreads();

    // 4. out[d] = reduce_add(8 lane chains) + the seq % 8 tail in order,
    // then the 32-group quantization of the output projection's input
    if (tid < kDecDims) {
        float lj[8];
#pragma unroll
        for (int j = 0; j < 8; j++) lj[j] = part[j * kDecDims + tid];
        float out = reduce_add8(lj);
#pragma unroll
        for (int i = 0; i < 7; i++)
            if (n_chunks * 8 + i < seq) out = fadd(out, fmul(sc[n_chunks * 8 + i], vtail[i]));
        const size_t col = (size_t)h * HD + (size_t)ds * kDecDims + tid;
        if (att_f32) att_f32[col] = out;
        if constexpr (QF >= 0) {
            float am = fabsf(out);
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 32));
            am = fmaxf(am, 0.0f);
            const float s = group_scale<QF>(am);
            aq[col] = (int8_t)quant_one<QF>(out, s);
            if (tid == 0) as[col / kGroup] = s;
        }
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

size_t attn_decode_lds_bytes(int max_seq) { return attn_decode_lds_floats(max_seq) * sizeof(float); }

template <int QF, int HD>
static hipError_t launch_attn_decode_k(const float* sq, const float* kc, const float* vc, const StepState* st,
                                       int max_seq, int n_heads, int n_kv_heads, float scale, int8_t* aq, float* as,
                                       float* att_f32, hipStream_t s) {
    const size_t smem = attn_decode_lds_bytes(max_seq);
    if (smem > 65536) {
        // long contexts: opt in to more than the default 64 KiB of LDS
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_decode<QF, HD>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_attn_decode<QF, HD>), dim3(n_heads, HD / kDecDims), dim3(kDecThreads), smem, s, sq, kc, vc,
                       st, n_heads, n_kv_heads, scale, max_seq, aq, as, att_f32);
    return hipGetLastError();
}

template <int QF>
static hipError_t launch_attn_decode_q(const float* sq, const float* kc, const float* vc, const StepState* st,
                                       int max_seq, int n_heads, int n_kv_heads, int hd, float scale, int8_t* aq,
                                       float* as, float* att_f32, hipStream_t s) {
    switch (hd) {
    case 32: return launch_attn_decode_k<QF, 32>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, scale, aq, as, att_f32, s);
    case 64: return launch_attn_decode_k<QF, 64>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, scale, aq, as, att_f32, s);
    case 128: return launch_attn_decode_k<QF, 128>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, scale, aq, as, att_f32, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_decode(const float* sq, const float* kc, const float* vc, const StepState* st, int max_seq,
                              int n_heads, int n_kv_heads, int head_size, float scale, int qfmt, int8_t* aq, float* as,
                              float* att_f32, hipStream_t s) {
    if (qfmt == kQ8)
        return launch_attn_decode_q<kQ8>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, head_size, scale, aq, as,
                                         att_f32, s);
    if (qfmt == kQ4)
        return launch_attn_decode_q<kQ4>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, head_size, scale, aq, as,
                                         att_f32, s);
    return launch_attn_decode_q<-1>(sq, kc, vc, st, max_seq, n_heads, n_kv_heads, head_size, scale, aq, as, att_f32,
                                    s);
}

}  // namespace yl
