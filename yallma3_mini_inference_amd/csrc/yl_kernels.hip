// yl_kernels.hip -- standalone op kernels of the forward path (the per-op C
// ABI entry points and the embedding lookup).  The decode/prefill pipeline's
// fused kernels live in yl_gemv.hip, yl_attn.hip and yl_logits.hip.
//
// Each kernel reproduces the f32 operation order of the reference CPU path
// (paths relative to the reference repository):
//   quantize            quantization.rs:29-52, weight_type.rs:52-74
//   rmsnorm             util.rs:389-426
//   rope_gguf           util.rs:653-718
//   SwiGLU              forward.rs:220-237
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kThreads = 256;

// RMSNorm (+ quantize) of `batch` rows, one workgroup per row.  The
// quantized row and its scales go straight to global memory (no LDS copy),
// so a workgroup holds only the transposed row and the norm weights in LDS
// and a whole 2048-row batch is resident at once.
template <int QF>
__global__ __launch_bounds__(kThreads) void k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w,
                                                      int dim, float eps, float* xn, int8_t* xq, float* xs) {
    extern __shared__ __align__(16) float xt[];
    const int t = blockIdx.x;
    // 8 elements per thread and pass, every load issued before the first
    // store (a load per iteration would wait out one memory round trip each)
    for (int i0 = threadIdx.x; i0 < dim; i0 += 8 * kThreads) {
        float xv[8], wv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = min(i0 + k * kThreads, dim - 1);
            xv[k] = x[(size_t)t * dim + i];
            wv[k] = w[i];
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (i0 + k * kThreads < dim) store_norm_input(xt, dim, i0 + k * kThreads, xv[k], wv[k]);
    }
    __syncthreads();
    rmsnorm_quant_block<QF, false>(xt, dim, eps, QF >= 0 ? xq + (size_t)t * dim : nullptr,
                                   QF >= 0 ? xs + (size_t)t * (dim / kGroup) : nullptr,
                                   xn ? xn + (size_t)t * dim : nullptr);
}

// Embedding lookup (base_transformer.rs:143-161: out-of-range ids give
// zeros; the row is the f32 dequantization q*scale of the Q8_0 table,
// transformer_llama_gguf.rs:459-473), written to x.
__global__ __launch_bounds__(kThreads) void k_embed(EmbQ8 e, const uint32_t* __restrict__ tokens,
                                                    float* __restrict__ x) {
    const int t = blockIdx.x;
    const int dim = e.dim;
    const uint32_t tok = tokens[t];
    const int lane = (int)(tok & 63u);
    const size_t tile = tok >> 6;
    // 8 elements per thread and pass, computed (loads issued) before any is stored
    for (int i0 = threadIdx.x; i0 < dim; i0 += 8 * (int)blockDim.x) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = min(i0 + k * (int)blockDim.x, dim - 1);
            v[k] = 0.0f;
            if (tok < (uint32_t)e.vocab) {
                const size_t off = emb_q_off(e.tiles, tile, i >> 4, lane) + (i & 15);
                if (e.fmt == 3) {
                    v[k] = fmul((float)e.q[off], e.d32[((size_t)(i / e.gs) * e.tiles + tile) * 64 + lane]);
                } else if (e.fmt == 1) {
                    v[k] = f16_to_f32(reinterpret_cast<const uint16_t*>(e.q)[off]);
                } else {
                    const int q = (int)(uint8_t)e.q[off] - 128;
                    v[k] = fmul((float)q, f16_to_f32(e.d[emb_d_idx(e.tiles, tile, i >> 5, lane)]));
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (i0 + k * (int)blockDim.x < dim) x[(size_t)t * dim + i0 + k * (int)blockDim.x] = v[k];
    }
}

// Activation quantization over a flat array: one thread per 32-group.
template <int QF>
__global__ void k_quantize(int8_t* __restrict__ q, float* __restrict__ s, const float* __restrict__ x,
                           size_t groups) {
    const size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    const float* xg = x + g * kGroup;
    float amax = 0.0f;
    for (int k = 0; k < kGroup; k++) amax = fmaxf(amax, fabsf(xg[k]));
    const float sc = group_scale<QF>(amax);
    s[g] = sc;
    for (int k8 = 0; k8 < kGroup; k8 += 8) {
        float v[8];
        int qv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = xg[k8 + k];
        quant8<QF>(v, sc, qv);
#pragma unroll
        for (int k = 0; k < 8; k++) q[g * kGroup + k8 + k] = (int8_t)qv[k];
    }
}

// out[c * out_ld + r] = in[r][c], 32x32 tiles through LDS.
__global__ __launch_bounds__(kThreads) void k_transpose(const float* __restrict__ in, float* __restrict__ out, int rows,
                                                        int cols, int out_ld) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    for (int i = threadIdx.x; i < 32 * 32; i += kThreads) {
        const int r = r0 + i / 32, c = c0 + i % 32;
        if (r < rows && c < cols) tile[i / 32][i % 32] = in[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 32 * 32; i += kThreads) {
        const int c = c0 + i / 32, r = r0 + i % 32;
        if (r < rows && c < cols) out[(size_t)c * out_ld + r] = tile[i % 32][i / 32];
    }
}

// RoPE on q [batch][n_heads*hd] and k [batch][n_kv_heads*hd] at positions
// pos+t, one thread per (head, pair).
__global__ void k_rope(const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                       const StepState* __restrict__ st, float* __restrict__ q, float* __restrict__ k,
                       int n_heads, int n_kv_heads, int hd) {
    const int t = blockIdx.y;
    const int half = hd / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int nq = n_heads * half, nk = n_kv_heads * half;
    if (i >= nq + nk) return;
    const int pos = st->pos + t;
    const int pair = (i < nq ? i : i - nq) % half;
    const float c = cos_t[(size_t)pos * half + pair], s = sin_t[(size_t)pos * half + pair];
    float* v = i < nq ? q + (size_t)t * n_heads * hd + 2 * (size_t)i
                      : k + (size_t)t * n_kv_heads * hd + 2 * (size_t)(i - nq);
    const float v0 = v[0], v1 = v[1];
    v[0] = fmul(v0, c) - fmul(v1, s);
    v[1] = fadd(fmul(v0, s), fmul(v1, c));
}

// SwiGLU + group quantization: one 32-lane half-wave per 32-group of hidden.
template <int QF>
__global__ void k_swiglu_quant(const float* __restrict__ gate, const float* __restrict__ up, int hidden,
                               float* __restrict__ h_f32, int8_t* __restrict__ hq, float* __restrict__ hs) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = i < hidden;
    const size_t off = (size_t)t * hidden + (live ? i : 0);
    float h = 0.0f;
    if (live) {
        const float g = gate[off];
        const float den = fadd(1.0f, expf_rn(-g));
        h = fmul(g / den, up[off]);
        if (h_f32) h_f32[off] = h;
    }
    if constexpr (QF >= 0) {
        float am = live ? fabsf(h) : 0.0f;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 32));
        am = fmaxf(am, 0.0f);
        const float sc = group_scale<QF>(am);
        if (live) {
            hq[off] = (int8_t)quant_one<QF>(h, sc);
            if ((i & 31) == 0) hs[(size_t)t * (hidden / kGroup) + i / kGroup] = sc;
        }
    }
}

// Elementwise probes of the device arithmetic the forward path depends on:
// exp (expf_rn), correctly rounded sqrt and division, f16 widening.
__global__ void k_math_selftest(const float* __restrict__ x, int n, float* exp_out, float* sqrt_out,
                                float* div_out, float* f16_out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    exp_out[i] = expf_rn(v);
    sqrt_out[i] = sqrtf(fabsf(v));
    div_out[i] = 1.0f / v;
    f16_out[i] = f16_to_f32((uint16_t)(i & 0xffff));
}

// One wavefront per case: the serial sum of v[offs[c] .. offs[c+1]), in one
// call (seg 0) or in consecutive segments of seg values, each continuing
// from the previous segment's sum.
__global__ __launch_bounds__(64) void k_serial_sum_selftest(const float* __restrict__ v,
                                                            const uint32_t* __restrict__ offs, int seg, float* out) {
    const int c = blockIdx.x;
    const uint32_t a = offs[c], b = offs[c + 1];
    const int n = (int)(b - a);
    float s;
    if (seg <= 0) {
        s = wave_serial_sum(v + a, n);
    } else {
        s = 0.0f;
        for (int i = 0; i < n; i += seg) s = wave_serial_sum(v + a + i, min(seg, n - i), s);
    }
    if (threadIdx.x == 0) out[c] = s;
}

// seg_serial_sum (the decode attention's softmax denominator) over one case
// per workgroup of 4 wavefronts: the values staged into LDS with +0 up to
// the next multiple of 64, as the attention's exponential row holds them.
constexpr int kSegSumWaves = 4;
__global__ __launch_bounds__(64 * kSegSumWaves) void k_seg_sum_selftest(const float* __restrict__ v,
                                                                        const uint32_t* __restrict__ offs,
                                                                        float* out, unsigned* fault) {
    extern __shared__ __align__(16) float lds[];
    const int c = blockIdx.x;
    const uint32_t a = offs[c], b = offs[c + 1];
    const int n = (int)(b - a), pad = (n + 63) & ~63;
    float* sx = lds + pad;
    double* segsum = reinterpret_cast<double*>(sx + 2 * kSegSumWaves * 65);
    int* ctr = reinterpret_cast<int*>(segsum + 2 * kSegSumWaves);
    for (int i = threadIdx.x; i < pad; i += blockDim.x) lds[i] = i < n ? v[a + i] : 0.0f;
    if (threadIdx.x == 0) *ctr = 0;
    __syncthreads();
    seg_sums_f64<kSegSumWaves>(lds, n, segsum);
    __syncthreads();
    const float s = seg_serial_sum<kSegSumWaves>(lds, n, segsum, sx, ctr, 0, fault);
    if (threadIdx.x == 0) out[c] = s;
}

// seg_serial_sum_wide (the long-context softmax denominator) over one case
// per workgroup of 8 wavefronts, the values staged as the softmax kernel
// stages them (+0 up to the next multiple of 64).
constexpr int kSegSumWideWaves = 8;
__global__ __launch_bounds__(64 * kSegSumWideWaves) void k_seg_sum_wide_selftest(const float* __restrict__ v,
                                                                                 const uint32_t* __restrict__ offs,
                                                                                 float* out, unsigned* fault) {
    extern __shared__ __align__(16) float lds[];
    const int c = blockIdx.x;
    const uint32_t a = offs[c], b = offs[c + 1];
    const int n = (int)(b - a), pad = (n + 63) & ~63;
    float* sx = lds + pad + 64;
    double* segsum = reinterpret_cast<double*>(sx + 16 * 64 + 8);
    int* ctr = reinterpret_cast<int*>(segsum + kSegSumWideWaves);
    for (int i = threadIdx.x; i < pad + 64; i += blockDim.x) lds[i] = i < n ? v[a + i] : 0.0f;
    if (threadIdx.x == 0) *ctr = 0;
    __syncthreads();
    seg_sums_f64_wide<kSegSumWideWaves>(lds, n, segsum);
    __syncthreads();
    const float s = seg_serial_sum_wide<kSegSumWideWaves>(lds, n, segsum, sx, ctr, 0, fault);
    if (threadIdx.x == 0) out[c] = s;
}

// The step state of an op call: its first position (and token).
__global__ void k_set_state(StepState* st, int32_t pos, uint32_t token) {
    if (threadIdx.x == 0) {
        st->pos = pos;
        st->token = token;
        st->n_out = 0;
        st->logits_done = 0;
        st->argmax = 0ull;
    }
}

// A plain stream of two byte ranges (a GEMV class's weights and scales): each
// workgroup reads its contiguous slice of each with 16-byte non-temporal
// loads (as the GEMV), every lane issuing up to 16 loads before it uses any;
// the loaded words reach memory only through a comparison that is never
// true in practice, so no load is dropped.  Measurement only.
typedef unsigned int stream_u4 __attribute__((ext_vector_type(4)));
constexpr int kStreamAhead = 16;
__global__ __launch_bounds__(1024) void k_stream(const stream_u4* __restrict__ a, size_t na,
                                                 const stream_u4* __restrict__ b, size_t nb, unsigned* __restrict__ sink) {
    uint32_t x = 0;
    for (int part = 0; part < 2; part++) {
        const stream_u4* p = part ? b : a;
        const size_t n = part ? nb : na;
        const size_t per = (n + gridDim.x - 1) / gridDim.x;
        const size_t lo = (size_t)blockIdx.x * per, hi = lo + per < n ? lo + per : n;
        for (size_t i0 = lo + threadIdx.x; i0 < hi; i0 += (size_t)kStreamAhead * blockDim.x) {
            stream_u4 v[kStreamAhead];
#pragma unroll
            for (int k = 0; k < kStreamAhead; k++) {
                const size_t i = i0 + (size_t)k * blockDim.x;
                v[k] = __builtin_nontemporal_load(p + (i < hi ? i : i0));
            }
#pragma unroll
            for (int k = 0; k < kStreamAhead; k++)
                if (i0 + (size_t)k * blockDim.x < hi) x ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        }
    }
    if (x == 0x9e3779b9u) sink[blockIdx.x] = x;
}

// ------------------------------------------------------------- launchers --

hipError_t launch_stream(const void* a, size_t abytes, const void* b, size_t bbytes, int grid, int threads,
                         unsigned* sink, hipStream_t s) {
    if (grid <= 0 || threads <= 0 || threads > 1024 || threads % 64 || (size_t)grid > abytes / 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_stream, dim3(grid), dim3(threads), 0, s, reinterpret_cast<const stream_u4*>(a), abytes / 16,
                       reinterpret_cast<const stream_u4*>(b), bbytes / 16, sink);
    return hipGetLastError();
}

hipError_t launch_set_state(StepState* st, int32_t pos, uint32_t token, hipStream_t s) {
    hipLaunchKernelGGL(k_set_state, dim3(1), dim3(64), 0, s, st, pos, token);
    return hipGetLastError();
}

hipError_t launch_quantize(int fmt, int8_t* q, float* scale, const float* x, size_t n, hipStream_t s) {
    const size_t groups = n / kGroup;
    if (groups == 0) return hipSuccess;
    const dim3 grid((unsigned)((groups + kThreads - 1) / kThreads));
    if (fmt == kQ8) hipLaunchKernelGGL((k_quantize<kQ8>), grid, dim3(kThreads), 0, s, q, scale, x, groups);
    else if (fmt == kQ4) hipLaunchKernelGGL((k_quantize<kQ4>), grid, dim3(kThreads), 0, s, q, scale, x, groups);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_rmsnorm(int qfmt, const float* x, const float* w, int dim, float eps, int batch, float* xn,
                          int8_t* xq, float* xs, hipStream_t s) {
    if (dim > 8192) return hipErrorInvalidValue;
    const size_t smem = norm_lds_floats(dim) * sizeof(float);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_rmsnorm<kQ8>), dim3(batch), dim3(kThreads), smem, s, x, w, dim, eps, xn, xq, xs);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_rmsnorm<kQ4>), dim3(batch), dim3(kThreads), smem, s, x, w, dim, eps, xn, xq, xs);
    else
        hipLaunchKernelGGL((k_rmsnorm<-1>), dim3(batch), dim3(kThreads), smem, s, x, w, dim, eps, xn, xq, xs);
    return hipGetLastError();
}

hipError_t launch_transpose(const float* in, float* out, int rows, int cols, int out_ld, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (out_ld < rows) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_transpose, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(kThreads), 0, s, in, out, rows, cols,
                       out_ld);
    return hipGetLastError();
}

hipError_t launch_embed(const EmbQ8& e, const uint32_t* tokens, int batch, float* x, hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3(batch), dim3(kThreads), 0, s, e, tokens, x);
    return hipGetLastError();
}

hipError_t launch_rope(const float* cos_t, const float* sin_t, const StepState* st, int batch, float* q, float* k,
                       int n_heads, int n_kv_heads, int head_size, hipStream_t s) {
    const int items = (n_heads + n_kv_heads) * (head_size / 2);
    const dim3 grid((items + kThreads - 1) / kThreads, batch);
    hipLaunchKernelGGL(k_rope, grid, dim3(kThreads), 0, s, cos_t, sin_t, st, q, k, n_heads, n_kv_heads, head_size);
    return hipGetLastError();
}

hipError_t launch_swiglu_quant(int qfmt, const float* gate, const float* up, int hidden, int batch, float* h_f32,
                               int8_t* hq, float* hs, hipStream_t s) {
    const dim3 grid((hidden + kThreads - 1) / kThreads, batch);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_swiglu_quant<kQ8>), grid, dim3(kThreads), 0, s, gate, up, hidden, h_f32, hq, hs);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_swiglu_quant<kQ4>), grid, dim3(kThreads), 0, s, gate, up, hidden, h_f32, hq, hs);
    else
        hipLaunchKernelGGL((k_swiglu_quant<-1>), grid, dim3(kThreads), 0, s, gate, up, hidden, h_f32, hq, hs);
    return hipGetLastError();
}

hipError_t launch_math_selftest(const float* x, int n, float* exp_out, float* sqrt_out, float* div_out,
                                float* f16_out, hipStream_t s) {
    hipLaunchKernelGGL(k_math_selftest, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, x, n, exp_out,
                       sqrt_out, div_out, f16_out);
    return hipGetLastError();
}

// what a bounded wait that gives up does to the fault word
__global__ void k_raise_fault(unsigned* fault) {
    if (threadIdx.x == 0) __hip_atomic_store(fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
hipError_t launch_raise_fault(unsigned* fault, hipStream_t s) {
    hipLaunchKernelGGL(k_raise_fault, dim3(1), dim3(64), 0, s, fault);
    return hipGetLastError();
}

hipError_t launch_serial_sum_selftest(const float* v, const uint32_t* offs, int cases, int seg, float* out,
                                      hipStream_t s) {
    if (cases <= 0) return hipSuccess;
    if (seg == -2) {
        // the wide segmented sum: LDS for the longest case
        std::vector<uint32_t> h((size_t)cases + 1);
        hipError_t e = hipMemcpy(h.data(), offs, h.size() * sizeof(uint32_t), hipMemcpyDeviceToHost);
        if (e != hipSuccess) return e;
        uint32_t mx = 0;
        for (int c = 0; c < cases; c++) mx = std::max(mx, h[c + 1] - h[c]);
        const size_t smem = ((((size_t)mx + 63) & ~(size_t)63) + 64 + 16 * 64 + 8 + 2 * kSegSumWideWaves + 4) * 4;
        if (smem > 150 * 1024) return hipErrorInvalidValue;
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_seg_sum_wide_selftest),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_seg_sum_wide_selftest, dim3(cases), dim3(64 * kSegSumWideWaves), smem, s, v, offs, out,
                           wait_fault_word(false));
        return hipGetLastError();
    }
    if (seg < 0) {
        // the segmented sum: LDS for the longest case
        std::vector<uint32_t> h((size_t)cases + 1);
        hipError_t e = hipMemcpy(h.data(), offs, h.size() * sizeof(uint32_t), hipMemcpyDeviceToHost);
        if (e != hipSuccess) return e;
        uint32_t mx = 0;
        for (int c = 0; c < cases; c++) mx = std::max(mx, h[c + 1] - h[c]);
        const size_t smem = (((size_t)mx + 63) & ~(size_t)63) * 4 + (2 * kSegSumWaves * 65 + 4 * kSegSumWaves + 4) * 4;
        if (smem > 150 * 1024) return hipErrorInvalidValue;
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_seg_sum_selftest),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_seg_sum_selftest, dim3(cases), dim3(64 * kSegSumWaves), smem, s, v, offs, out,
                           wait_fault_word(false));
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_serial_sum_selftest, dim3(cases), dim3(64), 0, s, v, offs, seg, out);
    return hipGetLastError();
}

}  // namespace yl
