// yl_q8g.hip -- Q8 weights with f32 block scales and any group size (a
// multiple of 32): the form the reference's lm.rs and safetensors loaders
// produce (util.rs:452-589: scales are f32, the group size comes from the
// file), beside the GGUF path's f16-scaled 32-blocks.
//
// matmul_q8_slices (weight_type.rs:122-226) per output column: the exact
// int32 dot of each group, then acc = acc + ((float)isum * w_scale) *
// x_scale in group order.  The accumulator starts from the output's old
// value for the first 4*floor(o/4) columns (`+=`) and from 0 for the rest
// (`=`); callers that zero the output first (forward.rs fills q, gate, up and
// the FFN output with 0) pass acc_cols = 0.  One lane per (column, token).
#include <hip/hip_runtime.h>

#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

// EPI 0: out = chain; EPI 1: out = out + chain-from-0 (the residual add of
// forward.rs:196-204 after a zeroed FFN output).
// Output element (token t, column c) at out[pos * pos_stride + t * stride_tok
// + c * stride_row], pos = st->pos (0 without a step state).
template <int EPI>
__global__ __launch_bounds__(64) void k_matmul_q8g(const int8_t* __restrict__ w, const float* __restrict__ wsc, int n,
                                                   int o, int gs, const int8_t* __restrict__ xq,
                                                   const float* __restrict__ xs, float* __restrict__ out,
                                                   const StepState* __restrict__ st, long pos_stride, long stride_row,
                                                   long stride_tok, int acc_cols) {
    extern __shared__ __align__(16) int xl[];
    const int t = blockIdx.y, lane = threadIdx.x;
    const int c = blockIdx.x * 64 + lane;
    const int* xr = reinterpret_cast<const int*>(xq + (size_t)t * n);
    for (int i = lane; i < n / 4; i += 64) xl[i] = xr[i];
    __syncthreads();
    if (c >= o) return;
    const int G = n / gs;
    const float* xsr = xs + (size_t)t * G;
    const int8_t* wr = w + (size_t)c * n;
    const float* wsr = wsc + (size_t)c * G;
    const size_t at = (st ? (size_t)st->pos * pos_stride : 0) + (size_t)t * stride_tok + (size_t)c * stride_row;
    float acc = (EPI == 0 && c < acc_cols) ? out[at] : 0.0f;
    for (int g = 0; g < G; g++) {
        int isum = 0;
        for (int k = 0; k < gs; k += 16) {
            const int4 wv = *reinterpret_cast<const int4*>(wr + (size_t)g * gs + k);
            const int* xv = xl + (g * gs + k) / 4;
            isum = __builtin_amdgcn_sdot4(wv.x, xv[0], isum, false);
            isum = __builtin_amdgcn_sdot4(wv.y, xv[1], isum, false);
            isum = __builtin_amdgcn_sdot4(wv.z, xv[2], isum, false);
            isum = __builtin_amdgcn_sdot4(wv.w, xv[3], isum, false);
        }
        acc = fadd(acc, fmul(fmul((float)isum, wsr[g]), xsr[g]));
    }
    out[at] = EPI == 0 ? acc : fadd(out[at], acc);
}

// quantization::quantize (quantization.rs:29-52) over `groups` groups of gs.
__global__ void k_quantize_gs(const float* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ s, int gs,
                              size_t groups) {
    const size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    const float* xg = x + g * gs;
    float amax = 0.0f;
    for (int k = 0; k < gs; k++) amax = fmaxf(amax, fabsf(xg[k]));
    const float sc = group_scale<kQ8>(amax);
    s[g] = sc;
    for (int k = 0; k < gs; k++) q[g * gs + k] = (int8_t)quant_one<kQ8>(xg[k], sc);
}

// RoPE in place on q [batch][att] and on the keys of positions pos..pos+batch-1
// in the transposed cache [kv][kv_ld]: pairs (2j, 2j+1) (util.rs:653-718) or
// (j, j + head/2) (util.rs rope), angles of the table [ctx][head/2].
__global__ void k_rope_cache(const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                             const StepState* __restrict__ st, float* __restrict__ q, float* __restrict__ kc, int att,
                             int kv, int hd, int kv_ld, int hf_pairs) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2, nq = att / 2, nk = kv / 2;
    if (i >= nq + nk) return;
    const int pos = st->pos + t;
    const bool isq = i < nq;
    const int p = isq ? i : i - nq;
    const int head = p / half, j = p % half;
    const int e0 = head * hd + (hf_pairs ? j : 2 * j), e1 = e0 + (hf_pairs ? half : 1);
    const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
    float* a0 = isq ? q + (size_t)t * att + e0 : kc + (size_t)e0 * kv_ld + pos;
    float* a1 = isq ? q + (size_t)t * att + e1 : kc + (size_t)e1 * kv_ld + pos;
    const float v0 = *a0, v1 = *a1;
    *a0 = fmul(v0, c) - fmul(v1, s);
    *a1 = fadd(fmul(v0, s), fmul(v1, c));
}

hipError_t launch_matmul_q8g(const int8_t* w, const float* wsc, int n, int o, int gs, const int8_t* xq,
                             const float* xs, int batch, float* out, const StepState* st, long pos_stride,
                             long stride_row, long stride_tok, int acc_cols, int epi, hipStream_t s) {
    if (gs <= 0 || gs % 32 || n % gs || batch <= 0 || batch > 65535) return hipErrorInvalidValue;
    const size_t lds = (size_t)n;
    auto k = epi == 0 ? k_matmul_q8g<0> : k_matmul_q8g<1>;
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, dim3((o + 63) / 64, batch), dim3(64), lds, s, w, wsc, n, o, gs, xq, xs, out, st, pos_stride,
                       stride_row, stride_tok, acc_cols);
    return hipGetLastError();
}

hipError_t launch_quantize_gs(const float* x, int8_t* q, float* sc, int gs, size_t n, hipStream_t s) {
    if (gs <= 0 || n % gs) return hipErrorInvalidValue;
    const size_t groups = n / gs;
    if (!groups) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_gs, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s, x, q, sc, gs, groups);
    return hipGetLastError();
}

hipError_t launch_rope_cache(const float* cos_t, const float* sin_t, const StepState* st, int batch, float* q,
                             float* kc, int att, int kv, int hd, int kv_ld, int hf_pairs, hipStream_t s) {
    const int n = att / 2 + kv / 2;
    hipLaunchKernelGGL(k_rope_cache, dim3((n + 255) / 256, batch), dim3(256), 0, s, cos_t, sin_t, st, q, kc, att, kv,
                       hd, kv_ld, hf_pairs);
    return hipGetLastError();
}

}  // namespace yl
