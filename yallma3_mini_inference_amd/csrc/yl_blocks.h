// yl_blocks.h -- workgroup-level building blocks shared by the kernels.
#pragma once

#include "yl_device.h"

namespace yl {

// Row stride (floats) of the transposed RMSNorm layout: lane chain j of the
// f32x8 accumulator reads its elements x[8i+j] contiguously at xt[j*S + i].
// S is a multiple of 4 (float4 reads) and S % 32 == 4 or 12 or 20 ... so the
// 8 chain lanes hit distinct LDS banks.
__host__ __device__ inline int norm_stride(int dim) { return (((dim / 8) + 3) & ~3) + 4; }
// transposed row 8*S | reduction 16 | norm weights dim
__host__ __device__ inline size_t norm_lds_floats(int dim) { return (size_t)8 * norm_stride(dim) + 16 + dim; }

// Position of element i inside the activation staging buffer of a Q4_0
// matmul: each 8-group is stored as its 4 even elements then its 4 odd ones,
// matching the low/high nibbles of one weight dword.
__device__ __forceinline__ int q4_pos(int i) {
    const int k = i & 7;
    return (i & ~7) | ((k & 1) ? 4 + (k >> 1) : (k >> 1));
}

// RMSNorm of one row (util.rs:389-426) followed by group quantization.
//   xt  : LDS, norm_lds_floats(dim); the row and the norm weights must
//         already be stored there by store_norm_input() (transposed row, so
//         the serial lane chains read float4s without waiting on HBM).
//   QF  : kQ8 / kQ4 -> q_lds/s_lds receive the quantized row (Q4 reordered
//         when PERM); QF < 0 -> no quantization.
//   xn  : optional f32 output of the normalized row (global or LDS).
// The 8 lane sums run as 8 serial chains (one lane each) over float4 reads;
// normalization and quantization use every thread, one element per thread,
// a 32-group per half-wave (absmax by shuffles: order-free max).
// Stores element i of the row (v) and of the norm weight (w) for the block.
__device__ __forceinline__ void store_norm_input(float* xt, int dim, int i, float v, float w) {
    const int n8 = (dim / 8) * 8;
    const int S = norm_stride(dim);
    if (i < n8) xt[(i & 7) * S + (i >> 3)] = v;
    xt[8 * S + 16 + i] = w;
}

template <int QF, bool PERM>
__device__ void rmsnorm_quant_block(float* xt, int dim, float eps, int8_t* q_lds, float* s_lds, float* xn) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int S = norm_stride(dim);
    const int n_simd = dim / 8;
    float* red = xt + 8 * S;
    const float* wl = red + 16;
    if (tid < 8) {
        const float* row = xt + tid * S;
        float l = 0.0f;
        int m = 0;
        const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll 16
        for (; m < n_simd / 4; m++) {
            const float4 v = r4[m];
            l = fadd(l, fmul(v.x, v.x));
            l = fadd(l, fmul(v.y, v.y));
            l = fadd(l, fmul(v.z, v.z));
            l = fadd(l, fmul(v.w, v.w));
        }
        for (int i = m * 4; i < n_simd; i++) l = fadd(l, fmul(row[i], row[i]));
        red[tid] = l;
    }
    __syncthreads();
    float part[8];
#pragma unroll
    for (int j = 0; j < 8; j++) part[j] = red[j];
    float ss = reduce_add8(part);
    ss = ss / (float)dim;
    ss = fadd(ss, eps);
    ss = 1.0f / sqrtf(ss);
    const int n8 = n_simd * 8;
    const int rounds = (dim + nthr - 1) / nthr;
    for (int rd = 0; rd < rounds; rd++) {
        const int i = rd * nthr + tid;
        float v = 0.0f;
        if (i < n8) v = fmul(wl[i], fmul(ss, xt[(i & 7) * S + (i >> 3)]));
        if (xn && i < dim) xn[i] = v;
        if constexpr (QF >= 0) {
            // groups of 32 never straddle `dim` (dim % 32 == 0 when quantizing)
            float am = fabsf(v);
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 32));
            am = fmaxf(am, 0.0f);
            const float sc = group_scale<QF>(am);
            if (i < dim) {
                q_lds[PERM ? q4_pos(i) : i] = (int8_t)quant_one<QF>(v, sc);
                if ((i & 31) == 0) s_lds[i >> 5] = sc;
            }
        }
    }
    __syncthreads();
}

}  // namespace yl
