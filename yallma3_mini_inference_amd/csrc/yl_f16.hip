// yl_f16.hip -- the F16 weight format (WeightFormat::F16, weight_type.rs:17-22):
// matmul_f32 (weight_type.rs:228-270) on f16 weights, and the QKV step of
// the F16 forward pass (forward.rs:149-179 with the F16Kernel, whose
// quantize is a copy and whose matmul assigns every column).
//
// matmul_f32 sums each output column in one f32 accumulator, in column
// order: sum = ((x[0]*w[0] + x[1]*w[1]) + ...), every product and every add
// rounded on its own.  The weights are binary16 on disk and exactly binary32
// in the reference's memory, so the device keeps them as f16 (half the
// bytes) and widens them exactly.  Each output is one lane's serial chain;
// the kernels keep that chain fed:
//   decode (one token): four product wavefronts multiply a 64-row x 64-column
//   weight tile by the activations into LDS while a fifth wavefront adds the
//   previous tile's products into its 64 row accumulators, so the chain wave
//   issues one LDS read per four adds;
//   batches: a workgroup takes 64 rows x 4 tokens, one wavefront per token,
//   each lane multiplying and adding its own (token, row) chain, the weight
//   tile shared through LDS.
#include <hip/hip_runtime.h>

#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kF16Rows = 64;     // output rows per workgroup
constexpr int kF16Cols = 64;     // columns per tile
constexpr int kF16Tok = 4;       // tokens per workgroup (batched kernel)

__device__ __forceinline__ float h2f(uint32_t bits16) { return f16_to_f32((uint16_t)bits16); }

// 8 halves of a uint4 -> w[8]
__device__ __forceinline__ void widen8(const uint4& v, float w[8]) {
    w[0] = h2f(v.x & 0xffffu); w[1] = h2f(v.x >> 16);
    w[2] = h2f(v.y & 0xffffu); w[3] = h2f(v.y >> 16);
    w[4] = h2f(v.z & 0xffffu); w[5] = h2f(v.z >> 16);
    w[6] = h2f(v.w & 0xffffu); w[7] = h2f(v.w >> 16);
}

// ------------------------------------------------------------- one token
// 320 threads: waves 0-3 make products, wave 4 holds the accumulators.
// LDS: x [n] f32, then two product buffers P[16][64] of float4 (column group
// c4 of row r at P[c4][r]: the chain lane reads 16 contiguous bytes, the 64
// lanes 1 KiB).
template <int EPI>
__global__ __launch_bounds__(320) void k_matmul_f16_tok1(const uint16_t* __restrict__ w, int n, int o,
                                                         const float* __restrict__ x, float* __restrict__ out) {
    extern __shared__ __align__(16) float lds[];
    float* xl = lds;
    vf4* P = reinterpret_cast<vf4*>(lds + ((n + 3) & ~3));
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = blockIdx.x * kF16Rows;
    for (int i = tid; i < n; i += 320) xl[i] = x[i];
    __syncthreads();
    const int ntile = (n + kF16Cols - 1) / kF16Cols;
    // product thread t: row r = t / 4, columns (t % 4) * 16 .. + 16 of the tile
    const int pr = tid >> 2, pq = tid & 3;
    const int prow = min(row0 + pr, o - 1);
    const uint16_t* wrow = w + (size_t)prow * n;
    float acc = 0.0f;
    uint4 wv[2];
    auto load = [&](int t) {
        const int k = t * kF16Cols + pq * 16;
        const int kc = min(k, n - 16 < 0 ? 0 : n - 16);   // a partial tile re-reads in range
        const uint4* src = reinterpret_cast<const uint4*>(wrow + (k < n ? k : kc));
        wv[0] = src[0];
        wv[1] = src[1];
    };
    auto products = [&](int t, vf4* buf) {
        const int k0 = t * kF16Cols + pq * 16;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float wf[8];
            widen8(wv[h], wf);
#pragma unroll
            for (int g = 0; g < 2; g++) {
                const int k = k0 + h * 8 + g * 4;
                vf4 p;
                p.x = k + 0 < n ? fmul(xl[k + 0], wf[g * 4 + 0]) : 0.0f;
                p.y = k + 1 < n ? fmul(xl[k + 1], wf[g * 4 + 1]) : 0.0f;
                p.z = k + 2 < n ? fmul(xl[k + 2], wf[g * 4 + 2]) : 0.0f;
                p.w = k + 3 < n ? fmul(xl[k + 3], wf[g * 4 + 3]) : 0.0f;
                buf[(pq * 4 + h * 2 + g) * kF16Rows + pr] = p;
            }
        }
    };
    if (wave < 4) {
        load(0);
        products(0, P);
    }
    __syncthreads();
    for (int t = 0; t < ntile; t++) {
        vf4* cur = P + (t & 1) * 16 * kF16Rows;
        vf4* nxt = P + ((t + 1) & 1) * 16 * kF16Rows;
        if (wave < 4) {
            if (t + 1 < ntile) {
                load(t + 1);
                products(t + 1, nxt);
            }
        } else {
            const int kn = min(kF16Cols, n - t * kF16Cols);   // columns in this tile (a multiple of 4)
            for (int c4 = 0; c4 < kn / 4; c4++) {
                const vf4 p = cur[c4 * kF16Rows + lane];
                acc = fadd(acc, p.x);
                acc = fadd(acc, p.y);
                acc = fadd(acc, p.z);
                acc = fadd(acc, p.w);
            }
        }
        __syncthreads();
    }
    if (wave == 4 && row0 + lane < o) {
        float* dst = out + row0 + lane;
        *dst = EPI == 0 ? acc : fadd(*dst, acc);
    }
}

// --------------------------------------------------------------- batches
// 256 threads: wave t takes token blockIdx.y * 4 + t over the workgroup's
// 64 rows.  LDS: the weight tile transposed to [8 chunks][64 rows][8
// halves], double-buffered, and the 4 tokens' activation tiles.
template <int EPI>
__global__ __launch_bounds__(256) void k_matmul_f16_batch(const uint16_t* __restrict__ w, int n, int o,
                                                          const float* __restrict__ x, int batch,
                                                          float* __restrict__ out, int out_ld) {
    __shared__ __align__(16) uint4 wt[2][8 * kF16Rows];
    __shared__ __align__(16) float xt[2][kF16Tok * kF16Cols];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = blockIdx.x * kF16Rows;
    const int tok = blockIdx.y * kF16Tok + wave;
    const int ntile = (n + kF16Cols - 1) / kF16Cols;
    // loader thread t: chunk c = t % 8 of rows t / 8 and t / 8 + 32; x: float4 t % 16 of token t / 16
    const int lc = tid & 7, lr = tid >> 3;
    uint4 wreg[2];
    vf4 xreg;
    auto load = [&](int t) {
        const int k = t * kF16Cols + lc * 8;
        const int kk = k < n ? k : n - 8;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int r = min(row0 + lr + 32 * h, o - 1);
            wreg[h] = *reinterpret_cast<const uint4*>(w + (size_t)r * n + kk);
        }
        const int xtok = blockIdx.y * kF16Tok + (tid >> 4), xk = t * kF16Cols + (tid & 15) * 4;
        xreg = vf4{0.0f, 0.0f, 0.0f, 0.0f};
        if (tid < 64 && xtok < batch && xk < n) xreg = *reinterpret_cast<const vf4*>(x + (size_t)xtok * n + xk);
    };
    auto store = [&](int b) {
#pragma unroll
        for (int h = 0; h < 2; h++) wt[b][lc * kF16Rows + lr + 32 * h] = wreg[h];
        if (tid < 64) *reinterpret_cast<vf4*>(&xt[b][(tid >> 4) * kF16Cols + (tid & 15) * 4]) = xreg;
    };
    load(0);
    store(0);
    __syncthreads();
    float acc = 0.0f;
    for (int t = 0; t < ntile; t++) {
        const int b = t & 1;
        if (t + 1 < ntile) load(t + 1);
        const int kn = min(kF16Cols, n - t * kF16Cols);
        for (int c = 0; c < kn / 8; c++) {
            float wf[8];
            widen8(wt[b][c * kF16Rows + lane], wf);
            const float* xk = &xt[b][wave * kF16Cols + c * 8];
#pragma unroll
            for (int j = 0; j < 8; j++) acc = fadd(acc, fmul(xk[j], wf[j]));
        }
        if (t + 1 < ntile) store(b ^ 1);
        __syncthreads();
    }
    if (tok < batch && row0 + lane < o) {
        float* dst = out + (size_t)tok * out_ld + row0 + lane;
        *dst = EPI == 0 ? acc : fadd(*dst, acc);
    }
}

// ------------------------------------------------------------------ QKV
// raw [batch][att + 2 kv] (q | k | v rows of the fused projection) ->
// RoPE on q and k (util.rs:653-718 pairs (2i, 2i+1) of each head; util.rs
// rope, HF layout, pairs (j, j + head/2)) with the angles of position
// pos + t, q to sq, k and v assigned into the caches (keys transposed).
__global__ void k_qkv_f16(const float* __restrict__ raw, const float* __restrict__ cos_t,
                          const float* __restrict__ sin_t, const StepState* __restrict__ st, float* __restrict__ sq,
                          float* __restrict__ kc, float* __restrict__ vc, int att, int kv, int hd, int kv_ld,
                          int hf_pairs) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2;
    const int nq = att / 2, nk = kv / 2;
    const int pos = st->pos + t;
    const float* r = raw + (size_t)t * (att + 2 * kv);
    if (i < nq + nk) {
        const bool isq = i < nq;
        const int p = isq ? i : i - nq;            // pair index within q or k
        const int head = p / half, j = p % half;
        const int e0 = head * hd + (hf_pairs ? j : 2 * j), e1 = e0 + (hf_pairs ? half : 1);
        const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
        const float* src = isq ? r : r + att;
        const float v0 = src[e0], v1 = src[e1];
        const float a = fmul(v0, c) - fmul(v1, s);
        const float b = fadd(fmul(v0, s), fmul(v1, c));
        if (isq) {
            sq[(size_t)t * att + e0] = a;
            sq[(size_t)t * att + e1] = b;
        } else {
            kc[(size_t)e0 * kv_ld + pos] = a;
            kc[(size_t)e1 * kv_ld + pos] = b;
        }
    } else if (i < nq + nk + kv) {
        const int e = i - nq - nk;
        vc[(size_t)pos * kv + e] = r[att + kv + e];
    }
}

size_t matmul_f16_lds_bytes(int n) { return ((size_t)((n + 3) & ~3) + 2 * 16 * kF16Rows * 4) * sizeof(float); }

hipError_t launch_matmul_f16(const uint16_t* w, int n, int o, const float* x, int batch, float* out, int out_ld,
                             int epi, hipStream_t s) {
    if (n % 32 || n <= 0 || o <= 0 || batch <= 0) return hipErrorInvalidValue;
    const int rb = (o + kF16Rows - 1) / kF16Rows;
    if (batch == 1) {
        const size_t lds = matmul_f16_lds_bytes(n);
        auto k = epi == 0 ? k_matmul_f16_tok1<0> : k_matmul_f16_tok1<1>;
        if (lds > 65536) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k, dim3(rb), dim3(320), lds, s, w, n, o, x, out);
    } else {
        auto k = epi == 0 ? k_matmul_f16_batch<0> : k_matmul_f16_batch<1>;
        hipLaunchKernelGGL(k, dim3(rb, (batch + kF16Tok - 1) / kF16Tok), dim3(256), 0, s, w, n, o, x, batch, out,
                           out_ld);
    }
    return hipGetLastError();
}

hipError_t launch_qkv_f16(const float* raw, const float* cos_t, const float* sin_t, const StepState* st, int batch,
                          float* sq, float* kc, float* vc, int att, int kv, int hd, int kv_ld, int hf_pairs,
                          hipStream_t s) {
    const int n = att / 2 + kv / 2 + kv;
    hipLaunchKernelGGL(k_qkv_f16, dim3((n + 255) / 256, batch), dim3(256), 0, s, raw, cos_t, sin_t, st, sq, kc, vc,
                       att, kv, hd, kv_ld, hf_pairs);
    return hipGetLastError();
}

}  // namespace yl
