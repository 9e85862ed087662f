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
//   decode (one token): a workgroup owns 16 output rows.  Three product
//   wavefronts multiply a 16-row x 256-column weight tile by the activations
//   into LDS while the fourth wavefront's 16 lanes add the previous tile's
//   products onto their row accumulators, reading 16 bytes per four adds and
//   keeping two read batches in flight.  A chain of n dependent adds is the
//   kernel's floor (~n x 5.8 cycles), so the weight loads run four tiles
//   ahead in registers and many small workgroups share the chip.  The
//   prologue can apply RMSNorm (util.rs:389-426) to the input row, and the
//   epilogue add the residual or form SwiGLU from gate/up row pairs;
//   batches: a workgroup takes 64 rows x 4 tokens, one wavefront per token,
//   each lane multiplying and adding its own (token, row) chain, the weight
//   tile shared through LDS.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
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
constexpr int kFgThreads = 256;       // all wavefronts: products; wavefront 0 also the chains
constexpr int kFgRows = 16;           // output rows per workgroup (EPI 2: 8 gate rows, then their 8 up rows)
constexpr int kFgKT = 256;            // columns per tile
constexpr int kFgStride = kFgKT + 4;  // product row stride (floats)
constexpr int kFgDepth = 4;           // tiles of weight loads in flight
constexpr int kFgChunks = kFgRows * kFgKT / 8;                    // 16-byte weight chunks per tile
constexpr int kFgPer = kFgChunks / kFgThreads;                      // chunks per thread and tile
constexpr int kFgPairRows = kFgRows / 2;
static_assert(kFgChunks % kFgThreads == 0, "every thread takes whole chunks");

__host__ __device__ inline int fg_norm_len(int n) { return (n / 8 + 31) & ~31; }
__host__ __device__ inline int fg_norm_stride(int n) { return fg_norm_len(n) + 4; }
// LDS floats: x [n] | products 2 x [16][260] | (PRO 1) squares 8 x S, reduction 16, norm weights [n]
__host__ __device__ inline size_t fg_lds_floats(int n, int pro) {
    size_t f = (size_t)n + 2 * kFgRows * kFgStride;
    if (pro) f += (size_t)8 * fg_norm_stride(n) + 16 + n;
    return f;
}

// PRO 1: x <- RMSNorm(x) * norm_w first.  EPI 0: out[r] = sum; EPI 1: out[r]
// += sum (the residual add); EPI 2: out[8 * blockIdx.x + c] = silu(g) * u of
// rows (c, c + 8) of the tile (forward.rs:220-237).
template <int PRO, int EPI>
__global__ __launch_bounds__(kFgThreads) void k_f16_gemv(const uint16_t* __restrict__ w, int n, int o,
                                                         const float* __restrict__ x, const float* __restrict__ norm_w,
                                                         float eps, float* __restrict__ out) {
    extern __shared__ __align__(16) float lds[];
    float* xl = lds;                                   // [n]
    float* P = lds + n;                                // [2][16][260]
    float* sq = P + 2 * kFgRows * kFgStride;           // (PRO) squares, then reduction, then norm weights
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = blockIdx.x * kFgRows;
    const int ntile = (n + kFgKT - 1) / kFgKT;
    uint4 wr[kFgDepth][kFgPer];
    // chunk j = tid + 256 i of a tile: row j / 32, 8 columns from 8 * (j % 32).
    // Every load is issued unconditionally (tiles past the last and columns
    // past n re-read in range, unused), so the compiler's wait counts stay
    // exact: a consumer waits only for its own tile, not the ones behind it.
    auto load_tile = [&](uint4 (&dst)[kFgPer], int t) {
        const int k0 = min(t, ntile - 1) * kFgKT;
#pragma unroll
        for (int i = 0; i < kFgPer; i++) {
            const int j = tid + kFgThreads * i;
            const int k = min(k0 + 8 * (j & 31), n - 8);
            dst[i] = *reinterpret_cast<const uint4*>(w + (size_t)(row0 + (j >> 5)) * n + k);
        }
    };
#pragma unroll
    for (int d = 0; d < kFgDepth; d++) load_tile(wr[d], d);
    // the input row (RMSNorm first when PRO): 16-byte loads, 8 per thread in flight
    {
        const vf4* x4 = reinterpret_cast<const vf4*>(x);
        const vf4* w4 = reinterpret_cast<const vf4*>(norm_w);
        vf4* xl4 = reinterpret_cast<vf4*>(xl);
        const int S = fg_norm_stride(n), L8 = fg_norm_len(n), n8 = n / 8;
        float* red = sq + 8 * S;
        vf4* wn4 = reinterpret_cast<vf4*>(red + 16);
        for (int b = 0; b < n / 4; b += 8 * kFgThreads) {
            vf4 v[8], nv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i4 = b + k * kFgThreads + tid;
                if (i4 < n / 4) {
                    v[k] = x4[i4];
                    if constexpr (PRO) nv[k] = w4[i4];
                }
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i4 = b + k * kFgThreads + tid;
                if (i4 < n / 4) {
                    xl4[i4] = v[k];
                    if constexpr (PRO) {
                        wn4[i4] = nv[k];
                        const int e = i4 * 4;
                        sq[((e + 0) & 7) * S + (e >> 3)] = fmul(v[k].x, v[k].x);
                        sq[((e + 1) & 7) * S + (e >> 3)] = fmul(v[k].y, v[k].y);
                        sq[((e + 2) & 7) * S + (e >> 3)] = fmul(v[k].z, v[k].z);
                        sq[((e + 3) & 7) * S + (e >> 3)] = fmul(v[k].w, v[k].w);
                    }
                }
            }
        }
        if constexpr (PRO) {
            for (int i = tid; i < 8 * (L8 - n8); i += kFgThreads) sq[(i / (L8 - n8)) * S + n8 + i % (L8 - n8)] = 0.0f;
            __syncthreads();
            if (tid < 8) red[tid] = lds_serial_sum(reinterpret_cast<const vf4*>(sq + tid * S), L8 / 32, 0.0f);
            __syncthreads();
            float part[8];
#pragma unroll
            for (int j = 0; j < 8; j++) part[j] = red[j];
            float ss = reduce_add8(part);
            ss = ss / (float)n;
            ss = fadd(ss, eps);
            ss = 1.0f / sqrtf(ss);
            const float* wn = red + 16;
            for (int i = tid; i < n; i += kFgThreads) xl[i] = fmul(wn[i], fmul(ss, xl[i]));
        }
        __syncthreads();
    }

    float acc = 0.0f;
    // iteration t: products of tile t -> P[t & 1], then the loads of tile
    // t + depth into the freed registers; wavefront 0's first 16 lanes add
    // tile t - 1.  The trip count is padded to whole rings of `depth`.
    const int nit = (ntile + 1 + kFgDepth - 1) / kFgDepth * kFgDepth;
    for (int t0 = 0; t0 < nit; t0 += kFgDepth) {
#pragma unroll
        for (int d = 0; d < kFgDepth; d++) {
            const int t = t0 + d;
            if (t < ntile) {
                float* buf = P + (t & 1) * kFgRows * kFgStride;
                const int k0 = t * kFgKT;
#pragma unroll
                for (int i = 0; i < kFgPer; i++) {
                    const int j = tid + kFgThreads * i;
                    const int kk = 8 * (j & 31);
                    if (k0 + kk < n) {
                        float wf[8];
                        widen8(wr[d][i], wf);
                        const vf4 xa = *reinterpret_cast<const vf4*>(xl + k0 + kk);
                        const vf4 xb = *reinterpret_cast<const vf4*>(xl + k0 + kk + 4);
                        float* dst = buf + (j >> 5) * kFgStride + kk;
                        *reinterpret_cast<vf4*>(dst) =
                            vf4{fmul(xa.x, wf[0]), fmul(xa.y, wf[1]), fmul(xa.z, wf[2]), fmul(xa.w, wf[3])};
                        *reinterpret_cast<vf4*>(dst + 4) =
                            vf4{fmul(xb.x, wf[4]), fmul(xb.y, wf[5]), fmul(xb.z, wf[6]), fmul(xb.w, wf[7])};
                    }
                }
            }
            load_tile(wr[d], t + kFgDepth);
            if (wave == 0 && lane < kFgRows && t >= 1 && t <= ntile) {
                const int tp = t - 1;
                const int kn = min(kFgKT, n - tp * kFgKT);   // a multiple of 32
                acc = lds_serial_sum(reinterpret_cast<const vf4*>(P + (tp & 1) * kFgRows * kFgStride + lane * kFgStride),
                                     kn / 32, acc);
            }
            __syncthreads();
        }
    }
    if (wave == 0) {
        if constexpr (EPI == 2) {
            const float u = __shfl_down(acc, kFgPairRows, 64);
            if (lane < kFgPairRows) {
                const float den = fadd(1.0f, expf_rn(-acc));
                out[blockIdx.x * kFgPairRows + lane] = fmul(acc / den, u);
            }
        } else if (lane < kFgRows) {
            float* dst = out + row0 + lane;
            *dst = EPI == 0 ? acc : fadd(*dst, acc);
        }
    }
}

// SwiGLU of a batched gate/up product in the pair layout (rows c, c + 8 of
// each 16-row block): raw [batch][2 * hidden] -> h [batch][hidden].
__global__ void k_swiglu_pairs(const float* __restrict__ raw, int hidden, float* __restrict__ h) {
    const int t = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= hidden) return;
    const float* r = raw + (size_t)t * 2 * hidden + (size_t)(c / kFgPairRows) * kFgRows + c % kFgPairRows;
    const float g = r[0], u = r[kFgPairRows];
    const float den = fadd(1.0f, expf_rn(-g));
    h[(size_t)t * hidden + c] = fmul(g / den, u);
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

hipError_t launch_matmul_f16(const uint16_t* w, int n, int o, const float* x, int batch, float* out, int out_ld,
                             int epi, hipStream_t s) {
    if (n % 32 || n <= 0 || o <= 0 || batch <= 0 || epi < 0 || epi > 1) return hipErrorInvalidValue;
    if (batch == 1 && o % kFgRows == 0) return launch_f16_gemv(w, n, o, x, nullptr, 0.0f, epi, out, s);
    const int rb = (o + kF16Rows - 1) / kF16Rows;
    auto k = epi == 0 ? k_matmul_f16_batch<0> : k_matmul_f16_batch<1>;
    hipLaunchKernelGGL(k, dim3(rb, (batch + kF16Tok - 1) / kF16Tok), dim3(256), 0, s, w, n, o, x, batch, out, out_ld);
    return hipGetLastError();
}

template <int PRO, int EPI>
static hipError_t launch_fg(const uint16_t* w, int n, int o, const float* x, const float* norm_w, float eps,
                            float* out, hipStream_t s) {
    const size_t lds = fg_lds_floats(n, PRO) * sizeof(float);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    auto k = k_f16_gemv<PRO, EPI>;
    static bool raised = false;
    if (lds > 65536 && !raised) {
        const hipError_t e =
            hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        raised = true;
    }
    hipLaunchKernelGGL(k, dim3(o / kFgRows), dim3(kFgThreads), lds, s, w, n, o, x, norm_w, eps, out);
    return hipGetLastError();
}

hipError_t launch_f16_gemv(const uint16_t* w, int n, int o, const float* x, const float* norm_w, float eps, int epi,
                           float* out, hipStream_t s) {
    if (n % 32 || n <= 0 || o <= 0 || o % kFgRows || epi < 0 || epi > 2) return hipErrorInvalidValue;
    if (norm_w) {
        if (epi == 0) return launch_fg<1, 0>(w, n, o, x, norm_w, eps, out, s);
        if (epi == 2) return launch_fg<1, 2>(w, n, o, x, norm_w, eps, out, s);
        return hipErrorInvalidValue;
    }
    if (epi == 0) return launch_fg<0, 0>(w, n, o, x, norm_w, eps, out, s);
    if (epi == 1) return launch_fg<0, 1>(w, n, o, x, norm_w, eps, out, s);
    return launch_fg<0, 2>(w, n, o, x, norm_w, eps, out, s);
}

hipError_t launch_swiglu_pairs(const float* raw, int hidden, int batch, float* h, hipStream_t s) {
    if (hidden % kFgPairRows || batch <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_swiglu_pairs, dim3((hidden + 255) / 256, batch), dim3(256), 0, s, raw, hidden, h);
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
