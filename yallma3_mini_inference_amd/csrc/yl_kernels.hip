// yl_kernels.hip -- HIP kernels (gfx950) of the quantized LLaMA forward path.
//
// Each kernel reproduces the f32 operation order of the reference CPU path
// (paths relative to the reference repository), so that its outputs are
// bit-identical to it wherever the reference's own arithmetic is fully
// specified by its source:
//   quantize            quantization.rs:29-52, weight_type.rs:52-74
//   matmul_q8_slices    weight_type.rs:122-226
//   rmsnorm             util.rs:389-426
//   rope_gguf           util.rs:653-718
//   fused_attention     forward.rs:299-400
//   SwiGLU              forward.rs:220-237
//   logits              forward.rs:261-279
//   sample_argmax       sampler.rs:67-79
#include <hip/hip_runtime.h>

#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// RMSNorm (+ group quantization) of one row held in LDS, by one workgroup.
// util.rs:389-426: lane j of an f32x8 accumulator sums x[8i+j]^2 in i order;
// ss = 1/sqrt(reduce_add/size + eps); o = w * (ss * x) for the first
// 8*floor(size/8) elements (the rest stay 0, as the reference's zeroed
// buffer).  Then each 32-group is quantized (QF = kQ8 / kQ4) or the f32 row
// is only stored (QF < 0).
// lds must hold dim + 8 floats, x already loaded into lds[0..dim).
// ---------------------------------------------------------------------------
template <int QF>
__device__ void block_rmsnorm_quant(float* lds, const float* __restrict__ w, int dim, float eps,
                                    float* __restrict__ xn, int8_t* __restrict__ xq,
                                    float* __restrict__ xs) {
    const int tid = threadIdx.x;
    const int n8 = (dim / 8) * 8;
    if (tid < 8) {
        float l = 0.0f;
#pragma unroll 8
        for (int i = tid; i < n8; i += 8) {
            const float v = lds[i];
            l = fadd(l, fmul(v, v));
        }
        lds[dim + tid] = l;
    }
    __syncthreads();
    float part[8];
#pragma unroll
    for (int j = 0; j < 8; j++) part[j] = lds[dim + j];
    float ss = reduce_add8(part);
    ss = ss / (float)dim;
    ss = fadd(ss, eps);
    ss = 1.0f / sqrtf(ss);
    for (int i = tid; i < dim; i += blockDim.x) {
        const float o = i < n8 ? fmul(w[i], fmul(ss, lds[i])) : 0.0f;
        lds[i] = o;
        if (xn) xn[i] = o;
    }
    if constexpr (QF >= 0) {
        __syncthreads();
        const int nb = dim / kGroup;
        for (int b = tid; b < nb; b += blockDim.x) {
            const float* g = lds + b * kGroup;
            float amax = 0.0f;
#pragma unroll
            for (int k = 0; k < kGroup; k++) amax = fmaxf(amax, fabsf(g[k]));
            const float sc = group_scale<QF>(amax);
            xs[b] = sc;
            int8_t* q = xq + b * kGroup;
#pragma unroll
            for (int k = 0; k < kGroup; k++) q[k] = (int8_t)quant_one<QF>(g[k], sc);
        }
    }
}

template <int QF>
__global__ __launch_bounds__(kThreads) void k_rmsnorm(const float* __restrict__ x,
                                                      const float* __restrict__ w, int dim, float eps,
                                                      float* xn, int8_t* xq, float* xs) {
    extern __shared__ __align__(16) float lds_f[];
    const int t = blockIdx.x;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) lds_f[i] = x[(size_t)t * dim + i];
    __syncthreads();
    block_rmsnorm_quant<QF>(lds_f, w, dim, eps, xn ? xn + (size_t)t * dim : nullptr,
                            xq ? xq + (size_t)t * dim : nullptr,
                            xs ? xs + (size_t)t * (dim / kGroup) : nullptr);
}

// Embedding lookup (base_transformer.rs:143-161: out-of-range ids give
// zeros; the row is the f32 dequantization q*scale of the Q8_0 table,
// transformer_llama_gguf.rs:459-473) fused with the first RMSNorm+quantize.
template <int QF>
__global__ __launch_bounds__(kThreads) void k_embed_norm(EmbQ8 e, const uint32_t* __restrict__ tokens,
                                                         float* __restrict__ x,
                                                         const float* __restrict__ w, float eps,
                                                         float* xn, int8_t* xq, float* xs) {
    extern __shared__ __align__(16) float lds_f[];
    const int t = blockIdx.x;
    const int dim = e.dim;
    const uint32_t tok = tokens[t];
    const int lane = (int)(tok & 63u);
    const size_t tile = tok >> 6;
    const int k16n = dim / 16, nbE = dim / kGroup;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        float v = 0.0f;
        if (tok < (uint32_t)e.vocab) {
            const int8_t q = e.q[((tile * k16n + (i >> 4)) * 64 + lane) * 16 + (i & 15)];
            const float sc = f16_to_f32(e.d[(tile * nbE + (i >> 5)) * 64 + lane]);
            v = fmul((float)q, sc);
        }
        lds_f[i] = v;
        x[(size_t)t * dim + i] = v;
    }
    __syncthreads();
    block_rmsnorm_quant<QF>(lds_f, w, dim, eps, xn ? xn + (size_t)t * dim : nullptr,
                            xq + (size_t)t * dim, xs + (size_t)t * (dim / kGroup));
}

// Standalone activation quantization (quantization::quantize /
// weight_type::q4_0_quantize over a flat array): one thread per 32-group.
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
    for (int k = 0; k < kGroup; k++) q[g * kGroup + k] = (int8_t)quant_one<QF>(xg[k], sc);
}

// ---------------------------------------------------------------------------
// Quantized GEMV / batched matvec (weight_type.rs:122-226).
//
// A workgroup owns R consecutive output rows of one batch row.  Its 256
// threads split the R*nb (row, block) pairs; each pair's exact int32 block
// dot (v_dot4_i32_i8, 8 per Q8_0 block) becomes the f32 term
//     ((float)isum * w_scale) * x_scale
// in LDS.  Thread r then sums row r's terms in block order starting from the
// row's initial value -- the reference's `xout += term` sequence, so the
// result is bit-identical for any grid.
//
// Q4_0 weights keep the reference nibble order (low nibble of byte j is
// element 2j, high nibble 2j+1, unsigned 0..15); the activation row is
// staged in LDS with each 8-group reordered to (even, odd) elements so that
// (w & 0x0f0f0f0f) and ((w >> 4) & 0x0f0f0f0f) dot against it directly.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint2 q4_reorder8(uint2 v) {
    const uint32_t ev = (v.x & 0xffu) | ((v.x >> 8) & 0xff00u) | ((v.y & 0xffu) << 16) |
                        ((v.y << 8) & 0xff000000u);
    const uint32_t od = ((v.x >> 8) & 0xffu) | ((v.x >> 16) & 0xff00u) | ((v.y << 8) & 0xff0000u) |
                        (v.y & 0xff000000u);
    return make_uint2(ev, od);
}

template <int WF>
__device__ __forceinline__ int block_dot(const uint8_t* __restrict__ wrow, int b, const int32_t* xw) {
    int acc = 0;
    if constexpr (WF == kQ8) {
        const uint4* wp = reinterpret_cast<const uint4*>(wrow + (size_t)b * 32);
        const uint4 w0 = wp[0];
        const uint4 w1 = wp[1];
        acc = __builtin_amdgcn_sdot4((int)w0.x, xw[0], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w0.y, xw[1], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w0.z, xw[2], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w0.w, xw[3], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w1.x, xw[4], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w1.y, xw[5], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w1.z, xw[6], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w1.w, xw[7], acc, false);
    } else {
        const uint4 w = *reinterpret_cast<const uint4*>(wrow + (size_t)b * 16);
        const uint32_t m = 0x0f0f0f0fu;
        acc = __builtin_amdgcn_sdot4((int)(w.x & m), xw[0], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.x >> 4) & m), xw[1], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.y & m), xw[2], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.y >> 4) & m), xw[3], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.z & m), xw[4], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.z >> 4) & m), xw[5], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.w & m), xw[6], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.w >> 4) & m), xw[7], acc, false);
    }
    return acc;
}

// LDS carve-up of k_gemv (bytes): x row n | x scales nb*4 | terms R*(nb+1)*4 |
// accs 64*4 | norm row (dim+8)*4 (kEpiResid only)
static size_t gemv_smem(int n, int nb, int R, int epi, int dim) {
    size_t s = (size_t)n + (size_t)nb * 4 + (size_t)R * (nb + 1) * 4 + 64 * 4;
    if (epi == kEpiResid) s += (size_t)(dim + 8) * 4;
    return s;
}

template <int WF, int R, int EPI>
__global__ __launch_bounds__(kThreads) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int n = a.n, nb = a.nb, o = a.o;
    const int t = blockIdx.y;
    const int row0 = blockIdx.x * R;
    int8_t* xl = reinterpret_cast<int8_t*>(smem);
    float* xsl = reinterpret_cast<float*>(smem + n);
    float* terms = xsl + nb;
    float* accs = terms + R * (nb + 1);
    const int tid = threadIdx.x;

    // 1. stage the activation row (int8 + scales)
    {
        const uint2* xg = reinterpret_cast<const uint2*>(a.xq + (size_t)t * n);
        uint2* xd = reinterpret_cast<uint2*>(xl);
        for (int i = tid; i < n / 8; i += kThreads) {
            uint2 v = xg[i];
            if constexpr (WF == kQ4) v = q4_reorder8(v);
            xd[i] = v;
        }
        const float* xsg = a.xs + (size_t)t * nb;
        for (int i = tid; i < nb; i += kThreads) xsl[i] = xsg[i];
    }
    __syncthreads();

    // 2. block terms
    {
        const size_t row_bytes = WF == kQ8 ? (size_t)n : (size_t)n / 2;
        const int total = R * nb;
        const int dr = kThreads / nb, db = kThreads % nb;
        int r = tid / nb, b = tid - (tid / nb) * nb;
#pragma unroll 4
        for (int p = tid; p < total; p += kThreads) {
            const int row = row0 + r;
            float term = 0.0f;
            if (row < o) {
                const int32_t* xw = reinterpret_cast<const int32_t*>(xl + b * 32);
                const int isum = block_dot<WF>(a.qs + (size_t)row * row_bytes, b, xw);
                const float ws = f16_to_f32(a.d[(size_t)row * nb + b]);
                term = fmul(fmul((float)isum, ws), xsl[b]);
            }
            terms[r * (nb + 1) + b] = term;
            r += dr;
            b += db;
            if (b >= nb) { b -= nb; r += 1; }
        }
    }
    __syncthreads();

    // 3. ordered per-row sums
    const int pos = (EPI == kEpiQkvRope) ? a.state->pos + t : 0;
    if (tid < R) {
        const int row = row0 + tid;
        if (row < o) {
            float acc = 0.0f;
            if constexpr (EPI == kEpiStore) {
                if (row < a.accumulate_cols) acc = a.out[(size_t)t * o + row];
            } else if constexpr (EPI == kEpiQkvRope) {
                const int kv = a.kv_dim, acc_cols = (kv / 4) * 4;
                if (row >= a.att_dim && row < a.att_dim + kv) {
                    const int c = row - a.att_dim;
                    if (c < acc_cols) acc = a.k_cache[(size_t)pos * kv + c];
                } else if (row >= a.att_dim + kv) {
                    const int c = row - a.att_dim - kv;
                    if (c < acc_cols) acc = a.v_cache[(size_t)pos * kv + c];
                }
            }
            const float* tr = terms + tid * (nb + 1);
#pragma unroll 8
            for (int b = 0; b < nb; b++) acc = fadd(acc, tr[b]);
            accs[tid] = acc;
            if constexpr (EPI == kEpiStore) a.out[(size_t)t * o + row] = acc;
        }
    }
    if constexpr (EPI == kEpiStore) return;
    __syncthreads();

    // 4. epilogues
    if constexpr (EPI == kEpiQkvRope) {
        // rope_gguf (util.rs:653-718): pair (2i, 2i+1) of a head rotated by the
        // angle table row `pos`; v rows are stored as summed.
        if (tid < R) {
            const int row = row0 + tid;
            if (row < o) {
                const int att = a.att_dim, kv = a.kv_dim, hd = a.head_size;
                const float v = accs[tid];
                if (row >= att + kv) {
                    a.v_cache[(size_t)pos * kv + (row - att - kv)] = v;
                } else {
                    const int col = row < att ? row : row - att;
                    const int pair = (col % hd) >> 1;
                    const float c = a.rope_cos[(size_t)pos * (hd >> 1) + pair];
                    const float s = a.rope_sin[(size_t)pos * (hd >> 1) + pair];
                    const float v0 = accs[tid & ~1], v1 = accs[tid | 1];
                    const float r = (tid & 1) ? fadd(fmul(v0, s), fmul(v1, c))
                                              : fmul(v0, c) - fmul(v1, s);
                    if (row < att) a.q_out[(size_t)t * att + col] = r;
                    else a.k_cache[(size_t)pos * kv + col] = r;
                }
            }
        }
    } else if constexpr (EPI == kEpiResid) {
        // residual add (forward.rs:196-204 / 245-253), then the last workgroup
        // of this batch row normalizes the finished row for the next matmul.
        __shared__ int is_last;
        if (tid < R) {
            const int row = row0 + tid;
            if (row < o) {
                float* xp = a.x + (size_t)t * o + row;
                *xp = fadd(*xp, accs[tid]);
            }
        }
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            __threadfence();
            const unsigned prev = atomicAdd(a.counters + t, 1u);
            is_last = (prev == gridDim.x - 1) ? 1 : 0;
        }
        __syncthreads();
        if (!is_last) return;
        __threadfence();
        float* nrow = accs + 64;
        const int dim = a.dim;
        for (int i = tid; i < dim; i += kThreads)
            nrow[i] = __hip_atomic_load(a.x + (size_t)t * dim + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (tid == 0) a.counters[t] = 0u;
        __syncthreads();
        float* xn = a.xn ? a.xn + (size_t)t * dim : nullptr;
        int8_t* nq = a.nq ? a.nq + (size_t)t * dim : nullptr;
        float* ns = a.ns ? a.ns + (size_t)t * (dim / kGroup) : nullptr;
        if (a.norm_fmt == kQ8) block_rmsnorm_quant<kQ8>(nrow, a.norm_w, dim, a.eps, xn, nq, ns);
        else if (a.norm_fmt == kQ4) block_rmsnorm_quant<kQ4>(nrow, a.norm_w, dim, a.eps, xn, nq, ns);
        else block_rmsnorm_quant<-1>(nrow, a.norm_w, dim, a.eps, xn, nullptr, nullptr);
    } else if constexpr (EPI == kEpiSwiglu) {
        // SwiGLU (forward.rs:220-237): h = (g / (1 + exp(-g))) * u, then the
        // 32 values of this group are quantized for the down projection.
        if (tid < 32) {
            const float g = accs[tid];
            const float u = accs[32 + tid];
            const float den = fadd(1.0f, expf_rn(-g));
            const float h = fmul(g / den, u);
            const int grp = blockIdx.x;
            const size_t base = (size_t)t * a.hidden + (size_t)grp * kGroup;
            if (a.h_f32) a.h_f32[base + tid] = h;
            float am = fabsf(h);
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 32));
            am = fmaxf(am, 0.0f);
            const float sc = a.h_fmt == kQ4 ? group_scale<kQ4>(am) : group_scale<kQ8>(am);
            const int q = a.h_fmt == kQ4 ? quant_one<kQ4>(h, sc) : quant_one<kQ8>(h, sc);
            a.hq[base + tid] = (int8_t)q;
            if (tid == 0) a.hs[(size_t)t * (a.hidden / kGroup) + grp] = sc;
        }
    }
}

template <int WF, int EPI>
static hipError_t gemv_dispatch_r(const GemvArgs& a, int R, int batch, hipStream_t s) {
    const size_t smem = gemv_smem(a.n, a.nb, R, EPI, a.dim);
    const dim3 grid((a.o + R - 1) / R, batch);
    switch (R) {
    case 4:
        if constexpr (EPI != kEpiSwiglu) {
            hipLaunchKernelGGL((k_gemv<WF, 4, EPI>), grid, dim3(kThreads), smem, s, a);
            return hipGetLastError();
        }
        break;
    case 8:
        if constexpr (EPI != kEpiSwiglu) {
            hipLaunchKernelGGL((k_gemv<WF, 8, EPI>), grid, dim3(kThreads), smem, s, a);
            return hipGetLastError();
        }
        break;
    case 16:
        if constexpr (EPI != kEpiSwiglu) {
            hipLaunchKernelGGL((k_gemv<WF, 16, EPI>), grid, dim3(kThreads), smem, s, a);
            return hipGetLastError();
        }
        break;
    case 64:
        hipLaunchKernelGGL((k_gemv<WF, 64, EPI>), grid, dim3(kThreads), smem, s, a);
        return hipGetLastError();
    default:
        break;
    }
    return hipErrorInvalidValue;
}

// Rows per workgroup: enough workgroups to cover the 256 CUs several times
// for the small matrices, fewer rows (more workgroups) for long rows.
static int gemv_rows_per_wg(int o, int nb, int epi) {
    if (epi == kEpiSwiglu) return 64;
    if (nb >= 192) return 4;
    if (o >= 8192) return 16;
    return 8;
}

template <int WF>
static hipError_t gemv_dispatch(const GemvArgs& a, int epi, int batch, hipStream_t s) {
    const int R = gemv_rows_per_wg(a.o, a.nb, epi);
    switch (epi) {
    case kEpiStore: return gemv_dispatch_r<WF, kEpiStore>(a, R, batch, s);
    case kEpiQkvRope: return gemv_dispatch_r<WF, kEpiQkvRope>(a, R, batch, s);
    case kEpiResid: return gemv_dispatch_r<WF, kEpiResid>(a, R, batch, s);
    case kEpiSwiglu: return gemv_dispatch_r<WF, kEpiSwiglu>(a, R, batch, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const GemvArgs& a, int wfmt, int epi, int batch, hipStream_t s) {
    if (wfmt == kQ8) return gemv_dispatch<kQ8>(a, epi, batch, s);
    if (wfmt == kQ4) return gemv_dispatch<kQ4>(a, epi, batch, s);
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Attention over the device KV cache (forward.rs:299-400), one workgroup per
// (query head, token).  seq_len = pos + batch (the whole call's span), the
// token's own position is pos + t; later positions are masked to -1e10.
//   scores : 8-lane partial dot q.k over head_size, reduce_add, * scale
//   softmax: max from -1e10, e = exp(s - max), serial sum over seq_len,
//            p = e * (1/sum)
//   P.V    : for each d, lane j sums p[8c+j]*v[8c+j][d] over c in order,
//            reduce_add, then the seq_len%8 tail in order
// The head's output is then quantized (its 32-groups lie inside the head).
// LDS: scores seq_len | q head_size | partials 8*head_size | out head_size.
// ---------------------------------------------------------------------------
template <int QF>
__global__ __launch_bounds__(kThreads) void k_attention(const float* __restrict__ sq,
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
    const int kv_mul = n_heads / n_kv_heads;
    const int kvh = h / kv_mul;
    const int kv_dim = n_kv_heads * hd;
    const int att_dim = n_heads * hd;
    float* sc = lds_f;
    float* ql = sc + ((seq_len + 3) & ~3);
    float* part = ql + hd;
    float* outl = part + 8 * hd;

    for (int i = tid; i < hd; i += kThreads) ql[i] = sq[(size_t)t * att_dim + (size_t)h * hd + i];
    __syncthreads();

    // scores
    float lmax = -1e10f;
    const int n_simd = hd / 8;
    for (int t2 = tid; t2 <= max_t2; t2 += kThreads) {
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
    for (int t2 = max_t2 + 1 + tid; t2 < seq_len; t2 += kThreads) sc[t2] = -1e10f;
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) red[tid >> 6] = lmax;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < kThreads / 64; w++) mx = fmaxf(mx, red[w]);

    for (int t2 = tid; t2 < seq_len; t2 += kThreads) sc[t2] = expf_rn(sc[t2] - mx);
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
    for (int t2 = tid; t2 < seq_len; t2 += kThreads) sc[t2] = fmul(sc[t2], inv);
    __syncthreads();

    // P.V partial chains (d, j)
    const int n_chunks = seq_len / 8;
    const float* vbase = vc + (size_t)kvh * hd;
    for (int ch = tid; ch < 8 * hd; ch += kThreads) {
        const int d = ch % hd, j = ch / hd;
        float l = 0.0f;
        const float* vp = vbase + (size_t)j * kv_dim + d;
        for (int c = 0; c < n_chunks; c++) {
            l = fadd(l, fmul(sc[8 * c + j], vp[(size_t)(8 * c) * kv_dim]));
        }
        part[j * hd + d] = l;
    }
    __syncthreads();
    for (int d = tid; d < hd; d += kThreads) {
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
    // quantize this head's 32-groups for the output projection
    if constexpr (QF >= 0) {
        const int ng = hd / kGroup;
        for (int g = tid; g < ng; g += kThreads) {
            const float* v = outl + g * kGroup;
            float amax = 0.0f;
            for (int k = 0; k < kGroup; k++) amax = fmaxf(amax, fabsf(v[k]));
            const float s = group_scale<QF>(amax);
            const size_t gi = (size_t)t * (att_dim / kGroup) + ((size_t)h * hd) / kGroup + g;
            as[gi] = s;
            for (int k = 0; k < kGroup; k++) aq[gi * kGroup + k] = (int8_t)quant_one<QF>(v[k], s);
        }
    }
}

hipError_t launch_attention(const float* sq, const float* kc, const float* vc, const StepState* st,
                            int batch, int max_seq, int n_heads, int n_kv_heads, int head_size,
                            float scale, int qfmt, int8_t* aq, float* as, float* att_f32,
                            hipStream_t s) {
    const size_t smem = ((size_t)((max_seq + 3) & ~3) + 10 * (size_t)head_size) * sizeof(float);
    const dim3 grid(n_heads, batch);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_attention<kQ8>), grid, dim3(kThreads), smem, s, sq, kc, vc, st, batch,
                           n_heads, n_kv_heads, head_size, scale, aq, as, att_f32);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_attention<kQ4>), grid, dim3(kThreads), smem, s, sq, kc, vc, st, batch,
                           n_heads, n_kv_heads, head_size, scale, aq, as, att_f32);
    else
        hipLaunchKernelGGL((k_attention<-1>), grid, dim3(kThreads), smem, s, sq, kc, vc, st, batch,
                           n_heads, n_kv_heads, head_size, scale, aq, as, att_f32);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Standalone RoPE (util.rs:653-718) on q [batch][n_heads*hd] and k
// [batch][n_kv_heads*hd] at positions pos+t, one thread per (head, pair).
// ---------------------------------------------------------------------------
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

hipError_t launch_rope(const float* cos_t, const float* sin_t, const StepState* st, int batch,
                       float* q, float* k, int n_heads, int n_kv_heads, int head_size, hipStream_t s) {
    const int items = (n_heads + n_kv_heads) * (head_size / 2);
    const dim3 grid((items + kThreads - 1) / kThreads, batch);
    hipLaunchKernelGGL(k_rope, grid, dim3(kThreads), 0, s, cos_t, sin_t, st, q, k, n_heads,
                       n_kv_heads, head_size);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Standalone SwiGLU (forward.rs:220-237) + group quantization: one 32-lane
// half-wave per 32-group of hidden.
// ---------------------------------------------------------------------------
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

hipError_t launch_swiglu_quant(int qfmt, const float* gate, const float* up, int hidden, int batch,
                               float* h_f32, int8_t* hq, float* hs, hipStream_t s) {
    const dim3 grid((hidden + kThreads - 1) / kThreads, batch);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_swiglu_quant<kQ8>), grid, dim3(kThreads), 0, s, gate, up, hidden, h_f32, hq, hs);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_swiglu_quant<kQ4>), grid, dim3(kThreads), 0, s, gate, up, hidden, h_f32, hq, hs);
    else
        hipLaunchKernelGGL((k_swiglu_quant<-1>), grid, dim3(kThreads), 0, s, gate, up, hidden, h_f32, hq, hs);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Tied-embedding logits (forward.rs:261-279) + greedy argmax
// (sampler.rs:67-79).  One wavefront per 64 vocabulary rows; lane = row.
// Each lane keeps the 8 f32x8 lane partials of its row and walks the row in
// 16-element chunks (two f32x8 steps each), so every partial sees its terms
// in the reference's order.  The embedding value is the exact f32 product
// q * scale of the Q8_0 table (transformer_llama_gguf.rs:465-470).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_logits(EmbQ8 e, const float* __restrict__ xn,
                                                     float* __restrict__ logits,
                                                     unsigned long long* __restrict__ key) {
    extern __shared__ __align__(16) float xl[];
    const int dim = e.dim;
    for (int i = threadIdx.x; i < dim; i += kThreads) xl[i] = xn[i];
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tile = blockIdx.x * (kThreads / 64) + wave;
    if (tile >= e.tiles) return;
    const int k16n = dim / 16, nbE = dim / kGroup;
    const int4* qp = reinterpret_cast<const int4*>(e.q) + (size_t)tile * k16n * 64 + lane;
    const uint16_t* dp = e.d + (size_t)tile * nbE * 64 + lane;
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float scv = 0.0f;
#pragma unroll 4
    for (int k = 0; k < k16n; k++) {
        const int4 qv = qp[(size_t)k * 64];
        if ((k & 1) == 0) scv = f16_to_f32(dp[(size_t)(k >> 1) * 64]);
        const float* xk = xl + k * 16;
        const int w[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int m = 0; m < 4; m++) {
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                const int ei = m * 4 + bb;
                const float qf = (float)(int8_t)(w[m] >> (8 * bb));
                l[ei & 7] = fadd(l[ei & 7], fmul(xk[ei], fmul(qf, scv)));
            }
        }
    }
    const float logit = reduce_add8(l);
    const int row = tile * 64 + lane;
    unsigned long long kk = 0ull;
    if (row < e.vocab) {
        if (logits) logits[row] = logit;
        kk = argmax_key(logit, (uint32_t)row);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o2 = __shfl_xor(kk, off, 64);
        kk = o2 > kk ? o2 : kk;
    }
    if (lane == 0 && key) atomicMax(key, kk);
}

hipError_t launch_logits(const EmbQ8& e, const float* xn, float* logits, unsigned long long* key,
                         hipStream_t s) {
    const int per = kThreads / 64;
    const dim3 grid((e.tiles + per - 1) / per);
    hipLaunchKernelGGL(k_logits, grid, dim3(kThreads), (size_t)e.dim * sizeof(float), s, e, xn, logits, key);
    return hipGetLastError();
}

// End of a step: decode the argmax key into the next token, append it to the
// output ring, advance the position, and clear the key for the next step.
__global__ void k_finalize(StepState* st, uint32_t* out_tokens, uint32_t out_cap, int advance) {
    const unsigned long long k = st->argmax;
    const uint32_t tok = 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull);
    st->token = tok;
    if (out_tokens && st->n_out < out_cap) out_tokens[st->n_out] = tok;
    st->n_out += 1;
    st->pos += advance;
    st->argmax = 0ull;
}

hipError_t launch_finalize(StepState* st, uint32_t* out_tokens, uint32_t out_cap, int advance,
                           hipStream_t s) {
    hipLaunchKernelGGL(k_finalize, dim3(1), dim3(1), 0, s, st, out_tokens, out_cap, advance);
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

hipError_t launch_rmsnorm(int qfmt, const float* x, const float* w, int dim, float eps, int batch,
                          float* xn, int8_t* xq, float* xs, hipStream_t s) {
    const size_t smem = (size_t)(dim + 8) * sizeof(float);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_rmsnorm<kQ8>), dim3(batch), dim3(kThreads), smem, s, x, w, dim, eps, xn, xq, xs);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_rmsnorm<kQ4>), dim3(batch), dim3(kThreads), smem, s, x, w, dim, eps, xn, xq, xs);
    else
        hipLaunchKernelGGL((k_rmsnorm<-1>), dim3(batch), dim3(kThreads), smem, s, x, w, dim, eps, xn, xq, xs);
    return hipGetLastError();
}

hipError_t launch_embed_norm(const EmbQ8& e, const uint32_t* tokens, int batch, float* x,
                             const float* w, float eps, int qfmt, float* xn, int8_t* xq, float* xs,
                             hipStream_t s) {
    const size_t smem = (size_t)(e.dim + 8) * sizeof(float);
    if (qfmt == kQ8)
        hipLaunchKernelGGL((k_embed_norm<kQ8>), dim3(batch), dim3(kThreads), smem, s, e, tokens, x, w, eps, xn, xq, xs);
    else if (qfmt == kQ4)
        hipLaunchKernelGGL((k_embed_norm<kQ4>), dim3(batch), dim3(kThreads), smem, s, e, tokens, x, w, eps, xn, xq, xs);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
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

hipError_t launch_math_selftest(const float* x, int n, float* exp_out, float* sqrt_out,
                                float* div_out, float* f16_out, hipStream_t s) {
    hipLaunchKernelGGL(k_math_selftest, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, x, n,
                       exp_out, sqrt_out, div_out, f16_out);
    return hipGetLastError();
}

}  // namespace yl
