// yl_gemv.hip -- quantized GEMV / batched matvec (weight_type.rs:122-226)
// with the neighbouring elementwise work of forward.rs fused in.
//
// A workgroup owns R consecutive output rows of one batch row (blockIdx.y).
// Its threads split the R*nb (row, block) pairs.  Every thread first issues
// the loads of all its pairs' weights (two 16-byte loads per Q8_0 block, one
// per Q4_0 block, plus the f16 scale) into registers; only then does the
// workgroup prepare the activation row in LDS -- either staging an already
// quantized row, or (QKV and gate/up matmuls) computing RMSNorm + quantize of
// the f32 residual stream itself -- so that work overlaps the HBM latency.
//
// Each pair's exact int32 block dot (v_dot4_i32_i8) becomes the f32 term
//     ((float)isum * w_scale) * x_scale
// in LDS, and thread r sums row r's terms in block order from the row's
// initial value: the reference's `xout += term` sequence, so every output is
// bit-identical to matmul_q8_slices for any grid shape.
//
// Q4_0 weights keep the reference nibble order (low nibble of byte j is
// element 2j, high nibble 2j+1, unsigned 0..15); the activation row is
// staged with each 8-group reordered to (even, odd) elements so that
// (w & 0x0f0f0f0f) and ((w >> 4) & 0x0f0f0f0f) dot against it directly.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

__device__ __forceinline__ uint2 q4_reorder8(uint2 v) {
    const uint32_t ev = (v.x & 0xffu) | ((v.x >> 8) & 0xff00u) | ((v.y & 0xffu) << 16) |
                        ((v.y << 8) & 0xff000000u);
    const uint32_t od = ((v.x >> 8) & 0xffu) | ((v.x >> 16) & 0xff00u) | ((v.y << 8) & 0xff0000u) |
                        (v.y & 0xff000000u);
    return make_uint2(ev, od);
}

template <int WF>
struct WBlock;
template <>
struct WBlock<kQ8> { uint4 a, b; };
template <>
struct WBlock<kQ4> { uint4 a; };

template <int WF>
__device__ __forceinline__ void load_block(WBlock<WF>& w, const uint8_t* __restrict__ p) {
    if constexpr (WF == kQ8) {
        const uint4* q = reinterpret_cast<const uint4*>(p);
        w.a = q[0];
        w.b = q[1];
    } else {
        w.a = *reinterpret_cast<const uint4*>(p);
    }
}

template <int WF>
__device__ __forceinline__ int block_dot(const WBlock<WF>& w, const int32_t* xw) {
    int acc = 0;
    if constexpr (WF == kQ8) {
        acc = __builtin_amdgcn_sdot4((int)w.a.x, xw[0], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.a.y, xw[1], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.a.z, xw[2], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.a.w, xw[3], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.x, xw[4], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.y, xw[5], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.z, xw[6], acc, false);
        acc = __builtin_amdgcn_sdot4((int)w.b.w, xw[7], acc, false);
    } else {
        const uint32_t m = 0x0f0f0f0fu;
        acc = __builtin_amdgcn_sdot4((int)(w.a.x & m), xw[0], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.x >> 4) & m), xw[1], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.a.y & m), xw[2], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.y >> 4) & m), xw[3], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.a.z & m), xw[4], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.z >> 4) & m), xw[5], acc, false);
        acc = __builtin_amdgcn_sdot4((int)(w.a.w & m), xw[6], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((w.a.w >> 4) & m), xw[7], acc, false);
    }
    return acc;
}

// terms row stride (floats): float4-aligned rows for the ordered sums
__host__ __device__ inline int terms_stride(int nb) { return ((nb + 3) & ~3) + 4; }

static size_t gemv_smem(int n, int nb, int R, int epi, int dim) {
    size_t s = (size_t)n + (size_t)nb * 4;
    s = (s + 15) & ~(size_t)15;
    s += (size_t)R * terms_stride(nb) * 4 + 64 * 4;
    if (epi == kEpiQkvRope || epi == kEpiSwiglu) s += norm_lds_floats(dim) * 4;
    return s;
}

template <int WF, int R, int TPB, int PMAX, int EPI, bool EMB>
__global__ __launch_bounds__(TPB) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int n = a.n, nb = a.nb, o = a.o;
    const int tid = threadIdx.x;
    const int t = blockIdx.y;
    const int row0 = blockIdx.x * R;
    const int TS = terms_stride(nb);
    int8_t* xl = reinterpret_cast<int8_t*>(smem);
    float* xsl = reinterpret_cast<float*>(smem + n);
    float* terms = reinterpret_cast<float*>(smem + (((size_t)n + (size_t)nb * 4 + 15) & ~(size_t)15));
    float* accs = terms + R * TS;
    float* xt = accs + 64;
    constexpr bool kNorm = EPI == kEpiQkvRope || EPI == kEpiSwiglu;

    // Global loads are issued in the order they are needed: first the
    // activation inputs (recently written, cache-hot), then every weight block
    // of this thread.  Vector-memory loads retire in order, so waiting for the
    // activations then leaves the weights in flight while the prologue runs.
    // All loads are unconditional (out-of-range indices are clamped and their
    // data ignored): a load under a divergent branch makes the compiler wait
    // for it at the branch join, which would serialize the HBM round trips.
    const int dim = n;
    constexpr int kMaxPer = 8192 / TPB;          // normalized rows: dim <= 8192
    constexpr int kMaxStage = 16384 / 8 / TPB;   // staged int8 rows: n <= 16384
    constexpr int kMaxScale = (512 + TPB - 1) / TPB;
    float xv[kNorm ? kMaxPer : 1], wn[kNorm ? kMaxPer : 1];
    uint2 qv[kNorm ? 1 : kMaxStage];
    float sv[kNorm ? 1 : kMaxScale];

    // 1a. activation inputs -> registers (the decode position first: the
    // epilogue's cache addresses depend on it)
    const int pos = (EPI == kEpiQkvRope) ? a.state->pos + t : 0;
    int eqv[EMB ? kMaxPer : 1];
    uint16_t edv[EMB ? kMaxPer : 1];
    bool in_vocab = true;
    if constexpr (kNorm) {
        const float* __restrict__ nw = a.norm_w;
        if constexpr (EMB) {
            // layer 0: the residual stream starts as the token's embedding row
            // (base_transformer.rs:143-161, zero for ids >= vocab)
            const uint32_t tok = a.tokens[t];
            in_vocab = tok < (uint32_t)a.emb.vocab;
            const size_t tile = in_vocab ? tok >> 6 : 0;
            const int lane = (int)(tok & 63u);
            const int8_t* __restrict__ eq = a.emb.q;
            const uint16_t* __restrict__ ed = a.emb.d;
#pragma unroll
            for (int k = 0; k < kMaxPer; k++) {
                const int i = tid + k * TPB;
                if (k * TPB < dim) {
                    const int ic = i < dim ? i : 0;
                    eqv[k] = eq[((tile * (dim / 16) + (ic >> 4)) * 64 + lane) * 16 + (ic & 15)];
                    edv[k] = ed[(tile * (dim / 32) + (ic >> 5)) * 64 + lane];
                    wn[k] = nw[ic];
                }
            }
        } else {
            const float* __restrict__ xin = a.x + (size_t)t * dim;
#pragma unroll
            for (int k = 0; k < kMaxPer; k++) {
                const int i = tid + k * TPB;
                if (k * TPB < dim) {
                    const int ic = i < dim ? i : 0;
                    xv[k] = xin[ic];
                    wn[k] = nw[ic];
                }
            }
        }
    } else {
        const uint2* __restrict__ xg = reinterpret_cast<const uint2*>(a.xq + (size_t)t * n);
        const float* __restrict__ xsg = a.xs + (size_t)t * nb;
#pragma unroll
        for (int k = 0; k < kMaxStage; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < n / 8) qv[k] = xg[i < n / 8 ? i : 0];
        }
#pragma unroll
        for (int k = 0; k < kMaxScale; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < nb) sv[k] = xsg[i < nb ? i : 0];
        }
    }

    // 1a'. values the epilogue reads (cache initial values and RoPE angles,
    // the residual row, the accumulate-into output), fetched now
    float ep0 = 0.0f, ep1 = 1.0f, ep2 = 0.0f;
    bool ep_acc = false;
    {
        const int er = min(row0 + (tid < R ? tid : 0), o - 1);
        if constexpr (EPI == kEpiQkvRope) {
            // K/V rows accumulate into the cache (forward.rs:166-169)
            const int att = a.att_dim, kv = a.kv_dim, hd = a.head_size;
            const bool is_k = er >= att && er < att + kv, is_v = er >= att + kv;
            const int c = is_v ? er - att - kv : (is_k ? er - att : 0);
            ep_acc = (is_k || is_v) && c < (kv / 4) * 4;
            ep0 = (is_v ? a.v_cache : a.k_cache)[(size_t)pos * kv + c];
            const int col = er < att ? er : c;
            const int pair = (col % hd) >> 1;
            ep1 = a.rope_cos[(size_t)pos * (hd >> 1) + pair];
            ep2 = a.rope_sin[(size_t)pos * (hd >> 1) + pair];
        } else if constexpr (EPI == kEpiResid) {
            ep0 = a.x[(size_t)t * o + er];
        } else if constexpr (EPI == kEpiStore) {
            ep_acc = er < a.accumulate_cols;
            ep0 = a.out[(size_t)t * o + er];
        }
    }

    // 1b. weights of every pair of this thread -> registers
    const size_t row_bytes = WF == kQ8 ? (size_t)n : (size_t)n / 2;
    const int total = R * nb;
    WBlock<WF> wv[PMAX];
    uint16_t dv[PMAX];
    {
        const int dr = TPB / nb, db = TPB % nb;
        int r = tid / nb, b = tid - (tid / nb) * nb;
#pragma unroll
        for (int k = 0; k < PMAX; k++) {
            const bool ok = tid + k * TPB < total && row0 + r < o;
            const size_t row = ok ? (size_t)(row0 + r) : 0;
            load_block<WF>(wv[k], a.qs + row * row_bytes + (size_t)b * (WF == kQ8 ? 32 : 16));
            dv[k] = a.d[row * nb + b];
            r += dr;
            b += db;
            if (b >= nb) { b -= nb; r += 1; }
        }
    }

    // 2. activation row -> LDS (int8 values + f32 group scales)
    if constexpr (kNorm) {
#pragma unroll
        for (int k = 0; k < kMaxPer; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < dim && i < dim) {
                float v;
                if constexpr (EMB)
                    v = in_vocab ? fmul((float)((int)(uint8_t)eqv[k] - 128), f16_to_f32(edv[k])) : 0.0f;
                else v = xv[k];
                store_norm_input(xt, dim, i, v, wn[k]);
                if (EMB && blockIdx.x == 0) a.x[(size_t)t * dim + i] = v;
            }
        }
        __syncthreads();
        rmsnorm_quant_block<WF, WF == kQ4>(xt, dim, a.eps, xl, xsl, nullptr);
    } else {
        uint2* xd = reinterpret_cast<uint2*>(xl);
#pragma unroll
        for (int k = 0; k < kMaxStage; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < n / 8 && i < n / 8) {
                uint2 v = qv[k];
                if constexpr (WF == kQ4) v = q4_reorder8(v);
                xd[i] = v;
            }
        }
#pragma unroll
        for (int k = 0; k < kMaxScale; k++) {
            const int i = tid + k * TPB;
            if (k * TPB < nb && i < nb) xsl[i] = sv[k];
        }
        __syncthreads();
    }

    // 3. exact block dots -> f32 terms in LDS
    {
        const int dr = TPB / nb, db = TPB % nb;
        int r = tid / nb, b = tid - (tid / nb) * nb;
#pragma unroll
        for (int k = 0; k < PMAX; k++) {
            if (tid + k * TPB < total) {
                float term = 0.0f;
                if (row0 + r < o) {
                    const int isum = block_dot<WF>(wv[k], reinterpret_cast<const int32_t*>(xl + b * 32));
                    term = fmul(fmul((float)isum, f16_to_f32(dv[k])), xsl[b]);
                }
                terms[r * TS + b] = term;
            }
            r += dr;
            b += db;
            if (b >= nb) { b -= nb; r += 1; }
        }
    }
    __syncthreads();

    // 4. ordered per-row sums
    if (tid < R) {
        const int row = row0 + tid;
        if (row < o) {
            float acc = ep_acc ? ep0 : 0.0f;
            const float* tr = terms + tid * TS;
            const float4* t4 = reinterpret_cast<const float4*>(tr);
            int b = 0;
#pragma unroll 4
            for (; b < nb / 4; b++) {
                const float4 v = t4[b];
                acc = fadd(acc, v.x);
                acc = fadd(acc, v.y);
                acc = fadd(acc, v.z);
                acc = fadd(acc, v.w);
            }
            for (int bb = b * 4; bb < nb; bb++) acc = fadd(acc, tr[bb]);
            accs[tid] = acc;
            if constexpr (EPI == kEpiStore) a.out[(size_t)t * o + row] = acc;
            if constexpr (EPI == kEpiResid) {
                // residual add (forward.rs:196-204 / 245-253)
                a.x[(size_t)t * o + row] = fadd(ep0, acc);
            }
        }
    }
    if constexpr (EPI == kEpiStore || EPI == kEpiResid) return;
    __syncthreads();

    // 5. epilogues over neighbouring rows
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
                    const float c = ep1, s = ep2;
                    const float v0 = accs[tid & ~1], v1 = accs[tid | 1];
                    const float r = (tid & 1) ? fadd(fmul(v0, s), fmul(v1, c)) : fmul(v0, c) - fmul(v1, s);
                    if (row < att) a.q_out[(size_t)t * att + col] = r;
                    else a.k_cache[(size_t)pos * kv + col] = r;
                }
            }
        }
    } else if constexpr (EPI == kEpiSwiglu) {
        // SwiGLU (forward.rs:220-237): h = (g / (1 + exp(-g))) * u, then this
        // 32-group of h is quantized for the down projection.
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

// ------------------------------------------------------------ dispatch ----

struct GemvShape {
    int R, TPB, PMAX;
};

// Rows per workgroup and threads: enough workgroups to cover the 256 CUs,
// 32-128 KiB of weights in flight per CU, and every pair of a thread loaded
// before its first use.
static GemvShape pick_shape(int o, int nb, int epi) {
    GemvShape s;
    if (epi == kEpiSwiglu) {
        s.R = 64;
        s.TPB = 512;
    } else if (nb >= 192) {
        s.R = 4;
        s.TPB = 256;
    } else if (o >= 8192) {
        s.R = 16;
        s.TPB = 256;
    } else {
        s.R = 8;
        s.TPB = 256;
    }
    const int p = (s.R * nb + s.TPB - 1) / s.TPB;
    s.PMAX = p <= 1 ? 1 : p <= 2 ? 2 : p <= 4 ? 4 : p <= 8 ? 8 : p <= 16 ? 16 : 0;
    return s;
}

template <int WF, int R, int TPB, int EPI, bool EMB>
static hipError_t launch_r2(const GemvArgs& a, int pmax, int batch, hipStream_t st) {
    const size_t smem = gemv_smem(a.n, a.nb, R, EPI, a.n);
    const dim3 grid((a.o + R - 1) / R, batch);
    switch (pmax) {
    case 1: hipLaunchKernelGGL((k_gemv<WF, R, TPB, 1, EPI, EMB>), grid, dim3(TPB), smem, st, a); break;
    case 2: hipLaunchKernelGGL((k_gemv<WF, R, TPB, 2, EPI, EMB>), grid, dim3(TPB), smem, st, a); break;
    case 4: hipLaunchKernelGGL((k_gemv<WF, R, TPB, 4, EPI, EMB>), grid, dim3(TPB), smem, st, a); break;
    case 8: hipLaunchKernelGGL((k_gemv<WF, R, TPB, 8, EPI, EMB>), grid, dim3(TPB), smem, st, a); break;
    case 16: hipLaunchKernelGGL((k_gemv<WF, R, TPB, 16, EPI, EMB>), grid, dim3(TPB), smem, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int WF, int R, int TPB, int EPI>
static hipError_t launch_r(const GemvArgs& a, int pmax, int batch, hipStream_t st) {
    if constexpr (EPI == kEpiQkvRope) {
        if (a.emb.q) return launch_r2<WF, R, TPB, EPI, true>(a, pmax, batch, st);
    }
    return launch_r2<WF, R, TPB, EPI, false>(a, pmax, batch, st);
}

template <int WF, int EPI>
static hipError_t launch_epi(const GemvArgs& a, int batch, hipStream_t st) {
    const GemvShape s = pick_shape(a.o, a.nb, EPI);
    if (s.PMAX == 0) return hipErrorInvalidValue;
    if constexpr (EPI == kEpiSwiglu) {
        return launch_r<WF, 64, 512, EPI>(a, s.PMAX, batch, st);
    } else {
        if (s.R == 4) return launch_r<WF, 4, 256, EPI>(a, s.PMAX, batch, st);
        if (s.R == 16) return launch_r<WF, 16, 256, EPI>(a, s.PMAX, batch, st);
        return launch_r<WF, 8, 256, EPI>(a, s.PMAX, batch, st);
    }
}

template <int WF>
static hipError_t launch_wf(const GemvArgs& a, int epi, int batch, hipStream_t st) {
    switch (epi) {
    case kEpiStore: return launch_epi<WF, kEpiStore>(a, batch, st);
    case kEpiQkvRope: return launch_epi<WF, kEpiQkvRope>(a, batch, st);
    case kEpiResid: return launch_epi<WF, kEpiResid>(a, batch, st);
    case kEpiSwiglu: return launch_epi<WF, kEpiSwiglu>(a, batch, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const GemvArgs& a, int wfmt, int epi, int batch, hipStream_t s) {
    if ((epi == kEpiQkvRope || epi == kEpiSwiglu) && (a.n % 32 || a.n > 8192)) return hipErrorInvalidValue;
    if (a.n % 32 || a.n > 16384) return hipErrorInvalidValue;
    if (wfmt == kQ8) return launch_wf<kQ8>(a, epi, batch, s);
    if (wfmt == kQ4) return launch_wf<kQ4>(a, epi, batch, s);
    return hipErrorInvalidValue;
}

size_t gemv_bytes_per_row_block(int wfmt) { return wfmt == kQ8 ? 34 : 18; }

}  // namespace yl
