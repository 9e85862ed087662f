// yl_attn_split.hip -- decode attention split over the context, the
// tolerance mode of forward.rs:299-400 (fused_attention at batch 1).
//
// The reference computes, per query head, scores s_p = (q . k_p) * scale over
// every position, m = max s_p, e_p = exp(s_p - m), sum = serial sum of e_p
// and out = sum_p (e_p / sum) v_p.  The exact path (yl_attn.hip) keeps that
// order bit for bit, which makes the denominator one serial chain over the
// whole context.  This kernel computes the same quantity as a split softmax:
// the positions of one kv head are dealt to `ns` workgroups; each keeps, per
// query head of the group, a running maximum m_i, sum l_i and unnormalised
// output o_i over its positions (tiles of kSplitTile, rescaled by
// exp(m_old - m_new) when the maximum grows), and the last workgroup of the
// kv head to finish combines them:
//   M = max_i m_i,  L = sum_i l_i exp(m_i - M),  out = sum_i o_i exp(m_i - M) / L.
// The result differs from the reference's in rounding only (f32 sums in
// another order, a hardware exp2); it is for configurations whose bar is
// logits within 1e-3 rather than identical bits.
//
// Workgroup (kv head g, split i), 256 threads:
//   scores: half-wavefront hw of wavefront w takes key dimensions
//     [(2w + hw) * HD/8, ...) of every position, lane l % 32 four positions
//     (one 16-byte load per dimension from the transposed key cache); the 8
//     partial dot products meet in LDS.
//   values: the tile's V rows (HD floats each) come into LDS by LDS DMA,
//     issued after the key loads so that the scores do not wait for them.
//   P.V: thread t owns outputs (head, dim) t, t + 256, ... of the group.
// The partials go out with agent-scope stores, then an agent-scope atomic
// count per kv head picks the last workgroup, which reads them back with
// agent-scope loads (coherent across the XCDs' L2s), writes the output
// (f32 and/or its 32-group quantization for the Wo matmul) and clears the
// count for the next launch.
#include <hip/hip_runtime.h>

#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kSplitThreads = 256;
constexpr int kSplitTile = 128;    // positions per tile
constexpr int kSplitMaxParts = 64; // workgroups per kv head

__host__ __device__ constexpr int split_lds_floats(int hd, int r) {
    return kSplitTile * hd          // V tile
           + 8 * r * kSplitTile     // score partials of the 8 dimension groups
           + r * hd                 // queries
           + r * kSplitTile         // scores, then exponentials
           + 4 * r + 4;             // per head: running max, sum, rescale; last-workgroup flag
}

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// sum over the 64 lanes (any order: this path has a tolerance, not an order)
__device__ __forceinline__ float wave_sum_any(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int QF, int HD, int R>
__global__ __launch_bounds__(kSplitThreads) void k_attn_split(const float* __restrict__ sq,
                                                              const float* __restrict__ kc,
                                                              const float* __restrict__ vc,
                                                              const StepState* __restrict__ st, int n_kv_heads,
                                                              int kv_ld, float scale, int ns, float* part,
                                                              unsigned* counters, int8_t* __restrict__ aq,
                                                              float* __restrict__ as, float* __restrict__ att_f32) {
    extern __shared__ __align__(16) float lds[];
    constexpr int T = kSplitTile;
    constexpr int DG = HD / 8;                    // key dimensions per group
    constexpr int NOUT = (R * HD + kSplitThreads - 1) / kSplitThreads;
    constexpr int PS = HD + 2;                    // floats per (split, head) partial: o, m, l
    float* vt = lds;
    float* red = vt + T * HD;
    float* ql = red + 8 * R * T;
    float* el = ql + R * HD;
    float* hs = el + R * T;                       // [R][4]: m, l, alpha
    int* flag = reinterpret_cast<int*>(hs + 4 * R);

    const int kvh = blockIdx.x, sp = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int seq = st->pos + 1;
    const int kv_dim = n_kv_heads * HD;
    const int chunk = ((seq + ns - 1) / ns + 3) & ~3;
    const int p0 = sp * chunk;
    const int p1 = min(seq, p0 + chunk);

    for (int i = tid; i < R * HD; i += kSplitThreads) ql[i] = sq[(size_t)kvh * R * HD + i];
    if (tid < R) {
        hs[tid * 4 + 0] = -INFINITY;
        hs[tid * 4 + 1] = 0.0f;
        hs[tid * 4 + 2] = 1.0f;
    }
    float o[NOUT];
#pragma unroll
    for (int k = 0; k < NOUT; k++) o[k] = 0.0f;
    lds_barrier();

    const float* __restrict__ kb = kc + (size_t)kvh * HD * kv_ld;
    const int dg = wave * 2 + (lane >> 5);
    const int pl = (lane & 31) * 4;
    for (int t0 = p0; t0 < p1; t0 += T) {
        const int nt = min(T, p1 - t0);
        // key loads of this tile: quads past the split re-read its last quad
        // (rows are kv_ld >= seq long, a multiple of 4)
        const int q0 = min(t0 + pl, (p1 - 1) & ~3);
        vf4 kr[DG];
#pragma unroll
        for (int i = 0; i < DG; i++) kr[i] = *reinterpret_cast<const vf4*>(kb + (size_t)(dg * DG + i) * kv_ld + q0);
        // V rows of the tile into LDS (rows past the split re-read its last row)
        {
            constexpr int RPI = 1024 / (HD * 4);   // rows per 64-lane 16-byte DMA instruction
            constexpr int NI = T / RPI;
            const int lr = lane / (HD / 4), col = (lane % (HD / 4)) * 4;
            for (int i = wave; i < NI; i += kSplitThreads / 64) {
                const int row = min(t0 + i * RPI + lr, p1 - 1);
                __builtin_amdgcn_global_load_lds(vc + (size_t)row * kv_dim + kvh * HD + col, vt + i * RPI * HD, 16, 0,
                                                 0);
            }
        }
        float acc[R][4];
#pragma unroll
        for (int h = 0; h < R; h++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[h][c] = 0.0f;
#pragma unroll
        for (int i = 0; i < DG; i++) {
            const int d = dg * DG + i;
#pragma unroll
            for (int h = 0; h < R; h++) {
                const float qv = ql[h * HD + d];
#pragma unroll
                for (int c = 0; c < 4; c++) acc[h][c] = fmaf(qv, kr[i][c], acc[h][c]);
            }
        }
#pragma unroll
        for (int h = 0; h < R; h++)
            *reinterpret_cast<vf4*>(red + (dg * R + h) * T + pl) = vf4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
        lds_barrier();
        for (int i = tid; i < R * T; i += kSplitThreads) {
            const int h = i / T, p = i % T;
            float s = 0.0f;
#pragma unroll
            for (int g = 0; g < 8; g++) s += red[(g * R + h) * T + p];
            el[i] = p < nt ? s * scale : -INFINITY;
        }
        lds_barrier();
        // per head: the tile's maximum, the new running maximum, the rescale
        // of what came before, the exponentials and their sum
        for (int h = wave; h < R; h += kSplitThreads / 64) {
            float mx = -INFINITY;
            for (int p = lane; p < T; p += 64) mx = fmaxf(mx, el[h * T + p]);
            mx = wave_max(mx);
            const float m_old = hs[h * 4 + 0];
            const float m_new = fmaxf(m_old, mx);
            const float alpha = exp_fast(m_old - m_new);
            float sum = 0.0f;
            for (int p = lane; p < T; p += 64) {
                const float e = exp_fast(el[h * T + p] - m_new);
                el[h * T + p] = e;
                sum += e;
            }
            sum = wave_sum_any(sum);
            if (lane == 0) {
                hs[h * 4 + 0] = m_new;
                hs[h * 4 + 1] = hs[h * 4 + 1] * alpha + sum;
                hs[h * 4 + 2] = alpha;
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wavefront's V rows landed
        lds_barrier();
#pragma unroll
        for (int k = 0; k < NOUT; k++) {
            const int idx = tid + k * kSplitThreads;
            if (idx < R * HD) {
                const int h = idx / HD, d = idx % HD;
                float a = o[k] * hs[h * 4 + 2];
                const float* __restrict__ e = el + h * T;
                for (int p = 0; p < nt; p++) a = fmaf(e[p], vt[p * HD + d], a);
                o[k] = a;
            }
        }
        lds_barrier();   // vt, el and red are rewritten by the next tile
    }

    // this split's partials: o (unnormalised), m, l per head
    float* __restrict__ mine = part + ((size_t)kvh * ns + sp) * R * PS;
#pragma unroll
    for (int k = 0; k < NOUT; k++) {
        const int idx = tid + k * kSplitThreads;
        if (idx < R * HD)
            __hip_atomic_store(mine + (idx / HD) * PS + idx % HD, o[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < R) {
        __hip_atomic_store(mine + tid * PS + HD, hs[tid * 4 + 0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mine + tid * PS + HD + 1, hs[tid * 4 + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the stores are performed before the count
    lds_barrier();
    if (tid == 0) {
        const unsigned done = __hip_atomic_fetch_add(counters + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = done == (unsigned)ns - 1;
    }
    lds_barrier();
    if (!*flag) return;

    // the last workgroup of this kv head: combine the splits.  The (m, l)
    // pairs of every (split, head) come into LDS in one round of loads, the
    // weights exp(m_i - M) are formed there (a split with no positions has
    // m = -inf, weight 0), and each output's ns partial values are loaded 16
    // at a time, all in flight together.
    const float* __restrict__ all = part + (size_t)kvh * ns * R * PS;
    float* wl = red;            // [ns][R]: maxima, then weights
    float* ll = red + ns * R;   // [ns][R]: sums
    for (int i = tid; i < ns * R; i += kSplitThreads) {
        const float m = __hip_atomic_load(all + (size_t)i * PS + HD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float l = __hip_atomic_load(all + (size_t)i * PS + HD + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wl[i] = m;
        ll[i] = l;
    }
    lds_barrier();
    if (tid < R) {
        float M = -INFINITY;
        for (int i = 0; i < ns; i++) M = fmaxf(M, wl[i * R + tid]);
        float L = 0.0f;
        for (int i = 0; i < ns; i++) {
            const float w = exp_fast(wl[i * R + tid] - M);
            wl[i * R + tid] = w;
            L = fmaf(ll[i * R + tid], w, L);
        }
        hs[tid * 4 + 1] = L;
    }
    lds_barrier();
#pragma unroll
    for (int k = 0; k < NOUT; k++) {
        const int idx = tid + k * kSplitThreads;
        const bool live = idx < R * HD;
        const int h = live ? idx / HD : 0, d = idx % HD;
        float O = 0.0f;
        for (int i0 = 0; i0 < ns; i0 += 16) {
            // (splits past ns re-read the last one with weight 0)
            float ov[16];
#pragma unroll
            for (int j = 0; j < 16; j++)
                ov[j] = __hip_atomic_load(all + ((size_t)min(i0 + j, ns - 1) * R + h) * PS + d, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int j = 0; j < 16; j++) O = fmaf(ov[j], i0 + j < ns ? wl[min(i0 + j, ns - 1) * R + h] : 0.0f, O);
        }
        const float L = hs[h * 4 + 1];
        const float out = L > 0.0f ? O / L : 0.0f;
        const size_t col = (size_t)(kvh * R + h) * HD + d;
        if (live && att_f32) att_f32[col] = out;
        if constexpr (QF >= 0) {
            // 32 consecutive threads hold one 32-group of a head's outputs
            float am = live ? fabsf(out) : 0.0f;
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 32));
            am = fmaxf(am, 0.0f);
            const float sc = group_scale<QF>(am);
            if (live) {
                aq[col] = (int8_t)quant_one<QF>(out, sc);
                if ((d & 31) == 0) as[col / kGroup] = sc;
            }
        }
    }
    if (tid == 0) __hip_atomic_store(counters + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int attn_split_parts(int n_kv_heads) {
    const int ns = n_kv_heads > 0 ? 256 / n_kv_heads : 1;
    return ns < 1 ? 1 : (ns > kSplitMaxParts ? kSplitMaxParts : ns);
}

size_t attn_split_bytes(int n_heads, int n_kv_heads, int head_size) {
    const int ns = attn_split_parts(n_kv_heads);
    return (size_t)n_kv_heads * ns * (n_heads / n_kv_heads) * (head_size + 2) * sizeof(float) +
           256 + (size_t)n_kv_heads * sizeof(unsigned);
}

bool attn_split_supported(int n_heads, int n_kv_heads, int head_size) {
    if (n_kv_heads <= 0 || n_heads % n_kv_heads) return false;
    const int r = n_heads / n_kv_heads;
    return (head_size == 64 || head_size == 128) && (r == 1 || r == 2 || r == 4 || r == 8);
}

template <int QF, int HD, int R>
static hipError_t launch_split_k(const float* sq, const float* kc, const float* vc, const StepState* st,
                                 int n_kv_heads, int kv_ld, float scale, float* scratch, int8_t* aq, float* as,
                                 float* att_f32, hipStream_t s) {
    const int ns = attn_split_parts(n_kv_heads);
    const size_t part_bytes = (size_t)n_kv_heads * ns * R * (HD + 2) * sizeof(float);
    unsigned* counters = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(scratch) + ((part_bytes + 255) & ~(size_t)255));
    const size_t smem = (size_t)split_lds_floats(HD, R) * sizeof(float);
    if (smem > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_split<QF, HD, R>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_attn_split<QF, HD, R>), dim3(n_kv_heads, ns), dim3(kSplitThreads), smem, s, sq, kc, vc, st,
                       n_kv_heads, kv_ld, scale, ns, scratch, counters, aq, as, att_f32);
    return hipGetLastError();
}

template <int QF, int HD>
static hipError_t launch_split_r(int r, const float* sq, const float* kc, const float* vc, const StepState* st,
                                 int n_kv_heads, int kv_ld, float scale, float* scratch, int8_t* aq, float* as,
                                 float* att_f32, hipStream_t s) {
    switch (r) {
    case 1: return launch_split_k<QF, HD, 1>(sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    case 2: return launch_split_k<QF, HD, 2>(sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    case 4: return launch_split_k<QF, HD, 4>(sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    case 8: return launch_split_k<QF, HD, 8>(sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    default: return hipErrorInvalidValue;
    }
}

template <int QF>
static hipError_t launch_split_q(int hd, int r, const float* sq, const float* kc, const float* vc,
                                 const StepState* st, int n_kv_heads, int kv_ld, float scale, float* scratch,
                                 int8_t* aq, float* as, float* att_f32, hipStream_t s) {
    if (hd == 64) return launch_split_r<QF, 64>(r, sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    if (hd == 128) return launch_split_r<QF, 128>(r, sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    return hipErrorInvalidValue;
}

hipError_t launch_attn_split(const float* sq, const float* kc, const float* vc, const StepState* st, int kv_ld,
                             int n_heads, int n_kv_heads, int head_size, float scale, int qfmt, int8_t* aq, float* as,
                             float* att_f32, float* scratch, hipStream_t s) {
    if (!scratch || kv_ld % 4 || !attn_split_supported(n_heads, n_kv_heads, head_size)) return hipErrorInvalidValue;
    const int r = n_heads / n_kv_heads;
    if (qfmt == kQ8)
        return launch_split_q<kQ8>(head_size, r, sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    if (qfmt == kQ4)
        return launch_split_q<kQ4>(head_size, r, sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
    return launch_split_q<-1>(head_size, r, sq, kc, vc, st, n_kv_heads, kv_ld, scale, scratch, aq, as, att_f32, s);
}

}  // namespace yl
