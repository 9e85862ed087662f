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
// the FFN output with 0) pass acc_cols = 0.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

// Tile kernel: a workgroup of 256 threads owns R consecutive output rows
// (their weights are R*n contiguous bytes) and TB consecutive tokens.
//   0. The tokens' quantized rows and scales and the tile's weight scales go
//      to LDS.  With a prologue (one token per workgroup) the row is made
//      here from f32: RMSNorm (util.rs:389-426: the 8 lane chains of squares
//      in element order, o = w * (ss * x)) when PRO == 2, then quantization
//      in groups of gs (quantization.rs:29-52).  The first weight loads are
//      issued before the prologue.
//   1. Threads walk the tile in 16-byte chunks (consecutive threads,
//      consecutive chunks: each wavefront load is 1 KB of contiguous
//      weights).  A chunk's exact int32 dot with the activation (v_dot4) is
//      combined with the other chunks of its group -- integer sums, so in any
//      order -- by cross-lane xor shuffles when gs/16 is a power of two up to
//      64 (the group's chunks sit in consecutive lanes of one wavefront),
//      else by LDS atomic adds.
//   2. One thread per (token, row) forms the row's terms
//      ((float)isum * w_scale) * x_scale in group order and adds them onto
//      the accumulator one at a time: the reference's serial `xout += term`.
// Epilogues: EPI 0 stores to up to three row segments (q, k, v of a fused
// projection), each with its own addressing and `+=` columns; EPI 1 adds the
// chain (from 0) to the output (the residual adds of forward.rs:196-204,
// 244-253); EPI 2 takes tiles of R rows holding R/2 gate rows then the R/2
// up rows of the same columns (the upload interleaves w1 and w3 so, in
// blocks of 16 or 32 rows) and writes h = silu(gate) * up
// (forward.rs:220-237).  With perm_hd, segments 0 and 1 (q and k) hold
// each head's rows in util::rope's pair order (qk_column), and results go
// to the rows' own columns.
constexpr int kQ8gThreads = 256;
constexpr int kQ8gUnroll = 8;    // 16-byte weight loads per thread per batch (two batches in flight)

// rows [previous row_end, row_end) of the matrix go to `out`: element
// (token t, column c) at out[pos * pos_stride + t * stride_tok + c * stride_row]
// (pos = st->pos, 0 without a step state); columns below acc_cols start
// their chain from the output's value
struct Q8gSeg {
    float* out;
    long pos_stride, stride_row, stride_tok;
    int row_end, acc_cols;
};
struct Q8gOut {
    Q8gSeg seg[3];
    int nseg;
    int perm_hd;   // 0, or the head size of segments 0 and 1 stored in pair order
};

// squares row of one RMSNorm chain: n/8 values + zero padding to a multiple
// of 32 (whole read batches of lds_serial_sum; +0 added to a sum of squares
// changes nothing), + 4 floats so the 8 chains start on distinct bank quads
__host__ __device__ inline int q8g_norm_len(int n) { return (n / 8 + 31) & ~31; }
__host__ __device__ inline int q8g_norm_stride(int n) { return q8g_norm_len(n) + 4; }
// per-row stride of the scale and term arrays: G rounded up to 32, + 4
// (the chain lanes' 16-byte reads then start on distinct bank quads)
__host__ __device__ inline int q8g_gpad(int G) { return ((G + 31) & ~31) + 4; }

// activation scales: TB*G floats rounded up to 4 (keeps the term rows 16-byte aligned)
__host__ __device__ inline int q8g_xs_len(int tb, int G) { return (tb * G + 3) & ~3; }

// LDS bytes: xl TB*n | xsl q8g_xs_len*4 | wsl R*GP*4 | terms TB*R*GP*4 | res TB*R*4
// | prologue: xf n*4 | (PRO 2) xt 8*S*4 + red 64 + norm weights n*4
__host__ __device__ inline size_t q8g_lds_bytes(int tb, int pro, int n, int G, int R) {
    const size_t GP = (size_t)q8g_gpad(G);
    size_t b = (size_t)tb * n + (size_t)q8g_xs_len(tb, G) * 4 + (size_t)R * GP * 4 + (size_t)tb * R * GP * 4 +
               (size_t)((tb * R + 3) & ~3) * 4;
    if (pro >= 1) b += (size_t)n * 4;
    if (pro == 2) b += (size_t)8 * q8g_norm_stride(n) * 4 + 64 + (size_t)n * 4;
    return b;
}

template <int TB, int PRO, int EPI>
__global__ __launch_bounds__(kQ8gThreads) void k_matmul_q8g(
    const int8_t* __restrict__ w, const float* __restrict__ wsc, int n, int o, int gs, int R, int lg,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, const float* __restrict__ x,
    const float* __restrict__ norm_w, float eps, int batch, Q8gOut dst, const StepState* __restrict__ st) {
    static_assert(PRO == 0 || TB == 1, "a prologue makes one token's row");
    extern __shared__ __align__(16) int lds[];
    const int tid = threadIdx.x;
    const int G = n / gs, GP = q8g_gpad(G), cpr = n / 16;
    const int row0 = blockIdx.x * R;
    const int rows = min(R, o - row0);
    const int t0 = blockIdx.y * TB;
    int* xl = lds;                                              // [TB][n/4] quantized rows
    float* xsl = reinterpret_cast<float*>(xl + TB * (n / 4));   // [TB][G]
    float* wsl = xsl + q8g_xs_len(TB, G);                       // [R][GP] weight scales
    float* trm = wsl + R * GP;                                  // [TB][R][GP] terms (int sums first when lg < 0)
    float* res = trm + TB * R * GP;                             // [TB][R]
    float* xf = res + ((TB * R + 3) & ~3);                      // [n] (prologue)
    float* xt = xf + n;                                         // [8][S] squares (PRO 2)
    float* red = xt + 8 * q8g_norm_stride(n);                   // [16] (PRO 2)

    const int nch = rows * cpr;
    const int4* wt = reinterpret_cast<const int4*>(w + (size_t)row0 * n);
    const int span = kQ8gThreads * kQ8gUnroll;
    // two register batches of weight chunks (A: even batches, B: odd), loaded
    // unconditionally (chunks past the tile re-read its last one, unused) so
    // that each consumer waits only for its own batch
    int4 wa[kQ8gUnroll], wb[kQ8gUnroll];
    auto load_batch = [&](int4 (&dst)[kQ8gUnroll], int c0) {
#pragma unroll
        for (int u = 0; u < kQ8gUnroll; u++) dst[u] = wt[min(c0 + u * kQ8gThreads + tid, nch - 1)];
    };
    load_batch(wa, 0);   // the first weight loads go out before the staging
    load_batch(wb, span);

    if constexpr (PRO == 0) {
        for (int tb = 0; tb < TB; tb++) {
            const bool live = t0 + tb < batch;
            const int* xr = reinterpret_cast<const int*>(xq + (size_t)(t0 + tb) * n);
            for (int i = tid; i < n / 4; i += kQ8gThreads) xl[tb * (n / 4) + i] = live ? xr[i] : 0;
            for (int i = tid; i < G; i += kQ8gThreads) xsl[tb * G + i] = live ? xs[(size_t)(t0 + tb) * G + i] : 0.0f;
        }
    } else {
        // the row (and the norm weights) in 16-byte loads, eight per thread
        // in flight: n/4 vf4 over 256 threads
        const vf4* xr4 = reinterpret_cast<const vf4*>(x + (size_t)t0 * n);
        const vf4* nw4 = reinterpret_cast<const vf4*>(norm_w);
        vf4* xf4 = reinterpret_cast<vf4*>(xf);
        vf4* wn4 = reinterpret_cast<vf4*>(xt + 8 * q8g_norm_stride(n) + 16);   // (PRO 2) norm weights
        const int S = q8g_norm_stride(n), L8 = q8g_norm_len(n), n8 = n / 8;
        for (int b = 0; b < n / 4; b += 8 * kQ8gThreads) {
            vf4 v[8], wv8[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i4 = b + k * kQ8gThreads + tid;
                if (i4 < n / 4) {
                    v[k] = xr4[i4];
                    if constexpr (PRO == 2) wv8[k] = nw4[i4];
                }
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i4 = b + k * kQ8gThreads + tid;
                if (i4 < n / 4) {
                    xf4[i4] = v[k];
                    if constexpr (PRO == 2) {
                        wn4[i4] = wv8[k];
                        const int e = i4 * 4;   // elements e..e+3: chains e&7 .. (e&7)+3, index e>>3
                        xt[((e + 0) & 7) * S + (e >> 3)] = fmul(v[k].x, v[k].x);
                        xt[((e + 1) & 7) * S + (e >> 3)] = fmul(v[k].y, v[k].y);
                        xt[((e + 2) & 7) * S + (e >> 3)] = fmul(v[k].z, v[k].z);
                        xt[((e + 3) & 7) * S + (e >> 3)] = fmul(v[k].w, v[k].w);
                    }
                }
            }
        }
        if constexpr (PRO == 2) {
            for (int i = tid; i < 8 * (L8 - n8); i += kQ8gThreads) xt[(i / (L8 - n8)) * S + n8 + i % (L8 - n8)] = 0.0f;
            __syncthreads();
            if (tid < 8)   // chain tid: x[8i + tid]^2 for i = 0, 1, ... in order
                red[tid] = lds_serial_sum(reinterpret_cast<const vf4*>(xt + tid * S), L8 / 32, 0.0f);
            __syncthreads();
            float part[8];
#pragma unroll
            for (int j = 0; j < 8; j++) part[j] = red[j];
            float ss = reduce_add8(part);
            ss = ss / (float)n;
            ss = fadd(ss, eps);
            ss = 1.0f / sqrtf(ss);
            const float* wn = reinterpret_cast<const float*>(wn4);
            for (int i = tid; i < n; i += kQ8gThreads) xf[i] = fmul(wn[i], fmul(ss, xf[i]));
        }
        __syncthreads();
        // group absmax, one thread per group (order-free; fmaxf ignores NaN
        // as the reference's f32::max does)
        for (int g = tid; g < G; g += kQ8gThreads) {
            const vf4* v4 = reinterpret_cast<const vf4*>(xf + g * gs);
            float am = 0.0f;
            for (int k = 0; k < gs / 4; k++) {
                const vf4 v = v4[k];
                am = fmaxf(am, fabsf(v.x));
                am = fmaxf(am, fabsf(v.y));
                am = fmaxf(am, fabsf(v.z));
                am = fmaxf(am, fabsf(v.w));
            }
            xsl[g] = group_scale<kQ8>(am);
        }
        __syncthreads();
        // quantize 8 values at a time (x * 1/scale with the exact division
        // where rounding could differ)
        uint2* xb8 = reinterpret_cast<uint2*>(xl);
        for (int j = tid; j < n / 8; j += kQ8gThreads) {
            const vf4 a = xf4[2 * j], b = xf4[2 * j + 1];
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            int q[8];
            quant8<kQ8>(v, xsl[(j * 8) / gs], q);
            xb8[j] = make_uint2(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]));
        }
    }
    const float* wsr = wsc + (size_t)row0 * G;
    for (int i = tid; i < rows * G; i += kQ8gThreads) {
        const int r = i / G;
        wsl[r * GP + (i - r * G)] = wsr[i];
    }
    if (lg < 0)
        for (int i = tid; i < TB * R * GP; i += kQ8gThreads) trm[i] = 0.0f;   // int 0
    __syncthreads();

    // chunk c = c0 + u * 256 + tid lies in tile row r at chunk kc of the row;
    // (r, kc) advance by 256 chunks per step without a division
    const int dr = kQ8gThreads / cpr, dk = kQ8gThreads % cpr;
    int r_c = tid / cpr, k_c = tid - r_c * cpr;
    const int gmask = lg >= 0 ? (1 << lg) - 1 : 0;
    // one batch: U chunks per thread (uniform trip counts: the shuffles see every lane)
    auto consume = [&](const int4 (&wv)[kQ8gUnroll], int c0) {
#pragma unroll
        for (int u = 0; u < kQ8gUnroll; u++) {
            const int c = c0 + u * kQ8gThreads + tid;
            const bool live = c < nch;
            const int r = r_c, kc = k_c;
            k_c += dk;
            r_c += dr;
            if (k_c >= cpr) { k_c -= cpr; r_c++; }
            const int g = lg >= 0 ? kc >> lg : (kc * 16) / gs;
#pragma unroll
            for (int tb = 0; tb < TB; tb++) {
                const int4 xv = *reinterpret_cast<const int4*>(xl + tb * (n / 4) + kc * 4);
                int p = __builtin_amdgcn_sdot4(wv[u].x, xv.x, 0, false);
                p = __builtin_amdgcn_sdot4(wv[u].y, xv.y, p, false);
                p = __builtin_amdgcn_sdot4(wv[u].z, xv.z, p, false);
                p = __builtin_amdgcn_sdot4(wv[u].w, xv.w, p, false);
                float* d = trm + (tb * R + r) * GP + g;
                if (lg >= 0) {
                    for (int sh = 0; sh < lg; sh++) p += __shfl_xor(p, 1 << sh, 64);
                    // the group's first lane writes its term ((float)isum * w_scale) * x_scale
                    if (live && (kc & gmask) == 0) *d = fmul(fmul((float)p, wsl[r * GP + g]), xsl[tb * G + g]);
                } else if (live) {
                    atomicAdd(reinterpret_cast<int*>(d), p);
                }
            }
        }
    };
    for (int c0 = 0; c0 < nch; c0 += 2 * span) {
        consume(wa, c0);
        load_batch(wa, c0 + 2 * span);
        if (c0 + span < nch) consume(wb, c0 + span);
        load_batch(wb, c0 + 3 * span);
    }
    if (lg < 0) {   // integer sums -> terms
        __syncthreads();
        for (int i = tid; i < TB * R * GP; i += kQ8gThreads) {
            const int tb = i / (R * GP), rem = i - tb * R * GP, r = rem / GP, g = rem - r * GP;
            if (g < G)
                trm[i] = fmul(fmul((float)reinterpret_cast<const int*>(trm)[i], wsl[r * GP + g]), xsl[tb * G + g]);
        }
    }
    __syncthreads();

    for (int j = tid; j < TB * rows; j += kQ8gThreads) {
        const int tb = j / rows, r = j - tb * rows;
        const int t = t0 + tb;
        if (t >= batch) continue;
        const int c = row0 + r;
        int sg = 0;
        if constexpr (EPI == 0)
            while (sg + 1 < dst.nseg && c >= dst.seg[sg].row_end) sg++;
        const Q8gSeg& q = dst.seg[sg];
        int col = c - (sg ? dst.seg[sg - 1].row_end : 0);
        if constexpr (EPI == 0)
            if (sg < 2) col = qk_column(col, dst.perm_hd, dst.perm_hd);
        const size_t at = (st ? (size_t)st->pos * q.pos_stride : 0) + (size_t)t * q.stride_tok + (size_t)col * q.stride_row;
        float acc = (EPI == 0 && col < q.acc_cols) ? q.out[at] : 0.0f;
        const float* tr = trm + (tb * R + r) * GP;
        int g = 0;
        for (; g + 4 <= G; g += 4) {   // terms in group order, four per 16-byte read
            const vf4 v = *reinterpret_cast<const vf4*>(tr + g);
            acc = fadd(acc, v.x);
            acc = fadd(acc, v.y);
            acc = fadd(acc, v.z);
            acc = fadd(acc, v.w);
        }
        for (; g < G; g++) acc = fadd(acc, tr[g]);
        if constexpr (EPI == 0) q.out[at] = acc;
        else if constexpr (EPI == 1) q.out[at] = fadd(q.out[at], acc);
        else res[tb * R + r] = acc;
    }
    if constexpr (EPI == 2) {
        __syncthreads();
        const Q8gSeg& q = dst.seg[0];
        const int PR = R / 2;   // gate rows, then as many up rows
        for (int j = tid; j < TB * PR; j += kQ8gThreads) {
            const int tb = j / PR, cc = j - tb * PR;
            const int t = t0 + tb;
            if (t >= batch || cc >= rows / 2) continue;
            const float g = res[tb * R + cc], u = res[tb * R + PR + cc];
            const float den = fadd(1.0f, expf_rn(-g));
            q.out[(size_t)t * q.stride_tok + (size_t)(blockIdx.x * PR + cc) * q.stride_row] = fmul(g / den, u);
        }
    }
}

// quantization::quantize (quantization.rs:29-52) over `groups` groups of gs.
// Quantization in groups of gs = 8 * 2^LG (32 .. 512): 8 consecutive
// elements per lane (coalesced 16-byte loads), the group's absmax over its
// 2^LG lanes by xor shuffles, then quant8 (the same integers as quant_one).
template <int LG>
__global__ void k_quantize_gs_v(const float* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ s,
                                size_t n8) {
    constexpr int LPG = 1 << LG;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;   // 8-element slice
    const bool live = i < n8;   // a group's lanes are all live or all past the end
    vf4 a = vf4{0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (live) {
        a = reinterpret_cast<const vf4*>(x)[2 * i];
        b = reinterpret_cast<const vf4*>(x)[2 * i + 1];
    }
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(v[k]));
#pragma unroll
    for (int off = 1; off < LPG; off <<= 1) am = fmaxf(am, __shfl_xor(am, off, 64));
    const float sc = group_scale<kQ8>(am);
    int qv[8];
    quant8<kQ8>(v, sc, qv);
    if (live) {
        *reinterpret_cast<uint2*>(q + 8 * i) = make_uint2(pack4(qv[0], qv[1], qv[2], qv[3]), pack4(qv[4], qv[5], qv[6], qv[7]));
        if ((i & (LPG - 1)) == 0) s[i >> LG] = sc;
    }
}

// Any other group size: one thread per group.
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

template <int TB, int PRO, int EPI>
static hipError_t launch_q8g_t(const Q8gArgs& a, int R, int lg, size_t lds, hipStream_t s) {
    auto k = k_matmul_q8g<TB, PRO, EPI>;
    static bool raised = false;
    if (lds > 65536 && !raised) {
        const hipError_t e =
            hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        raised = true;
    }
    Q8gOut d{};
    d.nseg = a.nseg;
    d.perm_hd = a.perm_hd;
    for (int i = 0; i < a.nseg; i++)
        d.seg[i] = Q8gSeg{a.seg[i].out, a.seg[i].pos_stride, a.seg[i].stride_row, a.seg[i].stride_tok,
                          a.seg[i].row_end, a.seg[i].acc_cols};
    const int gy = (a.batch + TB - 1) / TB;
    hipLaunchKernelGGL(k, dim3((a.o + R - 1) / R, gy), dim3(kQ8gThreads), lds, s, a.w, a.wsc, a.n, a.o, a.gs, R, lg,
                       a.xq, a.xs, a.x, a.norm_w, a.eps, a.batch, d, a.st);
    return hipGetLastError();
}

hipError_t launch_matmul_q8g(const Q8gArgs& a, hipStream_t s) {
    const int n = a.n, o = a.o, gs = a.gs;
    if (gs <= 0 || gs % 32 || n <= 0 || n % gs || o <= 0 || a.batch <= 0 || a.nseg < 1 || a.nseg > 3 ||
        a.pro < 0 || a.pro > 2 || a.epi < 0 || a.epi > 2 || (a.pro > 0 && a.batch > 65535) ||
        (long)a.batch > 65535L * 4 || a.seg[a.nseg - 1].row_end != o)
        return hipErrorInvalidValue;
    if (a.epi == 2 && ((a.pair_rows != 16 && a.pair_rows != 32) || o % (2 * a.pair_rows))) return hipErrorInvalidValue;
    if (a.perm_hd && ((a.perm_hd & (a.perm_hd - 1)) || a.perm_hd < 2 || a.nseg < 2 || a.seg[0].row_end % a.perm_hd ||
                      (a.seg[1].row_end - a.seg[0].row_end) % a.perm_hd))
        return hipErrorInvalidValue;
    const int G = n / gs;
    int tb = a.pro > 0 || a.batch == 1 ? 1 : 4;
    // a SwiGLU tile of 32 + 32 rows over a long row takes one token per
    // workgroup when four do not fit in LDS
    if (a.epi == 2 && q8g_lds_bytes(tb, a.pro, n, G, 2 * a.pair_rows) > 160 * 1024) tb = 1;
    const int gy = (a.batch + tb - 1) / tb;
    // rows per workgroup: about 1024 workgroups over the chip (256 when each
    // workgroup makes its own input row), dividing every segment boundary,
    // within 64 KB of LDS (EPI 2: one gate/up tile pair)
    int R = 64;
    if (a.epi == 2) {
        R = 2 * a.pair_rows;
    } else {
        const long want = a.pro > 0 ? 256 : 1024;
        while (R > 1 && (long)((o + R - 1) / R) * gy < want) R /= 2;
        for (int i = 0; i < a.nseg; i++)
            while (R > 1 && a.seg[i].row_end % R) R /= 2;
        while (R > 1 && q8g_lds_bytes(tb, a.pro, n, G, R) > 65536) R /= 2;
    }
    const size_t lds = q8g_lds_bytes(tb, a.pro, n, G, R);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    const int cpg = gs / 16;
    const int lg = (cpg <= 64 && (cpg & (cpg - 1)) == 0) ? __builtin_ctz(cpg) : -1;
#define YL_Q8G(TB_, PRO_, EPI_) \
    if (tb == TB_ && a.pro == PRO_ && a.epi == EPI_) return launch_q8g_t<TB_, PRO_, EPI_>(a, R, lg, lds, s);
    YL_Q8G(1, 0, 0) YL_Q8G(1, 0, 1) YL_Q8G(1, 0, 2)
    YL_Q8G(4, 0, 0) YL_Q8G(4, 0, 1) YL_Q8G(4, 0, 2)
    YL_Q8G(1, 1, 0) YL_Q8G(1, 1, 1) YL_Q8G(1, 1, 2)
    YL_Q8G(1, 2, 0) YL_Q8G(1, 2, 1) YL_Q8G(1, 2, 2)
#undef YL_Q8G
    return hipErrorInvalidValue;
}

hipError_t launch_quantize_gs(const float* x, int8_t* q, float* sc, int gs, size_t n, hipStream_t s) {
    if (gs <= 0 || n % gs) return hipErrorInvalidValue;
    const size_t groups = n / gs;
    if (!groups) return hipSuccess;
    const size_t n8 = n / 8;
    const dim3 g8((unsigned)((n8 + 255) / 256));
    switch (gs) {
    case 32: hipLaunchKernelGGL(k_quantize_gs_v<2>, g8, dim3(256), 0, s, x, q, sc, n8); return hipGetLastError();
    case 64: hipLaunchKernelGGL(k_quantize_gs_v<3>, g8, dim3(256), 0, s, x, q, sc, n8); return hipGetLastError();
    case 128: hipLaunchKernelGGL(k_quantize_gs_v<4>, g8, dim3(256), 0, s, x, q, sc, n8); return hipGetLastError();
    case 256: hipLaunchKernelGGL(k_quantize_gs_v<5>, g8, dim3(256), 0, s, x, q, sc, n8); return hipGetLastError();
    case 512: hipLaunchKernelGGL(k_quantize_gs_v<6>, g8, dim3(256), 0, s, x, q, sc, n8); return hipGetLastError();
    default: break;
    }
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
