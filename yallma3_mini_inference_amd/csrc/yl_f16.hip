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
//   decode (one token): a workgroup owns 64 output rows, one chain lane
//   each, fed from LDS by three product wavefronts (below).  The prologue
//   can apply RMSNorm (util.rs:389-426) to the input row, and the epilogue
//   add the residual or form SwiGLU from gate/up row pairs;
//   batches: a workgroup takes 64 rows x 64 tokens, each lane running 16
//   token chains of its row, the weight and activation tiles shared through
//   LDS.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {


__device__ __forceinline__ float h2f(uint32_t bits16) { return f16_to_f32((uint16_t)bits16); }

// 8 halves of a uint4 -> w[8]
__device__ __forceinline__ void widen8(const uint4& v, float w[8]) {
    w[0] = h2f(v.x & 0xffffu); w[1] = h2f(v.x >> 16);
    w[2] = h2f(v.y & 0xffffu); w[3] = h2f(v.y >> 16);
    w[4] = h2f(v.z & 0xffffu); w[5] = h2f(v.z >> 16);
    w[6] = h2f(v.w & 0xffffu); w[7] = h2f(v.w >> 16);
}

// ------------------------------------------------------------- one token
// A workgroup owns R output rows.  Wavefront 0 is the chain wavefront: lane
// r adds row r's products in column order, one f32 add after another
// (matmul_f32's serial sum).  A dependent add issues every ~4-5 cycles, so
// the wavefront needs its SIMD to itself and its operands in LDS: PW
// product wavefronts (on the other SIMDs) widen the f16 weights, multiply
// them by the activations and write R-row x 64-column product tiles into a
// ring of LDS slots (8, or 4 for R = 64), their weight loads D tiles ahead
// in registers.  Hand-offs use LDS counters, not barriers: each product
// wavefront counts the tiles it has written, the chain wavefront counts the
// tiles it has read (`consumed`), a tile is ready when every product
// wavefront's count passed it, and a product wavefront refills a slot only
// once its previous tile was consumed.  The chain wavefront reads the next
// tile's 64 products per lane while it adds the current one's (two register
// sets, unconditional reads), so its adds never wait for LDS, and checks
// the counts only when it reaches the last tile it knew to be ready.
//
// One CU streams only ~20 GB/s of weights, so a projection needs about 256
// workgroups to reach HBM bandwidth: R is chosen per matrix (64 rows for
// the gate/up matrix, 8-32 for the others), and the chain, whose length n
// is fixed, runs on every CU at once.
constexpr int kFgThreadsMax = 256;
constexpr int kFgKT = 64;                   // columns per tile
constexpr int kFgStride = kFgKT + 4;        // product row stride (floats): the 16 lanes of a read hit distinct banks
constexpr int kFgPairRows = 32;             // EPI 2: 32 gate rows, then their 32 up rows (R = 64)
static_assert(kFgPairRows == kF16PairRows, "the upload's gate/up interleave");

// Shape of a variant: R rows, PW product wavefronts, each product lane
// taking CPL 16-byte chunks (8 columns of one row) per tile, D tiles of
// loads in flight.
template <int R>
struct FgShape {
    static constexpr int PW = R == 64 ? 3 : (R == 8 ? 1 : 2);
    static constexpr int CPL = (8 * R + 64 * PW - 1) / (64 * PW);
    static constexpr int D = R == 8 ? 12 : (R == 16 ? 8 : (R == 32 ? 8 : 4));
    static constexpr int threads = 64 * (1 + PW);
    static constexpr int slot_floats = R * kFgStride;
    static constexpr int slots = R == 64 ? 4 : 8;   // tiles in the LDS ring
};

// LDS floats: counters 8 | product slots [slots][R][68] | the input row:
// without PRO the row (rounded to whole 1 KiB DMA rows), with PRO the
// RMSNorm staging (squares in 8 chain rows | row | norm weights)
__host__ __device__ inline size_t fg_row_floats(int n, int pro) {
    return pro ? rowq_lds_floats(n) : (size_t)rowq_row_len(n);
}
__host__ __device__ inline size_t fg_lds_floats(int n, int pro, int R) {
    return 8 + (size_t)(R == 64 ? 4 : 8) * R * kFgStride + fg_row_floats(n, pro);
}

__device__ __forceinline__ float f16_prod(uint32_t bits16, float x) { return fmul(h2f(bits16), x); }

// half h of a tile row of products (32 floats, 8 reads) of row `row` from
// slot `s`
template <int R>
__device__ __forceinline__ void fg_read_half(vf4 (&v)[16], const float* P, int s, int row, int h) {
    const vf4* r = reinterpret_cast<const vf4*>(P + s * FgShape<R>::slot_floats + row * kFgStride) + 8 * h;
#pragma unroll
    for (int i = 0; i < 8; i++) v[8 * h + i] = r[i];
}
// the serial adds of half h of a tile row
__device__ __forceinline__ float fg_add_half(float acc, const vf4 (&v)[16], int h) {
#pragma unroll
    for (int i = 8 * h; i < 8 * h + 8; i++) {
        acc = fadd(acc, v[i].x); acc = fadd(acc, v[i].y); acc = fadd(acc, v[i].z); acc = fadd(acc, v[i].w);
    }
    return acc;
}
// The adds of tile row `cur` (kn = 64 or 32 columns) with the reads of the
// next tile's row into `nxt` issued half by half ahead of them: at most 8
// reads are new when an add waits, so the 4-bit LDS wait count (15) never
// makes an add wait for a read of the next tile.
template <int R>
__device__ __forceinline__ float fg_add_tile(float acc, const vf4 (&cur)[16], vf4 (&nxt)[16], const float* P, int s,
                                             int row, int kn) {
    fg_read_half<R>(nxt, P, s, row, 0);
    __builtin_amdgcn_sched_barrier(0);
    acc = fg_add_half(acc, cur, 0);
    __builtin_amdgcn_sched_barrier(0);
    fg_read_half<R>(nxt, P, s, row, 1);
    __builtin_amdgcn_sched_barrier(0);
    if (kn > 32) acc = fg_add_half(acc, cur, 1);
    __builtin_amdgcn_sched_barrier(0);
    return acc;
}

// PRO 1: x <- RMSNorm(x) * norm_w first.  EPI 0: out[r] = sum; EPI 1: out[r]
// += sum (the residual add); EPI 2 (R = 64): out[32 * blockIdx.x + c] =
// silu(g) * u of rows (c, c + 32) of the workgroup (forward.rs:220-237);
// EPI 3: the QKV step (F16Qkv): pairs of adjacent rows rotated, q stored, k
// and v assigned into the caches (forward.rs:149-179 with the F16Kernel).
template <int PRO, int EPI, int R>
__global__ __launch_bounds__(kFgThreadsMax) void k_f16_gemv(const uint16_t* __restrict__ w, int n, int o,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ norm_w, float eps,
                                                            float* __restrict__ out, unsigned* fault, F16Qkv qa) {
    using Sh = FgShape<R>;
    constexpr int PW = Sh::PW, CPL = Sh::CPL, D = Sh::D, SF = Sh::slot_floats, SL = Sh::slots;
    static_assert(EPI != 2 || R == 2 * kFgPairRows, "SwiGLU tiles are 64 rows");
    extern __shared__ __align__(16) float lds[];
    int* ctr = reinterpret_cast<int*>(lds);   // [0..PW-1] tiles written per product wavefront, [4] tiles consumed,
                                              // [5] input row ready
    float* P = lds + 8;                       // [SL][R][68]
    float* sq = P + SL * SF;
    float* xl = PRO ? sq + 8 * rowq_stride(n) : sq;   // the input row
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = blockIdx.x * R;
    const int ntile = (n + kFgKT - 1) / kFgKT;
    // the counters start at zero (LDS holds whatever the previous workgroup left)
    if (tid < 8) ctr[tid] = 0;
    __syncthreads();

    if (wave == 0) {
        // ------------------------------------------------- chain wavefront
        // first the input row, by LDS DMA (this wavefront has no other
        // loads in flight): with PRO, RMSNorm (util.rs:389-426: the 8 lane
        // chains of squares, o = w * (ss * x)) in place; then the product
        // wavefronts may start
        rowq_dma_f32(xl, x, n);
        if constexpr (PRO) rowq_dma_f32(xl + rowq_row_len(n), norm_w, n);
        wait_vm_all();
        if constexpr (PRO) {
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            rowq_squares_wave(n, sq);
            const float ss = rowq_chain(n, eps, sq);
            const float* wl = xl + rowq_row_len(n);
            for (int e = 8 * lane; e < n; e += 512) {
                vf4* xv = reinterpret_cast<vf4*>(xl + e);
                const vf4* wv = reinterpret_cast<const vf4*>(wl + e);
                const vf4 a = xv[0], b = xv[1], wa = wv[0], wb = wv[1];
                xv[0] = vf4{fmul(wa.x, fmul(ss, a.x)), fmul(wa.y, fmul(ss, a.y)), fmul(wa.z, fmul(ss, a.z)),
                            fmul(wa.w, fmul(ss, a.w))};
                xv[1] = vf4{fmul(wb.x, fmul(ss, b.x)), fmul(wb.y, fmul(ss, b.y)), fmul(wb.z, fmul(ss, b.z)),
                            fmul(wb.w, fmul(ss, b.w))};
            }
        }
        lds_arrive(ctr + 5);

        // tiles t < ready are known filled: the least of the product
        // wavefronts' counts
        auto refresh = [&](int t) {
            for (int it = 0; it < (1 << 22); it++) {
                int c[PW];
#pragma unroll
                for (int k = 0; k < PW; k++)
                    c[k] = __builtin_amdgcn_readfirstlane(
                        __hip_atomic_load(ctr + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
                int r = c[0];
#pragma unroll
                for (int k = 1; k < PW; k++) r = min(r, c[k]);
                if (r > t) return r;
            }
            // (every lane stores the same word: no divergent branch in the
            // chain's control flow, which stays in scalar registers)
            if (fault) __hip_atomic_store(fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return ntile;
        };
        // the chain's adds go first when a product wavefront shares the SIMD
        __builtin_amdgcn_s_setprio(3);
        // lanes past R re-read row R - 1 (unused)
        const int myrow = lane < R ? lane : R - 1;
        float acc = 0.0f;
        vf4 ra[16], rb[16];
        int ready = __builtin_amdgcn_readfirstlane(refresh(0));
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        fg_read_half<R>(ra, P, 0, myrow, 0);
        fg_read_half<R>(ra, P, 0, myrow, 1);
        // two tiles per pair: ra holds tile t, rb is read with tile t + 1.
        // Eight tiles per trip, so every slot index is a constant and the
        // reads address LDS by immediate offsets from one register; a read
        // past the last tile reads a stale slot whose adds never run.
        static_assert(8 % SL == 0, "slots per trip");
        for (int t0 = 0; t0 < ntile; t0 += 8) {
#pragma unroll
            for (int k = 0; k < 8; k += 2) {
                const int t = t0 + k;
                if (t >= ntile) break;
                if (t + 1 < ntile && t + 1 >= ready) ready = __builtin_amdgcn_readfirstlane(refresh(t + 1));
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                acc = fg_add_tile<R>(acc, ra, rb, P, (k + 1) % SL, myrow, min(kFgKT, n - t * kFgKT));
                if (t + 1 >= ntile) {
                    lds_arrive_nowait(ctr + 4);
                    break;
                }
                if (t + 2 < ntile && t + 2 >= ready) ready = __builtin_amdgcn_readfirstlane(refresh(t + 2));
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                acc = fg_add_tile<R>(acc, rb, ra, P, (k + 2) % SL, myrow, min(kFgKT, n - (t + 1) * kFgKT));
                // tiles t and t + 1 consumed (one count per two tiles; a
                // store: the chain wavefront is the counter's one writer)
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                if (lane == 0) __hip_atomic_store(ctr + 4, t + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
            }
        }
        const int row = row0 + lane;
        if constexpr (EPI == 3) {
            // rope_gguf (util.rs:653-718) on rows (2i, 2i+1), or util::rope's
            // pair (j, j + head/2) stored there (qk_column); the partner row
            // is the neighbouring lane (R is even, rows start even)
            const float other = dpp_mov<0xB1>(acc);   // quad_perm [1,0,3,2]: lane ^ 1
            if (lane < R && row < o) {
                const int pos = qa.st->pos;
                const int att = qa.att, kv = qa.kv, hd = qa.hd;
                if (row >= att + kv) {
                    qa.v_cache[(size_t)pos * kv + (row - att - kv)] = acc;
                } else {
                    const int scol = row < att ? row : row - att;
                    const int col = qk_column(scol, hd, qa.hf);
                    const int pair = (scol % hd) >> 1;
                    const float c = qa.rope_cos[(size_t)pos * (hd >> 1) + pair];
                    const float sn = qa.rope_sin[(size_t)pos * (hd >> 1) + pair];
                    const bool odd = row & 1;
                    const float v0 = odd ? other : acc, v1 = odd ? acc : other;
                    const float r = odd ? fadd(fmul(v0, sn), fmul(v1, c)) : fmul(v0, c) - fmul(v1, sn);
                    if (row < att) qa.q_out[col] = r;
                    else qa.k_cache[(size_t)col * qa.kv_ld + pos] = r;
                }
            }
        } else if constexpr (EPI == 2) {
            const float u = __shfl_down(acc, kFgPairRows, 64);
            if (lane < kFgPairRows) {
                const float den = fadd(1.0f, expf_rn(-acc));
                out[blockIdx.x * kFgPairRows + lane] = fmul(acc / den, u);
            }
        } else if (lane < R && row < o) {
            float* dst = out + row;
            *dst = EPI == 0 ? acc : fadd(*dst, acc);
        }
    } else {
        // ----------------------------------------------- product wavefronts
        // product lane p (0 .. 64 PW - 1) takes chunks j = p + 64 PW i of
        // each tile: row j / 8, columns 8 (j % 8) .. +8 of the tile.  All of
        // a lane's chunks share its 8 columns, so one pair of x reads serves
        // them; chunk i exists for the wavefronts with PW i + pw < R / 8 (a
        // uniform branch), and the others' loads re-read chunk 8R - 1 (one
        // address per wavefront).  Every load is issued unconditionally
        // (tiles past the last and columns past n re-read in range), so the
        // compiler's wait counts stay exact: a tile's products wait only for
        // that tile's loads.  In a last tile of 32 columns, lanes past n
        // compute products the chain never reads (their x reads stay inside
        // the row's rounded LDS region).
        const int p = tid - 64, pw = wave - 1;
        const int kk = 8 * (p & 7);
        const int r0 = p >> 3;   // row of chunk 0; chunk i is 8 PW i rows further
        uint4 wr[D][CPL];
        auto load_tile = [&](uint4 (&dst)[CPL], int t) {
            const int k0 = min(t, ntile - 1) * kFgKT;
#pragma unroll
            for (int i = 0; i < CPL; i++) {
                const int j = min(p + 64 * PW * i, 8 * R - 1);
                const int k = min(k0 + 8 * (j & 7), n - 8);
                dst[i] = *reinterpret_cast<const uint4*>(w + (size_t)min(row0 + (j >> 3), o - 1) * n + k);
            }
        };
        // iteration t: (once slot t % SL is free) the products of tile t into
        // it, then the loads of tile t + D into the registers tile t used.
        // The trip count is padded to whole rings of D.
        const int nit = (ntile + D - 1) / D * D;
#pragma unroll
        for (int d = 0; d < D; d++) load_tile(wr[d], d);
        lds_wait_count(ctr + 5, 1, fault);   // the input row
        int seen = 0;                        // tiles consumed, as last read
        // the lane's 8 activations of tile t, read one tile ahead (two sets,
        // alternating with d; D is even); reads past the row's last tile
        // stay inside its rounded LDS region
        static_assert(D % 2 == 0, "x register sets alternate");
        vf4 xr[2][2];
        xr[0][0] = *reinterpret_cast<const vf4*>(xl + kk);
        xr[0][1] = *reinterpret_cast<const vf4*>(xl + kk + 4);
        for (int t0 = 0; t0 < nit; t0 += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                const int t = t0 + d;
                if (t < ntile) {
                    if (t >= SL && seen < t - SL + 1) seen = lds_wait_count(ctr + 4, t - SL + 1, fault);
                    const int tn = min(t + 1, ntile - 1);
                    xr[(d + 1) & 1][0] = *reinterpret_cast<const vf4*>(xl + tn * kFgKT + kk);
                    xr[(d + 1) & 1][1] = *reinterpret_cast<const vf4*>(xl + tn * kFgKT + kk + 4);
                    const vf4 xa = xr[d & 1][0], xb = xr[d & 1][1];
                    float* dst = P + (t % SL) * SF + r0 * kFgStride + kk;
#pragma unroll
                    for (int i = 0; i < CPL; i++) {
                        if (PW * i + pw < R / 8) {
                            const uint4 c = wr[d][i];
                            float* q = dst + i * 8 * PW * kFgStride;
                            *reinterpret_cast<vf4*>(q) =
                                vf4{f16_prod(c.x & 0xffffu, xa.x), f16_prod(c.x >> 16, xa.y),
                                    f16_prod(c.y & 0xffffu, xa.z), f16_prod(c.y >> 16, xa.w)};
                            *reinterpret_cast<vf4*>(q + 4) =
                                vf4{f16_prod(c.z & 0xffffu, xb.x), f16_prod(c.z >> 16, xb.y),
                                    f16_prod(c.w & 0xffffu, xb.z), f16_prod(c.w >> 16, xb.w)};
                        }
                    }
                    lds_arrive_nowait(ctr + pw);
                }
                load_tile(wr[d], t + D);
            }
        }
    }
}

// SwiGLU of a batched gate/up product in the pair layout (rows c, c + 32 of
// each 64-row block): raw [batch][2 * hidden] -> h [batch][hidden].
__global__ void k_swiglu_pairs(const float* __restrict__ raw, int hidden, float* __restrict__ h) {
    const int t = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= hidden) return;
    const float* r = raw + (size_t)t * 2 * hidden + (size_t)(c / kFgPairRows) * (2 * kFgPairRows) + c % kFgPairRows;
    const float g = r[0], u = r[kFgPairRows];
    const float den = fadd(1.0f, expf_rn(-g));
    h[(size_t)t * hidden + c] = fmul(g / den, u);
}

// --------------------------------------------------------------- batches
// A workgroup owns 64 rows x 64 tokens: lane r of wavefront w runs the
// chains of row r for the 16 tokens 16w .. 16w+15, one accumulator each, so
// every weight tile is read once per 64 tokens.  Per K tile of 32 columns
// the weights ([64 rows][32 halves], row stride 80 bytes) and the
// activations ([32 columns][64 tokens] f32, read as broadcast vf4 of 4
// tokens) sit in LDS, double-buffered; the next tile's global loads are in
// registers while the current tile is added.  Each chain adds its products
// x[t][k] * w[r][k] in column order (matmul_f32's serial sum).
constexpr int kFbRows = 64;          // rows per workgroup (lane = row)
constexpr int kFbTok = 64;           // tokens per workgroup (16 per wavefront)
constexpr int kFbKT = 32;            // columns per tile
constexpr int kFbWStride = 40;       // halves per weight row in LDS (32 + 8: 16-byte aligned, spread banks)
constexpr int kFbXStride = kFbTok + 4;   // floats per activation column in LDS

template <int EPI>
__global__ __launch_bounds__(256) void k_matmul_f16_batch(const uint16_t* __restrict__ w, int n, int o,
                                                          const float* __restrict__ x, int batch,
                                                          float* __restrict__ out, int out_ld) {
    __shared__ __align__(16) uint16_t wt[2][kFbRows * kFbWStride];
    __shared__ __align__(16) float xt[2][kFbKT * kFbXStride];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = blockIdx.x * kFbRows, tok0 = blockIdx.y * kFbTok;
    const int ntile = (n + kFbKT - 1) / kFbKT;
    // loader thread i: weight chunk (row i / 4, halves 8 (i % 4) .. +8); two
    // activation float4 (token i / 4 ... see below)
    const int wr_row = tid >> 2, wr_c = (tid & 3) * 8;
    uint4 wreg;
    vf4 xreg[2];
    auto load = [&](int t) {
        const int k0 = t * kFbKT;
        const int r = min(row0 + wr_row, o - 1);
        wreg = *reinterpret_cast<const uint4*>(w + (size_t)r * n + min(k0 + wr_c, n - 8));
        // activations: 64 tokens x 32 columns = 512 float4; thread i takes
        // float4 i and i + 256: token (j / 8), columns 4 (j % 8) .. +3
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int j = tid + 256 * h;
            const int tk = min(tok0 + (j >> 3), batch - 1);
            xreg[h] = *reinterpret_cast<const vf4*>(x + (size_t)tk * n + min(k0 + 4 * (j & 7), n - 4));
        }
    };
    auto store = [&](int b) {
        *reinterpret_cast<uint4*>(&wt[b][wr_row * kFbWStride + wr_c]) = wreg;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int j = tid + 256 * h;
            const int tk = j >> 3, c = 4 * (j & 7);
            xt[b][(c + 0) * kFbXStride + tk] = xreg[h].x;
            xt[b][(c + 1) * kFbXStride + tk] = xreg[h].y;
            xt[b][(c + 2) * kFbXStride + tk] = xreg[h].z;
            xt[b][(c + 3) * kFbXStride + tk] = xreg[h].w;
        }
    };
    load(0);
    store(0);
    __syncthreads();
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    for (int t = 0; t < ntile; t++) {
        const int b = t & 1;
        if (t + 1 < ntile) load(t + 1);
        const int kn = min(kFbKT, n - t * kFbKT);   // 32, or 32 (n % 32 == 0)
        const uint16_t* wrow = &wt[b][lane * kFbWStride];
        const float* xc = &xt[b][16 * wave];
#pragma unroll
        for (int c8 = 0; c8 < kFbKT / 8; c8++) {
            if (8 * c8 >= kn) break;
            float wf[8];
            widen8(*reinterpret_cast<const uint4*>(wrow + 8 * c8), wf);
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const float* xk = xc + (8 * c8 + kk) * kFbXStride;
                const vf4 x0 = *reinterpret_cast<const vf4*>(xk), x1 = *reinterpret_cast<const vf4*>(xk + 4),
                          x2 = *reinterpret_cast<const vf4*>(xk + 8), x3 = *reinterpret_cast<const vf4*>(xk + 12);
                const float xs[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                      x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
#pragma unroll
                for (int i = 0; i < 16; i++) acc[i] = fadd(acc[i], fmul(xs[i], wf[kk]));
            }
        }
        if (t + 1 < ntile) store(b ^ 1);
        __syncthreads();
    }
    const int row = row0 + lane;
    if (row < o) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int tk = tok0 + 16 * wave + i;
            if (tk < batch) {
                float* dst = out + (size_t)tk * out_ld + row;
                *dst = EPI == 0 ? acc[i] : fadd(*dst, acc[i]);
            }
        }
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
        // hf_pairs 0: pairs (2j, 2j+1); 1: (j, j + half); 2: util::rope's pair
        // (j, j + half) whose rows are stored at (2j, 2j+1) (qk_column): read
        // there, written to columns (j, j + half)
        const int e0 = head * hd + (hf_pairs == 0 ? 2 * j : j), e1 = e0 + (hf_pairs == 0 ? 1 : half);
        const int s0 = hf_pairs == 2 ? head * hd + 2 * j : e0, s1 = hf_pairs == 2 ? s0 + 1 : e1;
        const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
        const float* src = isq ? r : r + att;
        const float v0 = src[s0], v1 = src[s1];
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
    if (batch == 1) return launch_f16_gemv(w, n, o, x, nullptr, 0.0f, epi, out, s);
    const int rb = (o + kFbRows - 1) / kFbRows;
    auto k = epi == 0 ? k_matmul_f16_batch<0> : k_matmul_f16_batch<1>;
    hipLaunchKernelGGL(k, dim3(rb, (batch + kFbTok - 1) / kFbTok), dim3(256), 0, s, w, n, o, x, batch, out, out_ld);
    return hipGetLastError();
}

template <int PRO, int EPI, int R>
static hipError_t launch_fg(const uint16_t* w, int n, int o, const float* x, const float* norm_w, float eps,
                            float* out, hipStream_t s, const F16Qkv& qa = F16Qkv{}) {
    const size_t lds = fg_lds_floats(n, PRO, R) * sizeof(float);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    auto k = k_f16_gemv<PRO, EPI, R>;
    static bool raised = false;
    if (lds > 65536 && !raised) {
        const hipError_t e =
            hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        raised = true;
    }
    hipLaunchKernelGGL(k, dim3((o + R - 1) / R), dim3(FgShape<R>::threads), lds, s, w, n, o, x, norm_w, eps, out,
                       wait_fault_word(false), qa);
    return hipGetLastError();
}

// rows per workgroup: the fewest of 8, 16, 32, 64 that keep the grid within
// one workgroup per CU (a second chain wavefront on a CU can share a SIMD
// with the first and halve both)
template <int PRO, int EPI>
static hipError_t launch_fg_rows(const uint16_t* w, int n, int o, const float* x, const float* norm_w, float eps,
                                 float* out, hipStream_t s, const F16Qkv& qa = F16Qkv{}) {
    if (o <= 256 * 8) return launch_fg<PRO, EPI, 8>(w, n, o, x, norm_w, eps, out, s, qa);
    if (o <= 256 * 16) return launch_fg<PRO, EPI, 16>(w, n, o, x, norm_w, eps, out, s, qa);
    if (o <= 256 * 32) return launch_fg<PRO, EPI, 32>(w, n, o, x, norm_w, eps, out, s, qa);
    return launch_fg<PRO, EPI, 64>(w, n, o, x, norm_w, eps, out, s, qa);
}

hipError_t launch_f16_gemv(const uint16_t* w, int n, int o, const float* x, const float* norm_w, float eps, int epi,
                           float* out, hipStream_t s, const F16Qkv* qkv) {
    if (n % 32 || n <= 0 || o <= 0 || epi < 0 || epi > 3 || (epi == 2 && o % (2 * kFgPairRows)))
        return hipErrorInvalidValue;
    if (epi == 3) {
        if (!qkv || !norm_w || qkv->hd % 2 || qkv->att % qkv->hd || o != qkv->att + 2 * qkv->kv) return hipErrorInvalidValue;
        return launch_fg_rows<1, 3>(w, n, o, x, norm_w, eps, out, s, *qkv);
    }
    if (epi == 2) {
        if (norm_w) return launch_fg<1, 2, 64>(w, n, o, x, norm_w, eps, out, s);
        return launch_fg<0, 2, 64>(w, n, o, x, norm_w, eps, out, s);
    }
    if (norm_w) {
        if (epi == 0) return launch_fg_rows<1, 0>(w, n, o, x, norm_w, eps, out, s);
        return hipErrorInvalidValue;
    }
    if (epi == 0) return launch_fg_rows<0, 0>(w, n, o, x, norm_w, eps, out, s);
    return launch_fg_rows<0, 1>(w, n, o, x, norm_w, eps, out, s);
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
