// yl_pattn.hip -- attention of prompt batches (forward.rs:299-400), tiled.
//
// A prompt of B >= 64 tokens attends in three kernels that share every K, V
// and score tile among 64 query rows.  The arithmetic is the reference's,
// operation by operation:
//   score[t][t2] = reduce_add8(8 lane partials over head_size) * scale,
//     positions past the row's causal bound t1 = pos + t are -1e10;
//   max from -1e10; e = exp(score - max); sum_exp serial over all seq_len
//     positions (masked ones add exp(-1e10 - max), zero unless every score
//     of the row is at or below -1e10); p = e * (1 / sum_exp);
//   out[t][d] = reduce_add8(lane j sums p * v over t2 = 8c + j in c order)
//     + the seq_len % 8 tail in t2 order.
//
// 1. k_pattn_scores: workgroup (position tile, row tile, head) computes the
//    64 x 64 scores with 4 x 4 register tiles, one lane partial j at a time
//    (folded in reduce_add8's order), and the tile's row maxima.
// 2. k_pattn_expsum: workgroup (head, row tile): e = exp(score - max) in
//    place, chunk by chunk, while one wavefront adds each chunk to its rows'
//    serial denominators in position order; then inv = 1 / sum and the
//    masked p.
// 3. k_pattn_pv: workgroup (head, row tile) chains p * v for its 64 rows and
//    every dimension (4 rows x 4 dimensions x 8 lane chains per thread),
//    then the 32-group quantization of the output projection's input.
// Scores live in a scratch [head][position][row] (rows contiguous, so a
// wavefront reading one position of 64 rows reads 256 contiguous bytes).
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

constexpr int kPT = 64;         // rows (and positions) per tile
constexpr int kPTS = kPT + 4;   // LDS row stride of a 64-wide tile (16-byte aligned, banks spread)
constexpr int kBufRawP = 0x00020000;

__host__ __device__ inline int pattn_rows_ld(int batch) { return (batch + kPT - 1) / kPT * kPT; }
__host__ __device__ inline int pattn_tiles(int seq) { return (seq + kPT - 1) / kPT; }

// Scratch: scores [n_heads][seq_ld][Bp], tile maxima [n_heads][tiles][Bp],
// then per row: max, 1/sum, masked p ([n_heads][Bp] each).
struct PromptScratch {
    float *sc, *tm, *mx, *inv, *pm;
};
__host__ __device__ inline PromptScratch pattn_carve(float* base, int n_heads, int seq_ld, int batch) {
    const size_t Bp = pattn_rows_ld(batch);
    PromptScratch p;
    p.sc = base;
    p.tm = p.sc + (size_t)n_heads * seq_ld * Bp;
    p.mx = p.tm + (size_t)n_heads * pattn_tiles(seq_ld) * Bp;
    p.inv = p.mx + (size_t)n_heads * Bp;
    p.pm = p.inv + (size_t)n_heads * Bp;
    return p;
}
size_t prompt_attn_bytes(int n_heads, int seq_ld, int batch) {
    const size_t Bp = pattn_rows_ld(batch);
    return (size_t)n_heads * Bp * ((size_t)seq_ld + pattn_tiles(seq_ld) + 3) * sizeof(float);
}
// k_attention (one workgroup per head and token) holds the whole score row
// in LDS; batches of 2..63 tokens whose seq_len does not fit take the tiled
// path as one partial row tile
bool prompt_attn_applies(int batch, int seq_len, int head_size) {
    return batch >= kPT || (batch > 1 && !attention_row_fits(seq_len, head_size));
}

// ---------------------------------------------------------------------------
// 1. scores and tile row maxima.  Workgroup (head, row tile, segment): the
//    segment's position tiles (at most kScSeg of the row tile's causal ones)
//    in order, the Q tile loaded once, the next K tile's loads in flight
//    while the current one is computed.  Thread (ty, tx) of 16 x 16: rows
//    4ty..+3, positions 4tx..+3 of the tile.  Lane partial j (dimensions
//    8s + j, s in order) of all 16 scores, then folded:
//    a = ((l0 + l1) + l2) + l3, b = ((l4 + l5) + l6) + l7,
//    score = (a + b) * scale.  Grid (x only): heads fastest, then segments,
//    then row tiles from the last (the longest).
// ---------------------------------------------------------------------------
constexpr int kScSeg = 8;   // position tiles per workgroup at most
__host__ __device__ inline int pattn_score_segs(int seq_ld) { return (pattn_tiles(seq_ld) + kScSeg - 1) / kScSeg; }

template <int HD>
__global__ __launch_bounds__(256) void k_pattn_scores(const float* __restrict__ sq, const float* __restrict__ kc,
                                                      const StepState* __restrict__ st, int batch, int seq_ld,
                                                      int kv_ld, int n_heads, int n_kv_heads, float scale,
                                                      float* __restrict__ scratch) {
    __shared__ __align__(16) float qT[HD * kPTS];   // [dim][row]
    __shared__ __align__(16) float kT[HD * kPTS];   // [dim][position]
    const int nseg = pattn_score_segs(seq_ld);
    const int tid = threadIdx.x, h = (int)(blockIdx.x % n_heads), ys = (int)(blockIdx.x / n_heads);
    const int rt = pattn_tiles(batch) - 1 - ys / nseg, seg = ys % nseg;
    const int pos0 = st->pos, seq = pos0 + batch;
    const int row0 = rt * kPT;
    if (seq > seq_ld) return;
    // position tiles holding a causal position of some row of the tile
    const int last_pt = min(pos0 + row0 + kPT - 1, seq - 1) / kPT;
    const int pt0 = seg * kScSeg, pt1 = min(pt0 + kScSeg - 1, last_pt);
    if (pt0 > pt1) return;
    const PromptScratch S = pattn_carve(scratch, n_heads, seq_ld, batch);
    const int Bp = pattn_rows_ld(batch);
    const int kvh = h / (n_heads / n_kv_heads), att_dim = n_heads * HD;
    // q rows as 16-byte pieces and key quads: dimension d of position p at
    // kc[(kvh*HD + d) * kv_ld + p]; quads past the row (kv_ld is a multiple
    // of 4) re-read its last quad (positions past seq are never stored)
    constexpr int NV = HD / 16;   // 16-byte pieces per thread, q and keys each
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(kc + (size_t)kvh * HD * kv_ld), (short)0, HD * kv_ld * 4, kBufRawP);
    vf4 ka[NV];
    auto load_k = [&](int pt) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = tid + 256 * i, d = idx / (kPT / 4), q4 = idx % (kPT / 4);
            const int p = min(pt * kPT + 4 * q4, kv_ld - 4);
            ka[i] = __builtin_bit_cast(vf4, __builtin_amdgcn_raw_buffer_load_b128(krs, p * 4, d * kv_ld * 4, 0));
        }
    };
    // keys transposed
    auto store_k = [&]() {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = tid + 256 * i, d = idx / (kPT / 4), q4 = idx % (kPT / 4);
            *reinterpret_cast<vf4*>(kT + d * kPTS + 4 * q4) = ka[i];
        }
    };
    {
        // (q pieces: consecutive lanes take consecutive rows, so the
        // transposed LDS stores below hit consecutive banks)
        vf4 qa[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = tid + 256 * i, r = idx % kPT, d4 = idx / kPT;
            qa[i] = *reinterpret_cast<const vf4*>(sq + (size_t)min(row0 + r, batch - 1) * att_dim + (size_t)h * HD + 4 * d4);
        }
        load_k(pt0);
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = tid + 256 * i, r = idx % kPT, d4 = idx / kPT;
            const bool live = row0 + r < batch;
#pragma unroll
            for (int c = 0; c < 4; c++) qT[(4 * d4 + c) * kPTS + r] = live ? qa[i][c] : 0.0f;
        }
        store_k();
    }
    __syncthreads();
    const int ty = tid >> 4, tx = tid & 15;
    float A[4][4], Bh[4][4], l[4][4];
    // lane partial j of the 4 x 4 pairs.  The reference's lane sums start
    // from 0.0; these start from the first product, which differs only in
    // a zero's sign (0 + -0 = +0).  A score is only ever used as
    // exp(score - max) (and in the max), where +-0 - m = -m for m != 0 and
    // exp(+-0) = 1, so no result depends on that sign.
    auto partial = [&](int j) {
#pragma unroll
        for (int s = 0; s < HD / 8; s++) {
            const vf4 qv = *reinterpret_cast<const vf4*>(qT + (8 * s + j) * kPTS + 4 * ty);
            const vf4 kv = *reinterpret_cast<const vf4*>(kT + (8 * s + j) * kPTS + 4 * tx);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) l[a][b] = s == 0 ? fmul(qv[a], kv[b]) : fadd(l[a][b], fmul(qv[a], kv[b]));
        }
    };
    for (int pt = pt0; pt <= pt1; pt++) {
        if (pt < pt1) load_k(pt + 1);   // in flight while this tile is computed
        const int p0 = pt * kPT;
        // reduce_add8: A = ((l0 + l1) + l2) + l3, Bh = ((l4 + l5) + l6) + l7.
        // One partial at a time (unrolled, the compiler would hoist every
        // partial's LDS reads and run out of registers); each fold is a loop
        // of its own so that no per-element branch on j remains.
        partial(0);
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) A[a][b] = l[a][b];
#pragma unroll 1
        for (int j = 1; j < 4; j++) {
            partial(j);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) A[a][b] = fadd(A[a][b], l[a][b]);
        }
        partial(4);
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) Bh[a][b] = l[a][b];
#pragma unroll 1
        for (int j = 5; j < 8; j++) {
            partial(j);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) Bh[a][b] = fadd(Bh[a][b], l[a][b]);
        }
        float rmax[4] = {-1e10f, -1e10f, -1e10f, -1e10f};
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int p = p0 + 4 * tx + b;
            float v[4];
#pragma unroll
            for (int a = 0; a < 4; a++) {
                v[a] = fmul(fadd(A[a][b], Bh[a][b]), scale);
                if (p <= pos0 + row0 + 4 * ty + a) rmax[a] = fmaxf(rmax[a], v[a]);
            }
            if (p < seq)
                *reinterpret_cast<vf4*>(S.sc + ((size_t)h * seq_ld + p) * Bp + row0 + 4 * ty) = vf4{v[0], v[1], v[2], v[3]};
        }
        // row maxima over the 16 threads of a row group (tx = the low 4 bits)
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) rmax[a] = fmaxf(rmax[a], __shfl_xor(rmax[a], off, 16));
        if (tx == 0)
#pragma unroll
            for (int a = 0; a < 4; a++) S.tm[((size_t)h * pattn_tiles(seq_ld) + pt) * Bp + row0 + 4 * ty + a] = rmax[a];
        if (pt < pt1) {
            __syncthreads();   // every wavefront is done with this K tile
            store_k();
            __syncthreads();   // the next one is in LDS
        }
    }
}

// ---------------------------------------------------------------------------
// 2. exponentials and serial denominators, workgroup (head, row tile).  The
//    row max folds the tile maxima from -1e10.  Then, chunk by chunk of 64
//    positions up to the tile's causal bound, every thread computes 4
//    positions x 4 rows of e = exp(score - max), written back in place (for
//    P.V) and into an LDS tile, and wavefront 0 (lane r: row r) adds the
//    chunk's causal e to its rows' sums in position order while the other
//    wavefronts go on to the next chunk (two LDS tiles alternate; the next
//    chunk's scores are loaded while the current one is computed).  Last,
//    the masked positions' exp(-1e10 - max), inv = 1 / sum and the masked p.
//    Row tiles run longest first (heads fastest), as in P.V.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pattn_expsum(const StepState* __restrict__ st, int batch, int seq_ld,
                                                      int n_heads, float* __restrict__ scratch) {
    __shared__ float mxl[kPT];
    __shared__ __align__(16) float eT[2][kPT * kPTS];   // [position][row]
    const int h = blockIdx.x, rt = gridDim.y - 1 - blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int pos0 = st->pos, seq = pos0 + batch;
    if (seq > seq_ld) return;
    const PromptScratch S = pattn_carve(scratch, n_heads, seq_ld, batch);
    const int Bp = pattn_rows_ld(batch), ntl = pattn_tiles(seq_ld);
    const int row0 = rt * kPT;
    {
        // row r = tid % 64 folds tile maxima q = tid / 64 + 4k (loads issued
        // 8 at a time), then the 4 partial maxima meet in LDS
        __shared__ float mxp[4][kPT];
        const int r = lane, part = wave, t = row0 + r;
        const int last = min(pos0 + t, seq - 1) / kPT;
        const float* tmr = S.tm + (size_t)h * ntl * Bp + t;
        float mx = -1e10f;
        for (int q0 = part; q0 <= last; q0 += 32) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = tmr[(size_t)min(q0 + 4 * k, last) * Bp];
#pragma unroll
            for (int k = 0; k < 8; k++) mx = fmaxf(mx, v[k]);
        }
        mxp[part][r] = mx;
        __syncthreads();
        if (tid < kPT) {
            mx = fmaxf(fmaxf(mxp[0][tid], mxp[1][tid]), fmaxf(mxp[2][tid], mxp[3][tid]));
            mxl[tid] = mx;
            S.mx[(size_t)h * Bp + row0 + tid] = mx;
        }
        __syncthreads();
    }
    const int bound = min(seq, pos0 + row0 + kPT);   // positions < bound: every row's causal part
    const int nq = (bound + kPT - 1) / kPT;
    const ExpfK ek = expf_k_regs();   // 16 exponentials per thread and chunk
    // 4 positions x 4 consecutive rows per thread, as 16-byte accesses:
    // position pp = tid / 16 + 16k of the chunk, rows 4 * (tid % 16) + 0..3
    const int r4 = 4 * (tid & 15), tr = row0 + r4;
    float mr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) mr[i] = mxl[r4 + i];
    float* sch = S.sc + (size_t)h * seq_ld * Bp + row0 + r4;
    vf4 v[4];
    auto load = [&](int q0) {
#pragma unroll
        for (int k = 0; k < 4; k++)
            v[k] = *reinterpret_cast<const vf4*>(sch + (size_t)min(q0 + (tid >> 4) + 16 * k, seq - 1) * Bp);
    };
    const int t1 = pos0 + row0 + lane;   // wavefront 0: lane's row's last causal position
    float sum = 0.0f;
    load(0);
    for (int c = 0; c < nq; c++) {
        const int q0 = c * kPT;
        float* et = eT[c & 1];
        vf4 e[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) e[k][i] = expf_rn(v[k][i] - mr[i], ek);
        if (c + 1 < nq) load(q0 + kPT);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int pp = (tid >> 4) + 16 * k, p = q0 + pp;
            *reinterpret_cast<vf4*>(et + pp * kPTS + r4) = e[k];
            float* dst = sch + (size_t)p * Bp;
            // live: p < seq, row < batch and p <= pos0 + row (rising with the row)
            if (p < seq && tr + 3 < batch && p <= pos0 + tr) {
                *reinterpret_cast<vf4*>(dst) = e[k];
            } else if (p < seq) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (tr + i < batch && p <= pos0 + tr + i) dst[i] = e[k][i];
            }
        }
        __syncthreads();   // the chunk's tile is complete; eT[c & 1] is next written after the next barrier
        if (wave == 0) {
            // the row's causal e of this chunk in position order, read 16 at a time
#pragma unroll
            for (int g = 0; g < kPT; g += 16) {
                float ev[16];
#pragma unroll
                for (int i = 0; i < 16; i++) ev[i] = et[(g + i) * kPTS + lane];
#pragma unroll
                for (int i = 0; i < 16; i++)
                    if (q0 + g + i <= t1) sum = fadd(sum, ev[i]);
            }
        }
    }
    if (wave != 0) return;
    const int t = row0 + lane;
    if (t >= batch) return;
    // masked positions t1+1 .. seq-1 add exp(-1e10 - max) each
    const float em = t1 < seq - 1 ? expf_rn(-1e10f - mxl[lane], ek) : 0.0f;
    if (em != 0.0f)
        for (int i = t1 + 1; i < seq; i++) sum = fadd(sum, em);
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    S.inv[(size_t)h * Bp + t] = inv;
    S.pm[(size_t)h * Bp + t] = fmul(em, inv);
}

// ---------------------------------------------------------------------------
// 3. P.V chains and the output.  Thread (ty, tx): rows 4ty..+3, dimensions
//    4tx..+3, 8 lane chains each (acc[row][dim][j] += p * v over t2 = 8c + j,
//    c in order).  Positions run to the tile's causal bound (the last row's
//    t1) unless a row's masked p is nonzero or the V rows past the bound hold
//    an infinity or NaN (0 * v would then not vanish): masked positions add
//    p * v = +-0 to a partial that starts at +0, which changes nothing.
// ---------------------------------------------------------------------------
template <int QF, int HD>
__global__ __launch_bounds__(HD * 4) void k_pattn_pv(const float* __restrict__ vc, const StepState* __restrict__ st,
                                                     int batch, int seq_ld, int n_heads, int n_kv_heads,
                                                     float* __restrict__ scratch, int8_t* __restrict__ aq,
                                                     float* __restrict__ as, float* __restrict__ att_f32) {
    constexpr int NT = HD * 4, NX = HD / 4;   // threads; dimension groups
    constexpr int VS = HD + 4;                // LDS row stride of a V tile
    __shared__ __align__(16) float pT[kPT * kPTS];   // [position][row]
    __shared__ __align__(16) float vT[kPT * VS];     // [position][dim]
    __shared__ float invl[kPT], pml[kPT];
    __shared__ int full_sh;
    // a row tile's work grows with its causal bound: the grid runs heads
    // fastest and row tiles from the last, so the longest workgroups are
    // dispatched first and the short ones fill the slots they leave
    const int h = blockIdx.x, rt = gridDim.y - 1 - blockIdx.y, tid = threadIdx.x;
    const int pos0 = st->pos, seq = pos0 + batch;
    if (seq > seq_ld) return;
    const PromptScratch S = pattn_carve(scratch, n_heads, seq_ld, batch);
    const int Bp = pattn_rows_ld(batch);
    const int kvh = h / (n_heads / n_kv_heads), kv_dim = n_kv_heads * HD, att_dim = n_heads * HD;
    const int row0 = rt * kPT;
    const int n_chunks = seq / 8;
    const int bound = min(seq, pos0 + row0 + kPT);   // positions < bound hold every row's causal part
    if (tid == 0) full_sh = 0;
    __syncthreads();
    bool full = false;
    if (tid < kPT) {
        const int t = row0 + tid;
        invl[tid] = t < batch ? S.inv[(size_t)h * Bp + t] : 0.0f;
        pml[tid] = t < batch ? S.pm[(size_t)h * Bp + t] : 0.0f;
        full = pml[tid] != 0.0f;
    }
    // V past the bound (only the chunked part is chained), 16-byte pieces,
    // 8 loads in flight per thread
    const float* vh = vc + (size_t)kvh * HD;
    const int n_scan = max(0, n_chunks * 8 - bound) * NX;
    for (int i0 = tid; i0 < n_scan; i0 += 8 * NT) {
        vf4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = min(i0 + k * NT, n_scan - 1);
            v[k] = *reinterpret_cast<const vf4*>(vh + (size_t)(bound + i / NX) * kv_dim + 4 * (i % NX));
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int c = 0; c < 4; c++) full = full || !(__builtin_fabsf(v[k][c]) <= 3.402823466e38f);
    }
    if (full) atomicOr(&full_sh, 1);
    __syncthreads();
    const int end_c = full_sh ? n_chunks : min(n_chunks, (bound + 7) / 8);

    const int ty = tid / NX, tx = tid % NX;
    float acc[4][4][8];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int j = 0; j < 8; j++) acc[a][b][j] = 0.0f;
    const float* sch = S.sc + (size_t)h * seq_ld * Bp + row0;
    // tiles of 64 positions: the next tile's scores and V rows are loaded
    // into registers while the current tile is chained
    constexpr int SV = kPT * kPT / 4 / NT, VV = kPT * NX / NT;
    vf4 sreg[SV], vreg[VV];
    auto load_tile = [&](int q0) {
#pragma unroll
        for (int i = 0; i < SV; i++) {
            const int idx = tid + NT * i, pp = idx / (kPT / 4), r4 = idx % (kPT / 4);
            sreg[i] = *reinterpret_cast<const vf4*>(sch + (size_t)min(q0 + pp, seq - 1) * Bp + 4 * r4);
        }
#pragma unroll
        for (int i = 0; i < VV; i++) {
            const int idx = tid + NT * i, pp = idx / NX, d4 = idx % NX;
            vreg[i] = *reinterpret_cast<const vf4*>(vh + (size_t)min(q0 + pp, seq - 1) * kv_dim + 4 * d4);
        }
    };
    // p = e * inv on the causal entries, the row's masked p elsewhere
    auto store_tile = [&](int q0) {
#pragma unroll
        for (int i = 0; i < SV; i++) {
            const int idx = tid + NT * i, pp = idx / (kPT / 4), r4 = idx % (kPT / 4);
            float pv[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int r = 4 * r4 + c;
                pv[c] = q0 + pp <= pos0 + row0 + r ? fmul(sreg[i][c], invl[r]) : pml[r];
            }
            *reinterpret_cast<vf4*>(pT + pp * kPTS + 4 * r4) = vf4{pv[0], pv[1], pv[2], pv[3]};
        }
#pragma unroll
        for (int i = 0; i < VV; i++) {
            const int idx = tid + NT * i, pp = idx / NX, d4 = idx % NX;
            *reinterpret_cast<vf4*>(vT + pp * VS + 4 * d4) = vreg[i];
        }
    };
    if (end_c > 0) load_tile(0);
    for (int q0 = 0; q0 < 8 * end_c; q0 += kPT) {
        store_tile(q0);
        lds_barrier();   // (the next tile's loads, issued below, stay in flight across both barriers)
        if (q0 + kPT < 8 * end_c) load_tile(q0 + kPT);
        const int nc = min(kPT / 8, end_c - q0 / 8);
        for (int c = 0; c < nc; c++) {
            // lane j's p and V reads alternate between two register sets, so
            // that lane j + 1's reads are in flight while lane j's 32 ops run
            auto rd = [&](int j, vf4& pv, vf4& vv) {
                pv = *reinterpret_cast<const vf4*>(pT + (8 * c + j) * kPTS + 4 * ty);
                vv = *reinterpret_cast<const vf4*>(vT + (8 * c + j) * VS + 4 * tx);
            };
            auto step = [&](int j, const vf4& pv, const vf4& vv) {
#pragma unroll
                for (int a = 0; a < 4; a++)
#pragma unroll
                    for (int b = 0; b < 4; b++) acc[a][b][j] = fadd(acc[a][b][j], fmul(pv[a], vv[b]));
            };
            vf4 p0, v0, p1, v1;
            rd(0, p0, v0);
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                rd(j + 1, p1, v1);
                __builtin_amdgcn_sched_barrier(0);
                step(j, p0, v0);
                __builtin_amdgcn_sched_barrier(0);
                if (j + 2 < 8) rd(j + 2, p0, v0);
                __builtin_amdgcn_sched_barrier(0);
                step(j + 1, p1, v1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        lds_barrier();
    }
    // out = reduce_add8 + the seq % 8 tail in order, then the 32-groups
    // (8 threads of consecutive tx hold one group of a row)
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int r = 4 * ty + a, t = row0 + r;
        const int tcl = min(t, batch - 1);
        float o[4];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            o[b] = reduce_add8(acc[a][b]);
            for (int t2 = n_chunks * 8; t2 < seq; t2++) {
                const float p = t2 <= pos0 + tcl ? fmul(sch[(size_t)t2 * Bp + r], invl[r]) : pml[r];
                o[b] = fadd(o[b], fmul(p, vh[(size_t)t2 * kv_dim + 4 * tx + b]));
            }
        }
        const size_t col = (size_t)t * att_dim + (size_t)h * HD + 4 * tx;
        if (t < batch && att_f32)
#pragma unroll
            for (int b = 0; b < 4; b++) att_f32[col + b] = o[b];
        if constexpr (QF >= 0) {
            float am = 0.0f;
#pragma unroll
            for (int b = 0; b < 4; b++) am = fmaxf(am, fabsf(o[b]));
#pragma unroll
            for (int off = 1; off < 8; off <<= 1) am = fmaxf(am, __shfl_xor(am, off, 8));
            const float s = group_scale<QF>(am);
            if (t < batch) {
#pragma unroll
                for (int b = 0; b < 4; b++) aq[col + b] = (int8_t)quant_one<QF>(o[b], s);
                if ((tx & 7) == 0) as[col / kGroup] = s;
            }
        }
    }
}

template <int QF, int HD>
static hipError_t launch_pattn_hd(const float* sq, const float* kc, const float* vc, const StepState* st, int batch,
                                  int seq_ld, int kv_ld, int n_heads, int n_kv_heads, float scale, int8_t* aq,
                                  float* as, float* att_f32, float* scratch, hipStream_t s) {
    const dim3 tiles((unsigned)n_heads * pattn_tiles(batch) * pattn_score_segs(seq_ld));
    hipLaunchKernelGGL((k_pattn_scores<HD>), tiles, dim3(256), 0, s, sq, kc, st, batch, seq_ld, kv_ld, n_heads,
                       n_kv_heads, scale, scratch);
    hipLaunchKernelGGL(k_pattn_expsum, dim3(n_heads, pattn_tiles(batch)), dim3(256), 0, s, st, batch, seq_ld, n_heads,
                       scratch);
    hipLaunchKernelGGL((k_pattn_pv<QF, HD>), dim3(n_heads, pattn_tiles(batch)), dim3(HD * 4), 0, s, vc, st, batch,
                       seq_ld, n_heads, n_kv_heads, scratch, aq, as, att_f32);
    return hipGetLastError();
}

template <int QF>
static hipError_t launch_pattn_q(const float* sq, const float* kc, const float* vc, const StepState* st, int batch,
                                 int seq_ld, int kv_ld, int n_heads, int n_kv_heads, int hd, float scale, int8_t* aq,
                                 float* as, float* att_f32, float* scratch, hipStream_t s) {
    switch (hd) {
    case 32: return launch_pattn_hd<QF, 32>(sq, kc, vc, st, batch, seq_ld, kv_ld, n_heads, n_kv_heads, scale, aq, as, att_f32, scratch, s);
    case 64: return launch_pattn_hd<QF, 64>(sq, kc, vc, st, batch, seq_ld, kv_ld, n_heads, n_kv_heads, scale, aq, as, att_f32, scratch, s);
    case 128: return launch_pattn_hd<QF, 128>(sq, kc, vc, st, batch, seq_ld, kv_ld, n_heads, n_kv_heads, scale, aq, as, att_f32, scratch, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_prompt_attention(const float* sq, const float* kc, const float* vc, const StepState* st, int batch,
                                   int seq_ld, int kv_ld, int n_heads, int n_kv_heads, int head_size, float scale,
                                   int qfmt, int8_t* aq, float* as, float* att_f32, float* scratch, hipStream_t s) {
    if (!scratch || batch < 2 || seq_ld < batch || kv_ld < seq_ld || kv_ld % 4) return hipErrorInvalidValue;
    if (qfmt == kQ8)
        return launch_pattn_q<kQ8>(sq, kc, vc, st, batch, seq_ld, kv_ld, n_heads, n_kv_heads, head_size, scale, aq,
                                   as, att_f32, scratch, s);
    if (qfmt == kQ4)
        return launch_pattn_q<kQ4>(sq, kc, vc, st, batch, seq_ld, kv_ld, n_heads, n_kv_heads, head_size, scale, aq,
                                   as, att_f32, scratch, s);
    return launch_pattn_q<-1>(sq, kc, vc, st, batch, seq_ld, kv_ld, n_heads, n_kv_heads, head_size, scale, aq, as,
                              att_f32, scratch, s);
}

}  // namespace yl
