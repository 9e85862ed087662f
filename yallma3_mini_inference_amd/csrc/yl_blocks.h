// yl_blocks.h -- workgroup-level building blocks shared by the kernels.
#pragma once

#include "yl_device.h"

namespace yl {

// Position of element i inside the activation staging buffer of a Q4_0
// matmul: each 8-group is stored as its 4 even elements then its 4 odd ones,
// matching the low/high nibbles of one weight dword.
__device__ __forceinline__ int q4_pos(int i) {
    const int k = i & 7;
    return (i & ~7) | ((k & 1) ? 4 + (k >> 1) : (k >> 1));
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// ---------------------------------------------------------------------------
// General RMSNorm (+ quantize) of one row of any length, for the standalone
// rmsnorm entry point (util.rs:389-426: elements past the last whole 8-group
// are neither summed nor written).
//
// Row stride (floats) of the transposed layout: lane chain j of the f32x8
// accumulator reads its elements x[8i+j] contiguously at xt[j*S + i].  S is a
// multiple of 4 (float4 reads) and S % 32 == 4, 12, 20 or 28, so the 8 chain
// lanes hit distinct LDS banks.
__host__ __device__ inline int norm_stride(int dim) { return (((dim / 8) + 3) & ~3) + 4; }
// transposed row 8*S | reduction 16 | norm weights dim
__host__ __device__ inline size_t norm_lds_floats(int dim) { return (size_t)8 * norm_stride(dim) + 16 + dim; }

// Stores element i of the row (v) and of the norm weight (w) for the block.
__device__ __forceinline__ void store_norm_input(float* xt, int dim, int i, float v, float w) {
    const int n8 = (dim / 8) * 8;
    const int S = norm_stride(dim);
    if (i < n8) xt[(i & 7) * S + (i >> 3)] = v;
    xt[8 * S + 16 + i] = w;
}

//   xt  : LDS, norm_lds_floats(dim), filled by store_norm_input()
//   QF  : kQ8 / kQ4 -> q_lds/s_lds receive the quantized row (Q4 reordered
//         when PERM); QF < 0 -> no quantization.
//   xn  : optional f32 output of the normalized row (global or LDS).
// The 8 lane sums run as 8 serial chains (one lane each) over float4 reads;
// normalization and quantization use one element per thread, a 32-group per
// half-wave (absmax by shuffles: order-free max).
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
            // (DPP within 16-lane rows, one shuffle across them; the max of
            // absolute values is order-free)
            float am = group_max(fabsf(v), 32);
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

// ---------------------------------------------------------------------------
// RMSNorm + quantize of one row inside a fused kernel (dim % 32 == 0).
//
// A team of threads -- the whole workgroup, or one wavefront -- walks the row
// in passes; in pass p team member i holds the 8 elements from
// e = (p * team_size + i) * 8, so each 32-group belongs to an aligned quad of
// lanes and its absmax takes two DPP steps.  Members past the row load a
// clamped copy of the last slice and write nothing; they form whole quads.
//
// Sum of squares: the reference's f32x8 accumulator is 8 serial chains (lane
// j adds x[8i+j]^2 for i = 0, 1, ...; util.rs:398-405).  The squares go to LDS
// transposed (row j holds chain j), and lanes 0-7 of every wavefront of the
// team run the 8 chains over float4 reads kept in flight a block ahead; each
// wavefront reads the 8 results by readlane.
//
// The chains need no workgroup barrier when one wavefront staged the row
// (the LDS operations of one wavefront complete in issue order), so in a
// GEMV that wavefront runs them while the others issue weight loads: a
// workgroup barrier completes only once every wavefront has issued all its
// loads, which under full HBM load is most of the kernel's duration.
//
// Use: rowq_load_* issue the global loads into registers; rowq_stage moves
// the row, the norm weights and the squares to LDS (freeing the registers for
// the chain loop); rowq_chain yields the reciprocal RMS; rowq_quant
// normalizes and quantizes.
struct RowTeam {
    int idx, size;   // member index, member count (a multiple of 64)
};
__device__ __forceinline__ RowTeam team_workgroup() { return RowTeam{(int)threadIdx.x, (int)blockDim.x}; }
__device__ __forceinline__ RowTeam team_wave() { return RowTeam{(int)(threadIdx.x & 63), 64}; }

__host__ __device__ inline int rowq_passes(int dim, int team) { return (dim + 8 * team - 1) / (8 * team); }
// Chain row length: dim/8 squares padded with zeros to a multiple of 64
// (pairs of 8-vf4 read blocks; adding +0 to a sum of squares is exact), and
// a stride of that + 4 floats so the 8 chain lanes read distinct banks.
__host__ __device__ inline int rowq_chain_len(int dim) { return ((dim / 8) + 63) & ~63; }
__host__ __device__ inline int rowq_stride(int dim) { return rowq_chain_len(dim) + 4; }
// Row and norm-weight regions: dim floats rounded up to whole 1 KiB DMA rows.
__host__ __device__ inline int rowq_row_len(int dim) { return (dim + 255) & ~255; }
// LDS floats used: transposed squares | row | norm weights
__host__ __device__ inline size_t rowq_lds_floats(int dim) {
    return (size_t)8 * rowq_stride(dim) + 2 * (size_t)rowq_row_len(dim);
}

// first element of the member's slice in pass p (clamped past the row)
__device__ __forceinline__ int rowq_elem(RowTeam tm, int p, int dim) {
    const int e = (p * tm.size + tm.idx) * 8;
    return e < dim ? e : dim - 8;
}
__device__ __forceinline__ bool rowq_live(RowTeam tm, int p, int dim) { return (p * tm.size + tm.idx) * 8 < dim; }

// f32 slices of src -> registers, two vf4 per pass (issue only)
template <int MP>
__device__ __forceinline__ void rowq_load_f32(RowTeam tm, vf4 (&dst)[2 * MP], const float* __restrict__ src,
                                              int dim, int passes) {
#pragma unroll
    for (int p = 0; p < MP; p++)
        if (p < passes) {
            const vf4* s4 = reinterpret_cast<const vf4*>(src + rowq_elem(tm, p, dim));
            dst[2 * p] = s4[0];
            dst[2 * p + 1] = s4[1];
        }
}

// Raw bytes + scale of one token's row slices in the interleaved Q8_0
// embedding (bytes q+128 at [vocab/64][dim/16][64][16], f16 scales at
// [vocab/64][dim/32][64]).  Ids outside the vocabulary read row 0; their
// values are zeroed by rowq_embed_values.
template <int MP>
struct EmbRegs {
    uint2 q[MP];
    uint16_t d[MP];
};
template <int MP>
__device__ __forceinline__ void rowq_load_emb(RowTeam tm, EmbRegs<MP>& r, const EmbQ8& e, uint32_t tok,
                                              int passes) {
    const bool in_vocab = tok < (uint32_t)e.vocab;
    const size_t tile = in_vocab ? tok >> 6 : 0;
    const int lane = (int)(tok & 63u);
    const uint8_t* q = reinterpret_cast<const uint8_t*>(e.q);
#pragma unroll
    for (int p = 0; p < MP; p++)
        if (p < passes) {
            const int el = rowq_elem(tm, p, e.dim);
            r.q[p] = *reinterpret_cast<const uint2*>(q + emb_q_off(e.tiles, tile, el >> 4, lane) + (el & 15));
            r.d[p] = e.d[emb_d_idx(e.tiles, tile, el >> 5, lane)];
        }
}
// Embedding values q*scale (transformer_llama_gguf.rs:459-473), zero for ids
// outside the vocabulary (base_transformer.rs:143-161)
template <int MP>
__device__ __forceinline__ void rowq_embed_values(vf4 (&dst)[2 * MP], const EmbRegs<MP>& r, bool in_vocab,
                                                  int passes) {
#pragma unroll
    for (int p = 0; p < MP; p++)
        if (p < passes) {
            const float sc = f16_to_f32(r.d[p]);
            float v[8];
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint32_t w = b < 4 ? r.q[p].x : r.q[p].y;
                const int u = (int)((w >> (8 * (b & 3))) & 0xffu);
                v[b] = in_vocab ? fmul((float)(u - 128), sc) : 0.0f;
            }
            dst[2 * p] = vf4{v[0], v[1], v[2], v[3]};
            dst[2 * p + 1] = vf4{v[4], v[5], v[6], v[7]};
        }
}

// Row, norm weights and squares -> LDS (sq: rowq_lds_floats(dim) floats).
template <int MP>
__device__ __forceinline__ void rowq_stage(RowTeam tm, const vf4 (&x)[2 * MP], const vf4 (&w)[2 * MP],
                                           int dim, int passes, float* sq) {
    const int S = rowq_stride(dim);
    float* xl = sq + 8 * S;
    float* wl = xl + rowq_row_len(dim);
#pragma unroll
    for (int p = 0; p < MP; p++)
        if (p < passes && rowq_live(tm, p, dim)) {
            const int e = rowq_elem(tm, p, dim);
            const int i = e >> 3;
            const vf4 a = x[2 * p], b = x[2 * p + 1];
            sq[0 * S + i] = fmul(a.x, a.x);
            sq[1 * S + i] = fmul(a.y, a.y);
            sq[2 * S + i] = fmul(a.z, a.z);
            sq[3 * S + i] = fmul(a.w, a.w);
            sq[4 * S + i] = fmul(b.x, b.x);
            sq[5 * S + i] = fmul(b.y, b.y);
            sq[6 * S + i] = fmul(b.z, b.z);
            sq[7 * S + i] = fmul(b.w, b.w);
            *reinterpret_cast<vf4*>(xl + e) = a;
            *reinterpret_cast<vf4*>(xl + e + 4) = b;
            *reinterpret_cast<vf4*>(wl + e) = w[2 * p];
            *reinterpret_cast<vf4*>(wl + e + 4) = w[2 * p + 1];
        }
    const int n8 = dim / 8, pad = rowq_chain_len(dim) - n8;
    for (int i = tm.idx; i < 8 * pad; i += tm.size) sq[(i / pad) * S + n8 + i % pad] = 0.0f;
}

// Staging by one wavefront through LDS DMA (global_load_lds_dwordx4: 16
// bytes per lane straight into LDS, no registers).  Lanes past the row
// re-read its last 16 bytes into the padding of the 1 KiB-rounded region.
// The caller waits for the copies (wait_vm_all) before reading them.
__device__ __forceinline__ void rowq_dma_f32(float* dst, const float* __restrict__ src, int dim) {
    const int lane = threadIdx.x & 63;
    for (int j = 0; j * 256 < dim; j++) {
        const int e = min(j * 256 + lane * 4, dim - 4);
        __builtin_amdgcn_global_load_lds(src + e, dst + j * 256, 16, 0, 0);
    }
}
// Waits for every vector-memory load of the calling wavefront, LDS DMA
// included (the compiler does not order LDS reads after DMA writes itself).
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Squares of a row already in LDS (row region of sq) -> transposed chain rows,
// plus the zero padding of the chain rows; one wavefront.
__device__ __forceinline__ void rowq_squares_wave(int dim, float* sq) {
    const RowTeam tm = team_wave();
    const int S = rowq_stride(dim);
    const float* xl = sq + 8 * S;
    const int passes = rowq_passes(dim, 64);
    for (int p = 0; p < passes; p++) {
        if (!rowq_live(tm, p, dim)) break;
        const int e = rowq_elem(tm, p, dim);
        const int i = e >> 3;
        const vf4 a = *reinterpret_cast<const vf4*>(xl + e), b = *reinterpret_cast<const vf4*>(xl + e + 4);
        sq[0 * S + i] = fmul(a.x, a.x);
        sq[1 * S + i] = fmul(a.y, a.y);
        sq[2 * S + i] = fmul(a.z, a.z);
        sq[3 * S + i] = fmul(a.w, a.w);
        sq[4 * S + i] = fmul(b.x, b.x);
        sq[5 * S + i] = fmul(b.y, b.y);
        sq[6 * S + i] = fmul(b.z, b.z);
        sq[7 * S + i] = fmul(b.w, b.w);
    }
    const int n8 = dim / 8, pad = rowq_chain_len(dim) - n8;
    for (int i = tm.idx; i < 8 * pad; i += 64) sq[(i / pad) * S + n8 + i % pad] = 0.0f;
}

// acc += every element of nbatch batches of 8 float4s in LDS, in order (a
// serial f32 chain).  Three register batches rotate: each batch's reads are
// issued two batches (64 dependent adds, ~270 cycles) before its adds --
// about the LDS latency of a 16-byte read -- and the scheduling barriers
// keep the reads there.  Reads past the last batch re-read it (unused).
__device__ __forceinline__ void add_batch8(float& acc, const vf4 (&v)[8]) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
        acc = fadd(acc, v[k].x);
        acc = fadd(acc, v[k].y);
        acc = fadd(acc, v[k].z);
        acc = fadd(acc, v[k].w);
    }
}
__device__ __forceinline__ void load_batch8(vf4 (&v)[8], const vf4* t4, int bt, int nbatch) {
    const int b = bt < nbatch ? bt : nbatch - 1;
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = t4[b * 8 + k];
}
__device__ __forceinline__ float lds_serial_sum(const vf4* t4, int nbatch, float acc) {
    if (nbatch <= 0) return acc;
    vf4 v0[8], v1[8], v2[8];
    load_batch8(v0, t4, 0, nbatch);
    load_batch8(v1, t4, 1, nbatch);
    for (int bt = 0; bt < nbatch; bt += 3) {
        load_batch8(v2, t4, bt + 2, nbatch);
        __builtin_amdgcn_sched_barrier(0);
        add_batch8(acc, v0);
        if (bt + 1 >= nbatch) break;
        load_batch8(v0, t4, bt + 3, nbatch);
        __builtin_amdgcn_sched_barrier(0);
        add_batch8(acc, v1);
        if (bt + 2 >= nbatch) break;
        load_batch8(v1, t4, bt + 4, nbatch);
        __builtin_amdgcn_sched_barrier(0);
        add_batch8(acc, v2);
    }
    return acc;
}

// RMSNorm (util.rs:389-426) of a staged row, in two parts.
//
// rowq_chain: the sum of squares (the 8 serial chains, run by lanes 0-7 of
// each calling wavefront) -> the reciprocal RMS `ss`, returned to every lane.
// A single wavefront may call it without any workgroup barrier (its own LDS
// writes are complete in issue order).
__device__ __forceinline__ float rowq_chain(int dim, float eps, const float* sq) {
    const int S = rowq_stride(dim);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    float l = 0.0f;
    if ((threadIdx.x & 63) < 8)
        l = lds_serial_sum(reinterpret_cast<const vf4*>(sq + (threadIdx.x & 7) * S), rowq_chain_len(dim) / 32, 0.0f);
    float part[8];
#pragma unroll
    for (int j = 0; j < 8; j++) part[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l), j));
    float ss = reduce_add8(part);
    ss = ss / (float)dim;
    ss = fadd(ss, eps);
    return 1.0f / sqrtf(ss);
}

// rowq_quant: o = w * (ss * x) over the team's slices, then group
// quantization (quantization.rs:29-52 / weight_type.rs:52-74).
//   QF : kQ8 / kQ4 -> q_lds/s_lds (LDS) receive the quantized row, each
//        8-group reordered to (even, odd) elements when PERM; QF < 0 -> none
//   xn : optional f32 output of the normalized row (LDS or global)
template <int QF, bool PERM>
__device__ __forceinline__ void rowq_quant(RowTeam tm, int dim, float ss, const float* sq, int8_t* q_lds,
                                           float* s_lds, float* xn) {
    const int S = rowq_stride(dim);
    const float* xl = sq + 8 * S;
    const float* wl = xl + rowq_row_len(dim);
    const int passes = rowq_passes(dim, tm.size);
    for (int p = 0; p < passes; p++) {
        if (!rowq_live(tm, p, dim)) break;
        const int e = rowq_elem(tm, p, dim);
        const vf4 x0 = *reinterpret_cast<const vf4*>(xl + e), x1 = *reinterpret_cast<const vf4*>(xl + e + 4);
        const vf4 w0 = *reinterpret_cast<const vf4*>(wl + e), w1 = *reinterpret_cast<const vf4*>(wl + e + 4);
        float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float am = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            v[k] = fmul(w[k], fmul(ss, v[k]));
            am = fmaxf(am, fabsf(v[k]));
        }
        if constexpr (QF >= 0) {
            // the quad of this 32-group is live as a whole
            am = fmaxf(am, dpp_mov<0xB1>(am));   // quad_perm [1,0,3,2]
            am = fmaxf(am, dpp_mov<0x4E>(am));   // quad_perm [2,3,0,1]
            const float sc = group_scale<QF>(am);
            int q[8];
            quant8<QF>(v, sc, q);
            *reinterpret_cast<uint2*>(q_lds + e) =
                PERM ? make_uint2(pack4(q[0], q[2], q[4], q[6]), pack4(q[1], q[3], q[5], q[7]))
                     : make_uint2(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]));
            if ((tm.idx & 3) == 0) s_lds[e >> 5] = sc;
        }
        if (xn) {
            *reinterpret_cast<vf4*>(xn + e) = vf4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<vf4*>(xn + e + 4) = vf4{v[4], v[5], v[6], v[7]};
        }
    }
}

// Both parts by the whole workgroup (every wavefront runs the chains);
// starts and ends with a workgroup barrier.
template <int QF, bool PERM>
__device__ void rowq_norm_quant(int dim, float eps, float* sq, int8_t* q_lds, float* s_lds, float* xn) {
    __syncthreads();
    const float ss = rowq_chain(dim, eps, sq);
    rowq_quant<QF, PERM>(team_workgroup(), dim, ss, sq, q_lds, s_lds, xn);
    __syncthreads();
}

// Hand-offs between wavefronts of one workgroup through LDS counters
// (relaxed atomics: a volatile LDS access would make the compiler wait for
// every outstanding global load first).  LDS serves one wavefront's
// accesses in order, and a waiter's reads of the published data are issued
// only after it saw the count.  The waits are bounded: the counted
// wavefronts always arrive within microseconds, the bound only keeps a
// defect from hanging the device; a wait that gives up sets *fault, which the
// host reads after the call and reports as an error.
__device__ __forceinline__ void lds_arrive(int* ctr) {
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wavefront's LDS writes done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// lds_arrive without the wait: LDS performs one wavefront's operations in
// issue order, so a count added after LDS writes is seen only once those
// writes are performed, and a waiter reads the data only after it saw the
// count; the signal fence keeps the compiler from moving the writes past
// the add.  No wait on the wavefront's own outstanding LDS reads either.
__device__ __forceinline__ void lds_arrive_nowait(int* ctr) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Returns the count it saw (>= target unless the wait gave up).
__device__ __forceinline__ int lds_wait_count(int* ctr, int target, unsigned* fault) {
    int i = 0, c;
    for (; (c = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < target && i < (1 << 22); i++)
        __builtin_amdgcn_s_sleep(1);
    if (i == (1 << 22) && fault && (threadIdx.x & 63) == 0)
        __hip_atomic_store(fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return c;
}

// ---------------------------------------------------------------------------
// The serial f32 sum ((0 + v[0]) + v[1]) + ... + v[n-1] (the softmax
// denominator, forward.rs:356-361), bit-identical to the one-at-a-time loop,
// by wavefronts 0..NW-1 of a workgroup in about n / (2 NW) dependent adds
// instead of n.
//
// The row is cut into NS = 2 NW segments of L values (L = 8 * ceil(n / 8NS)).
// Segment i starts from the serial sum of the values before it, known only
// once those are added; so every lane of the wavefront that owns segment i
// runs the serial recurrence over the segment from its own candidate start:
// 64 consecutive f32 values around the float64 sum of the values before the
// segment (the one-at-a-time sum drifts from the exact sum by its rounding
// errors, a random walk of a few ulps at these lengths; candidate 32 is the
// exact sum rounded).  A lane whose start equals the true start bit for bit
// computes the true end.  Wavefront 0 then walks the segments in order:
// segment 0 starts at +0 (candidate 0), and each segment's true end selects
// the next segment's lane.  A true start outside its segment's candidates
// continues one value at a time from there, so the result is the serial sum
// for any input (a NaN or infinity included); only the speed depends on the
// data.  Each wavefront owns segments 2w and 2w+1, two independent chains per
// lane, fed from registers (see the chain below).
//
// v: LDS, holding +0 from n up to 64 * ceil(n / 64) (adding +0 leaves every
// start >= +0 unchanged) and readable for 8 values more.  segsum: LDS, the float64 sum of each segment (in
// any order: they only place the candidates).  sx: LDS scratch of NS * 64
// floats + NS ints, 16-byte aligned.  ctr: an LDS counter that reads `ctr0`
// on entry; it reads ctr0 + NW once every wavefront has arrived.  Every lane
// of wavefronts 0..NW-1 calls this with the same arguments; the sum is
// returned to wavefront 0 (the others return 0).
template <int CTRL>
__device__ __forceinline__ double dpp_mov_f64(double v) {
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = (int)b, hi = (int)(b >> 32);
    const int rl = __builtin_amdgcn_update_dpp(lo, lo, CTRL, 0xF, 0xF, false);
    const int rh = __builtin_amdgcn_update_dpp(hi, hi, CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)rh << 32) | (unsigned)rl));
}
__device__ __forceinline__ double lane_value_f64(double v, int lane) {
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_readlane((int)b, lane), hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
// Sum over the 64 lanes in some order (every lane active; the result, the
// same on every lane, only serves as an estimate).
__device__ __forceinline__ double wave_sum_f64(double x) {
    x += dpp_mov_f64<0xB1>(x);    // quad_perm [1,0,3,2]
    x += dpp_mov_f64<0x4E>(x);    // quad_perm [2,3,0,1]
    x += dpp_mov_f64<0x141>(x);   // row_half_mirror
    x += dpp_mov_f64<0x140>(x);   // row_mirror: every lane holds its row's total
    return (lane_value_f64(x, 0) + lane_value_f64(x, 16)) + (lane_value_f64(x, 32) + lane_value_f64(x, 48));
}
// Lane K of each 16-lane row, read by every lane of its row (DPP
// row_newbcast; the add that uses it takes it as its DPP operand).
template <int K>
__device__ __forceinline__ float row_bcast_lane(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + K, 0xF, 0xF,
                                                                 false));
}
// s0 += lanes 0..N-1 of v0's row one at a time, and s1 likewise from v1
// (two independent chains interleaved)
template <int N, int K = 0>
__device__ __forceinline__ void dpp_row_adds(float& s0, float v0, float& s1, float v1) {
    if constexpr (K < N) {
        s0 = fadd(s0, row_bcast_lane<K>(v0));
        s1 = fadd(s1, row_bcast_lane<K>(v1));
        dpp_row_adds<N, K + 1>(s0, v0, s1, v1);
    }
}
// Registers per chain that hold a short segment whole (16 values each).
constexpr int kSegShortRegs = 8;
// The chains over registers 0..L/16 of r0 and r1 (L a multiple of 8, at
// most 16 * kSegShortRegs), unrolled so that every register is named at
// compile time
template <int R = 0>
__device__ __forceinline__ void seg_chain_regs(float& s0, const float (&r0)[kSegShortRegs], float& s1,
                                               const float (&r1)[kSegShortRegs], int L) {
    if constexpr (R < kSegShortRegs) {
        if (16 * R + 16 <= L) {
            dpp_row_adds<16>(s0, r0[R], s1, r1[R]);
            seg_chain_regs<R + 1>(s0, r0, s1, r1, L);
        } else if (16 * R < L) {
            dpp_row_adds<8>(s0, r0[R], s1, r1[R]);
        }
    }
}
// Segment length of seg_serial_sum with NS segments: 8 * ceil(n / 8NS).
__host__ __device__ inline int seg_sum_len(int n, int NS) { return 8 * ((n + 8 * NS - 1) / (8 * NS)); }
// float64 sums of the NS = 2 NW segments of v (segsum, LDS), for callers
// that do not form them while writing v: wavefront w sums segments 2w and
// 2w+1.  Every lane of wavefronts 0..NW-1; a barrier must follow.
template <int NW>
__device__ void seg_sums_f64(const float* v, int n, double* segsum) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int L = seg_sum_len(n, 2 * NW);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int i = 2 * w + h;
        double acc = 0.0;
        for (int k = i * L + lane; k < (i + 1) * L; k += 64) acc += k < n ? (double)v[k] : 0.0;
        acc = wave_sum_f64(acc);
        if (lane == 0) segsum[i] = acc;
    }
}
template <int NW>
__device__ __forceinline__ float seg_serial_sum(const float* v, int n, const double* segsum, float* sx, int* ctr, int ctr0,
                                unsigned* fault) {
    constexpr int NS = 2 * NW;
    static_assert(NS <= 8, "one ds_read_b128 pair per lane holds the segment ends");
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int L = seg_sum_len(n, NS);
    const int i0 = 2 * w, i1 = 2 * w + 1;
    // float64 sum of the values before segment i0 (any order: an estimate)
    double sg[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) sg[i] = segsum[i];   // (all loads issued together)
    double before = 0.0, own = 0.0;
#pragma unroll
    for (int i = 0; i < NS - 1; i++) {
        before += i < i0 ? sg[i] : 0.0;
        own += i == i0 ? sg[i] : 0.0;
    }
    const double before1 = before + own;
    // candidate starts: 64 consecutive finite f32 bit patterns from `base`
    auto base_of = [](double est) {
        const int b = __float_as_int((float)est) - 32;
        return b < 0 ? 0 : (b > 0x7f7fffbf ? 0x7f7fffbf : b);
    };
    const int base0 = i0 == 0 ? 0 : base_of(before);
    const int base1 = base_of(before1);
    float s0 = __int_as_float(base0 + lane), s1 = __int_as_float(base1 + lane);
    // Each step of a chain is one add whose operand comes by DPP
    // row_newbcast from a register holding 16 of the segment's values in
    // every 16-lane row (lane l: value 16 r + l % 16), so no memory access
    // sits inside the chain (measured on gfx950: 8.5 cycles per dependent
    // add, 14 per step of two interleaved chains from registers, 23 with LDS
    // broadcast reads of the values in the loop).  Values from n on are +0
    // in v; positions past L belong to the next segment and are never added.
    const float* p0 = v + i0 * L + (lane & 15);
    const float* p1 = v + i1 * L + (lane & 15);
    if (L <= 16 * kSegShortRegs) {
        // Short segments (contexts up to 1024): every register is read
        // first, then the chains run straight through (an LDS read in flight
        // slows DPP adds down).  The reads are unconditional, so they all go
        // out before the first wait; registers past the segment re-read its
        // last one and are never added.
        float r0[kSegShortRegs], r1[kSegShortRegs];
        const int rlast = (L - 1) / 16;
#pragma unroll
        for (int r = 0; r < kSegShortRegs; r++) {
            r0[r] = p0[16 * (r < rlast ? r : rlast)];
            r1[r] = p1[16 * (r < rlast ? r : rlast)];
        }
        // (used here, so the compiler keeps every read ahead of the chains
        // instead of sinking each into the block of adds that needs it)
#pragma unroll
        for (int r = 0; r < kSegShortRegs; r++) asm volatile("" ::"v"(r0[r]), "v"(r1[r]));
        seg_chain_regs(s0, r0, s1, r1, L);
    } else {
        // Longer segments: chunks of 16 * kSegShortRegs values, each read
        // into registers whole before its adds (no LDS read in flight while
        // the chains run)
        for (int c0 = 0; c0 < L; c0 += 16 * kSegShortRegs) {
            const int len = L - c0 < 16 * kSegShortRegs ? L - c0 : 16 * kSegShortRegs;
            float r0[kSegShortRegs], r1[kSegShortRegs];
            const int rlast = (len - 1) / 16;
#pragma unroll
            for (int r = 0; r < kSegShortRegs; r++) {
                r0[r] = p0[c0 + 16 * (r < rlast ? r : rlast)];
                r1[r] = p1[c0 + 16 * (r < rlast ? r : rlast)];
            }
#pragma unroll
            for (int r = 0; r < kSegShortRegs; r++) asm volatile("" ::"v"(r0[r]), "v"(r1[r]));
            seg_chain_regs(s0, r0, s1, r1, len);
        }
    }
    // lane l's ends at sx[8 l + i]; the bases after them
    int* sbase = reinterpret_cast<int*>(sx + 8 * 64);
    sx[8 * lane + i0] = s0;
    sx[8 * lane + i1] = s1;
    if (lane == 0) {
        sbase[i0] = base0;
        sbase[i1] = base1;
    }
    lds_arrive(ctr);
    if (w != 0) return 0.0f;
    lds_wait_count(ctr, ctr0 + NW, fault);
    const vf4 e03 = *reinterpret_cast<const vf4*>(sx + 8 * lane);
    const vf4 e47 = *reinterpret_cast<const vf4*>(sx + 8 * lane + 4);
    const int myb = sbase[lane & (NS - 1)];
    const vf4 ends[2] = {e03, e47};
    // The walk is straight-line scalar code (the sum's bits in a scalar
    // register, selects, no branches): segment i's true start picks lane idx
    // of its ends; `from` is the first segment whose start is not among its
    // candidates (NS if none).
    int Sb = __builtin_amdgcn_readlane(__float_as_int(e03.x), 0);
    int from = NS;
#pragma unroll
    for (int i = 1; i < NS; i++) {
        const int idx = Sb - __builtin_amdgcn_readlane(myb, i);
        const bool live = i * L < n, hit = (unsigned)idx < 64u;
        const int next = __builtin_amdgcn_readlane(__float_as_int(ends[i / 4][i % 4]), idx & 63);
        const bool take = from == NS && live && hit;
        from = from == NS && live && !hit ? i : from;
        Sb = take ? next : Sb;
    }
    float S = __int_as_float(Sb);
    if (from < NS) {
        // the true start of segment `from` is not among its candidates:
        // one value at a time from there
        for (int k = from * L; k < n; k++) S = fadd(S, v[k]);
    }
    return S;
}

// seg_serial_sum for long rows: wavefront w sums segment w (NS = NW
// segments of L = 8 * ceil(n / 8NW) values) from 128 candidate starts, two
// chains per lane (base + lane and base + 64 + lane, base 64 below the float64
// estimate), since the one-at-a-time sum drifts further from the exact sum
// over thousands of values (a few tens of ulps at 8192).  Both chains read
// the same values, one register per 16.  Same contract as seg_serial_sum,
// with sx holding NW * 128 floats + NW ints and segsum one float64 sum per
// segment (seg_sums_f64_wide).
template <int NW>
__device__ void seg_sums_f64_wide(const float* v, int n, double* segsum) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int L = seg_sum_len(n, NW);
    double acc = 0.0;
    for (int k = w * L + lane; k < (w + 1) * L; k += 64) acc += k < n ? (double)v[k] : 0.0;
    acc = wave_sum_f64(acc);
    if (lane == 0) segsum[w] = acc;
}
template <int NW>
__device__ __forceinline__ float seg_serial_sum_wide(const float* v, int n, const double* segsum, float* sx, int* ctr,
                                                     int ctr0, unsigned* fault) {
    static_assert(NW <= 8, "two ds_read_b128 per lane and chain hold the segment ends");
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int L = seg_sum_len(n, NW);
    double sg[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) sg[i] = segsum[i];
    double before = 0.0;
#pragma unroll
    for (int i = 0; i < NW - 1; i++) before += i < w ? sg[i] : 0.0;
    int base = __float_as_int((float)before) - 64;
    base = base < 0 ? 0 : (base > 0x7f7fff7f ? 0x7f7fff7f : base);
    if (w == 0) base = 0;
    float s0 = __int_as_float(base + lane), s1 = __int_as_float(base + 64 + lane);
    const float* p = v + w * L + (lane & 15);
    if (L <= 16 * kSegShortRegs) {
        float r[kSegShortRegs];
        const int rlast = (L - 1) / 16;
#pragma unroll
        for (int k = 0; k < kSegShortRegs; k++) r[k] = p[16 * (k < rlast ? k : rlast)];
#pragma unroll
        for (int k = 0; k < kSegShortRegs; k++) asm volatile("" ::"v"(r[k]));   // (see seg_serial_sum)
        seg_chain_regs(s0, r, s1, r, L);
    } else {
        // chunks of 16 * kSegShortRegs values read into registers whole
        // before their adds (see seg_serial_sum)
        for (int c0 = 0; c0 < L; c0 += 16 * kSegShortRegs) {
            const int len = L - c0 < 16 * kSegShortRegs ? L - c0 : 16 * kSegShortRegs;
            float r[kSegShortRegs];
            const int rlast = (len - 1) / 16;
#pragma unroll
            for (int k = 0; k < kSegShortRegs; k++) r[k] = p[c0 + 16 * (k < rlast ? k : rlast)];
#pragma unroll
            for (int k = 0; k < kSegShortRegs; k++) asm volatile("" ::"v"(r[k]));
            seg_chain_regs(s0, r, s1, r, len);
        }
    }
    // lane l's ends at sx[16 l + 2 i + h] (segment i, chain h); bases after
    int* sbase = reinterpret_cast<int*>(sx + 16 * 64);
    sx[16 * lane + 2 * w] = s0;
    sx[16 * lane + 2 * w + 1] = s1;
    if (lane == 0) sbase[w] = base;
    lds_arrive(ctr);
    if (w != 0) return 0.0f;
    lds_wait_count(ctr, ctr0 + NW, fault);
    vf4 e[4];
#pragma unroll
    for (int k = 0; k < 4; k++) e[k] = *reinterpret_cast<const vf4*>(sx + 16 * lane + 4 * k);
    const int myb = sbase[lane & (NW - 1)];
    // the walk in scalar registers (see seg_serial_sum); candidate idx of
    // segment i is chain idx / 64 of lane idx % 64
    int Sb = __builtin_amdgcn_readlane(__float_as_int(e[0].x), 0);
    int from = NW;
#pragma unroll
    for (int i = 1; i < NW; i++) {
        const int idx = Sb - __builtin_amdgcn_readlane(myb, i);
        const bool live = i * L < n, hit = (unsigned)idx < 128u;
        const int n0 = __builtin_amdgcn_readlane(__float_as_int(e[(2 * i) / 4][(2 * i) % 4]), idx & 63);
        const int n1 = __builtin_amdgcn_readlane(__float_as_int(e[(2 * i + 1) / 4][(2 * i + 1) % 4]), idx & 63);
        const int next = idx >= 64 ? n1 : n0;
        const bool take = from == NW && live && hit;
        from = from == NW && live && !hit ? i : from;
        Sb = take ? next : Sb;
    }
    float S = __int_as_float(Sb);
    if (from < NW) {
        for (int k = from * L; k < n; k++) S = fadd(S, v[k]);
    }
    return S;
}

}  // namespace yl
