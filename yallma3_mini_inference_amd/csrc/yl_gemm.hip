// yl_gemm.hip -- quantized matmul over many tokens (prompt prefill, and
// yl_matmul with a large batch) on int8 MFMA, bit-identical to
// matmul_q8_slices (weight_type.rs:122-226).
//
// The reference sums, for each output (token t, row c), the block terms
//     term_b = ((float)isum_b * w_scale[c][b]) * x_scale[t][b]
// in ascending block order into an f32 accumulator, where isum_b is the
// exact int32 dot of one 32-element block.  v_mfma_i32_32x32x32_i8 has
// K = 32: one instruction yields exactly the 32x32 block dots of one block,
// and each lane then folds its 16 dots into its 16 f32 accumulators in
// block order with the reference's two roundings.  The f32 work per output
// and block is the bound, not the MFMA: with f16 scales (Q8_0, Q4_0) one
// fused multiply-add on a biased dot (the convert folded away; see `bias`
// in k_gemm), one product and one sum; with f32 scales a convert, two
// products and one sum.
//
// Tile: a 256-thread workgroup owns TM tokens x 128 weight rows (TM = 128,
// or 64 when the 128-token tiles would not give every CU two workgroups);
// wavefront w covers tokens (TM/2)*(w&1) .. +TM/2-1 and rows 64*(w>>1) ..
// +63 as (TM/64)x2 MFMA tiles.  MFMA lane layout (gfx950): operand lane l holds row l%32 (token
// for A, weight row for B) and k = 16*(l/32) .. +15 of the block; result
// register i of lane l is (token (i%4) + 8*(i/4) + 4*(l/32), row l%32).
// Stages of 2 blocks (activations 8 KiB, weights 8/4 KiB, both scale
// vectors) stream into LDS by LDS DMA, 4 stages deep, so no register holds
// data in flight.  Q4_0 weights keep the reference nibble order and are
// unpacked in registers to int8 in k order (values 0..15, no offset).
// Q8 with f32 scales (lm.rs, safetensors): per block (kQ8S), or per group
// of 2 or 4 blocks (kQ8S64, kQ8S128), whose block MFMAs accumulate into one
// int32 tile -- the group's exact dot -- before its one f32 term; the
// activations are quantized in the same groups.
#include <hip/hip_runtime.h>

#include "yl_blocks.h"
#include "yl_device.h"
#include "yl_internal.h"

namespace yl {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kGmThreads = 256;
constexpr int kGmTN = 128;      // weight rows per workgroup
constexpr int kGmBK = 2;        // blocks per stage
constexpr int kGmStages = 4;    // stages in flight

// 32-blocks per scale group
template <int WF>
constexpr int gm_bpg() { return WF == kQ8S64 ? 2 : (WF == kQ8S128 ? 4 : 1); }

template <int WF, int TM>
struct GmStage {
    static constexpr bool kF32 = WF == kQ8S || WF == kQ8S64 || WF == kQ8S128;
    static constexpr int kRowB = WF == kQ4 ? 16 : 32;         // weight bytes per row and block
    static constexpr int A = kGmBK * TM * 32;                 // [blk][token][32] int8
    static constexpr int B = kGmBK * kGmTN * kRowB;           // [blk][row][32 | 16]
    // activation scales: [blk][token] f32, or one per token for a stage
    // inside one group
    static constexpr int XS = gm_bpg<WF>() > 1 ? TM * 4 : kGmBK * TM * 4;
    // weight scales: [row][2] f16 (Q8_0 / Q4_0), [row][2] f32 (kQ8S), or one
    // f32 per row (the stage's group)
    static constexpr int WS = WF == kQ8S ? kGmTN * 8 : kGmTN * 4;
    static constexpr int bytes = A + B + XS + WS;
    // LDS DMA instructions per wavefront and stage (16-byte lanes move 1 KiB,
    // 4-byte lanes 256 B); every wavefront issues the same number
    static constexpr int dmaA = A / 1024 / 4;
    static constexpr int dmaB = B / 1024 / 4;
    static constexpr int dma = dmaA + dmaB + 1 + 1;
    static_assert(A % 4096 == 0 && B % 4096 == 0, "16-byte DMA split over 4 wavefronts");
    static_assert(XS % 256 == 0 && XS <= 4 * 256 && (WS == 2 * 256 || WS == 4 * 256), "scale DMA shapes");
};

template <int TM>
static size_t gemm_lds_bytes_tm(int wfmt) {
    switch (wfmt) {
    case kQ8: return (size_t)kGmStages * GmStage<kQ8, TM>::bytes;
    case kQ4: return (size_t)kGmStages * GmStage<kQ4, TM>::bytes;
    case kQ8S: return (size_t)kGmStages * GmStage<kQ8S, TM>::bytes;
    case kQ8S64: return (size_t)kGmStages * GmStage<kQ8S64, TM>::bytes;
    default: return (size_t)kGmStages * GmStage<kQ8S128, TM>::bytes;
    }
}
size_t gemm_lds_bytes(int wfmt, int tm) { return tm == 64 ? gemm_lds_bytes_tm<64>(wfmt) : gemm_lds_bytes_tm<128>(wfmt); }

template <int D>
__device__ __forceinline__ void gm_wait(int later) {
    // this wavefront's DMA of the current stage is done when at most
    // `later` younger stages (D instructions each) are still in flight
    static_assert(kGmStages - 2 == 2, "wait counts below cover two younger stages");
    if (later <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (later == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(D) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * D) : "memory");
}

// 8 Q4_0 bytes (16 nibbles, byte j = elements 2j | 2j+1 << 4) -> 16 int8
// in element order
__device__ __forceinline__ v4i q4_unpack16(uint2 p) {
    const uint32_t lo0 = p.x & 0x0f0f0f0fu, hi0 = (p.x >> 4) & 0x0f0f0f0fu;
    const uint32_t lo1 = p.y & 0x0f0f0f0fu, hi1 = (p.y >> 4) & 0x0f0f0f0fu;
    // v_perm_b32(hi, lo, sel): byte k of the result = byte sel_k of {hi:lo}
    // (lo = bytes 0..3, hi = bytes 4..7)
    v4i r;
    r.x = (int)__builtin_amdgcn_perm(hi0, lo0, 0x05010400u);   // lo0.b0 hi0.b0 lo0.b1 hi0.b1
    r.y = (int)__builtin_amdgcn_perm(hi0, lo0, 0x07030602u);   // lo0.b2 hi0.b2 lo0.b3 hi0.b3
    r.z = (int)__builtin_amdgcn_perm(hi1, lo1, 0x05010400u);
    r.w = (int)__builtin_amdgcn_perm(hi1, lo1, 0x07030602u);
    return r;
}

template <int WF, int EPI, int TM>
__global__ __launch_bounds__(kGmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm(GemvArgs a, int M) {
    // (device pass only: the host pass has no gfx950 MFMA builtins and
    // needs just the launch stub)
#if defined(__HIP_DEVICE_COMPILE__)
    using S = GmStage<WF, TM>;
    constexpr int TMW = TM / 64;   // 32-token MFMA tiles per wavefront
    constexpr int WT = TM / 2;     // tokens per wavefront
    extern __shared__ __align__(16) unsigned char gsm[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const int wm = wave & 1, wn = wave >> 1;
    const int c0 = blockIdx.x * kGmTN, t0 = blockIdx.y * TM;
    const int nst = a.nb / kGmBK;

    // accumulators: acc[tm][tn][i] = (token t0 + WT*wm + 32tm + (i%4) + 8(i/4) + 4lh,
    //                                 row c0 + 64wn + 32tn + li)
    float acc[TMW][2][16];
    int pos = 0;
    if constexpr (EPI == kEpiQkvRope) pos = a.state->pos;
    // QKV rows: each lane's stored column within q or k (RoPE pair order)
    // and its pair index, for its two 32-row blocks
    [[maybe_unused]] int kcol[2] = {0, 0}, qkcol[2] = {0, 0}, qpair[2] = {0, 0};
    if constexpr (EPI == kEpiQkvRope) {
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int c = c0 + 64 * wn + 32 * tn + li, att = a.att_dim;
            const int scol = c < att ? c : c - att;   // stored row within q or k
            kcol[tn] = qk_column(c - att, a.head_size, a.hf_rows);
            qkcol[tn] = qk_column(scol, a.head_size, a.hf_rows);
            qpair[tn] = (scol % a.head_size) >> 1;
        }
    }
    auto init_acc = [&]() {
#pragma unroll
    for (int tm = 0; tm < TMW; tm++)
#pragma unroll
        for (int tn = 0; tn < 2; tn++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float v = 0.0f;
                const int t = t0 + WT * wm + 32 * tm + (i & 3) + 8 * (i >> 2) + 4 * lh;
                const int c = c0 + 64 * wn + 32 * tn + li;
                if constexpr (EPI == kEpiStore) {
                    if (t < M && c < a.o && c < a.accumulate_cols) v = a.out[(size_t)t * a.o + c];
                } else if constexpr (EPI == kEpiQkvRope) {
                    // K/V rows accumulate into the cache (forward.rs:166-169);
                    // q rows start at 0.  A 32-row block is all q, all k or
                    // all v (att_dim and kv_dim are multiples of 32), so the
                    // branches are uniform; token t0 stands in for the rows
                    // past M in the (then unused) loads.
                    const int cb = c0 + 64 * wn + 32 * tn, att = a.att_dim, kv = a.kv_dim;
                    if (cb >= att && cb < a.o) {
                        const int tc = t < M ? t : t0;
                        const float u = cb < att + kv
                                            ? a.k_cache[(size_t)kcol[tn] * a.kv_ld + pos + tc]
                                            : a.v_cache[(size_t)(pos + tc) * kv + (c - att - kv)];
                        if (t < M) v = u;
                    }
                }
                acc[tm][tn][i] = v;
            }
    };

    // DMA of stage s (blocks 2s, 2s+1) into LDS buffer `buf`.  Token and
    // row indices past the matrix re-read the last valid one (results unused).
    auto issue = [&](unsigned char* buf, int s) {
        const int b0 = s * kGmBK;
        // activations: instruction j covers block j/(TM/32), tokens
        // 32*(j%(TM/32)) .. +31; lane i -> token i/2, half i%2
#pragma unroll
        for (int k = 0; k < S::dmaA; k++) {
            const int j = wave * S::dmaA + k;
            const int blk = j / (TM / 32), tok = min(t0 + 32 * (j % (TM / 32)) + (lane >> 1), M - 1);
            const int8_t* src = a.xq + (size_t)tok * a.n + (size_t)(b0 + blk) * 32 + 16 * (lane & 1);
            __builtin_amdgcn_global_load_lds(src, buf + j * 1024, 16, 0, 0);
        }
        // weights: Q8 as activations; Q4 instruction j covers block j/2, rows
        // 64*(j%2) .. +63, one 16-byte block per lane
#pragma unroll
        for (int k = 0; k < S::dmaB; k++) {
            const int j = wave * S::dmaB + k;
            const uint8_t* src;
            if constexpr (WF != kQ4) {
                const int blk = j / 4, row = min(c0 + 32 * (j % 4) + (lane >> 1), a.o - 1);
                src = a.qs + (size_t)row * a.n + (size_t)(b0 + blk) * 32 + 16 * (lane & 1);
            } else {
                const int blk = j / 2, row = min(c0 + 64 * (j % 2) + lane, a.o - 1);
                src = a.qs + (size_t)row * (a.n / 2) + (size_t)(b0 + blk) * 16;
            }
            __builtin_amdgcn_global_load_lds(src, buf + S::A + j * 1024, 16, 0, 0);
        }
        constexpr int G = gm_bpg<WF>();
        // activation scales in 256-byte pieces of 64 tokens, piece p by
        // wavefront p (the others repeat the first ones: identical bytes)
        constexpr int XP = S::XS / 256, TP = TM / 64;   // pieces; pieces per block
        const int p = wave % XP;
        if constexpr (G == 1) {
            // piece p: block p/TP, tokens 64*(p%TP) + lane
            const int tok = min(t0 + 64 * (p % TP) + lane, M - 1);
            __builtin_amdgcn_global_load_lds(a.xs + (size_t)tok * a.nb + b0 + p / TP, buf + S::A + S::B + p * 256, 4,
                                             0, 0);
        } else {
            // the group's scale per token: piece p -> tokens 64p + lane
            const int tok = min(t0 + 64 * p + lane, M - 1);
            __builtin_amdgcn_global_load_lds(a.xs + (size_t)tok * (a.nb / G) + b0 / G, buf + S::A + S::B + p * 256, 4,
                                             0, 0);
        }
        if constexpr (WF == kQ8S) {
            // f32 block scales [row][2]: wavefront w -> rows 32w .. +31, lane i
            // -> row i/2, block i%2
            const int row = min(c0 + 32 * wave + (lane >> 1), a.o - 1);
            __builtin_amdgcn_global_load_lds(a.sf + (size_t)row * a.nb + b0 + (lane & 1),
                                             buf + S::A + S::B + S::XS + wave * 256, 4, 0, 0);
        } else if constexpr (G > 1) {
            // the group's f32 scale per row: rows 64*(w%2) + lane (wavefronts 2
            // and 3 repeat 0 and 1)
            const int row = min(c0 + 64 * (wave & 1) + lane, a.o - 1);
            __builtin_amdgcn_global_load_lds(a.sf + (size_t)row * (a.nb / G) + b0 / G,
                                             buf + S::A + S::B + S::XS + (wave & 1) * 256, 4, 0, 0);
        } else {
            // weight scales: rows 64*(w%2) + lane, the stage's two f16 as one dword
            // (wavefronts 2 and 3 repeat 0 and 1)
            const int row = min(c0 + 64 * (wave & 1) + lane, a.o - 1);
            __builtin_amdgcn_global_load_lds(a.d + (size_t)row * a.nb + b0, buf + S::A + S::B + S::XS + (wave & 1) * 256,
                                             4, 0, 0);
        }
    };

    // f16 block scales (Q8_0, Q4_0): every block dot starts from the int32
    // bits of the float 3*2^22 instead of 0, so the MFMA's result reads as the
    // float f = 3*2^22 + isum, exactly (|isum| <= 32*128*128 < 2^22).  Then
    //     fma(f, ws, -3*2^22*ws) = round(isum * ws),
    // one rounding of the exact product (3*2^22*ws is exact for an f16 ws):
    // the convert drops out of the per-output work (3 VALU operations
    // instead of 4).  The value equals (float)isum * ws, except that an exact
    // cancellation gives +0 where isum = 0 or ws = 0 gives the product's
    // signed zero.  A zero term's sign changes the sum only while the
    // accumulator is -0, and an accumulator that does not start at -0 never
    // becomes -0 (+0 + -0 = +0, and x + -x = +0).  A non-finite scale makes
    // inf - inf.  So the fused pass is exact unless a -0 initial value or a
    // non-finite scale is present; the lanes that see one flag it, and the
    // workgroup then reloads its initial values (only the epilogue writes
    // them) and runs the reference's form.  The bias tuple is opaque to the
    // compiler, so it stays in registers rather than being rematerialized
    // before each MFMA.
    constexpr bool kBias = WF == kQ8 || WF == kQ4;
    constexpr float kBiasF = 12582912.0f;   // 3 * 2^22, bits 0x4B400000
    __shared__ int redo;
    v16i bias = {};
    if constexpr (kBias) {
#pragma unroll
        for (int i = 0; i < 16; i++) bias[i] = 0x4B400000;
        asm volatile("" : "+v"(bias));
        if (threadIdx.x == 0) redo = 0;   // ordered before any flag by the first stage's barrier
    }

    // group dots of the f32-scaled formats with 2 or 4 blocks per group,
    // accumulated over the group's blocks (exact int32)
    constexpr int G = gm_bpg<WF>();
    // the K loop: FUSED.value selects the biased form above
    auto run = [&](auto FUSED) -> bool {
    constexpr bool kFused = decltype(FUSED)::value;
    bool flag = false;   // this lane saw a -0 initial value or a non-finite scale
    if constexpr (kFused) {
#pragma unroll
        for (int tm = 0; tm < TMW; tm++)
#pragma unroll
            for (int tn = 0; tn < 2; tn++)
#pragma unroll
                for (int i = 0; i < 16; i++) flag = flag || __float_as_uint(acc[tm][tn][i]) == 0x80000000u;
    }
    // the initial values have landed before any DMA is issued, so the
    // stage waits below count DMA instructions only
    wait_vm_all();
    // prologue: the first kGmStages - 1 stages in flight
#pragma unroll
    for (int s = 0; s < kGmStages - 1; s++)
        if (s < nst) issue(gsm + s * S::bytes, s);

    v16i gd[TMW][2] = {};
    for (int s = 0; s < nst; s++) {
        gm_wait<S::dma>(min(kGmStages - 2, nst - 1 - s));
        __syncthreads();   // every wavefront's DMA of stage s landed; stage s-1's buffer is free
        if (s + kGmStages - 1 < nst)
            issue(gsm + ((s + kGmStages - 1) % kGmStages) * S::bytes, s + kGmStages - 1);
        const unsigned char* buf = gsm + (s % kGmStages) * S::bytes;
        const float* xsl = reinterpret_cast<const float*>(buf + S::A + S::B);
        const uint16_t* wsl = reinterpret_cast<const uint16_t*>(buf + S::A + S::B + S::XS);
#pragma unroll
        for (int blk = 0; blk < kGmBK; blk++) {
            const unsigned char* Ab = buf + blk * (TM * 32);
            const unsigned char* Bb = buf + S::A + blk * (kGmTN * S::kRowB);
            v4i av[TMW], bv[2];
#pragma unroll
            for (int tm = 0; tm < TMW; tm++)
                av[tm] = *reinterpret_cast<const v4i*>(Ab + (WT * wm + 32 * tm + li) * 32 + 16 * lh);
#pragma unroll
            for (int tn = 0; tn < 2; tn++) {
                if constexpr (WF != kQ4) {
                    bv[tn] = *reinterpret_cast<const v4i*>(Bb + (64 * wn + 32 * tn + li) * 32 + 16 * lh);
                } else {
                    bv[tn] = q4_unpack16(*reinterpret_cast<const uint2*>(Bb + (64 * wn + 32 * tn + li) * 16 + 8 * lh));
                }
            }
            if constexpr (G > 1) {
                // this block's dots join the group's (the first block of a
                // group starts from zero); the term follows the group's last
                const bool first = ((s * kGmBK + blk) % G) == 0;
#pragma unroll
                for (int tm = 0; tm < TMW; tm++)
#pragma unroll
                    for (int tn = 0; tn < 2; tn++) {
                        const v16i zero = {};
                        gd[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[tm], bv[tn], first ? zero : gd[tm][tn],
                                                                           0, 0, 0);
                    }
                if ((s * kGmBK + blk) % G != G - 1) continue;
                __builtin_amdgcn_sched_barrier(0);
                const float* wsf = reinterpret_cast<const float*>(wsl);
                float wsc[2];
#pragma unroll
                for (int tn = 0; tn < 2; tn++) wsc[tn] = wsf[64 * wn + 32 * tn + li];
#pragma unroll
                for (int tm = 0; tm < TMW; tm++)
#pragma unroll
                    for (int tn = 0; tn < 2; tn++)
#pragma unroll
                        for (int i = 0; i < 16; i++) {
                            const float xs = xsl[WT * wm + 32 * tm + (i & 3) + 8 * (i >> 2) + 4 * lh];
                            const float term = fmul(fmul((float)gd[tm][tn][i], wsc[tn]), xs);
                            acc[tm][tn][i] = fadd(acc[tm][tn][i], term);
                        }
                continue;
            }
            float wsc[2];
#pragma unroll
            for (int tn = 0; tn < 2; tn++) {
                if constexpr (WF == kQ8S)
                    wsc[tn] = reinterpret_cast<const float*>(wsl)[(64 * wn + 32 * tn + li) * 2 + blk];
                else
                    wsc[tn] = f16_to_f32(wsl[(64 * wn + 32 * tn + li) * 2 + blk]);
            }
            vf4 xv[TMW][4];
#pragma unroll
            for (int tm = 0; tm < TMW; tm++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    xv[tm][g] = *reinterpret_cast<const vf4*>(xsl + blk * TM + WT * wm + 32 * tm + 8 * g + 4 * lh);
            if constexpr (kFused) {
                // two tiles in flight: tile k+1's MFMA runs while tile k is
                // folded (the bias leaves no registers for all four)
                flag = flag || !(fabsf(wsc[0]) < INFINITY) || !(fabsf(wsc[1]) < INFINITY);
                const float cb[2] = {fmul(-kBiasF, wsc[0]), fmul(-kBiasF, wsc[1])};
                // f32 scales in registers: otherwise the compiler folds the f16
                // convert into each FMA (v_fma_mix_f32)
                asm volatile("" : "+v"(wsc[0]), "+v"(wsc[1]));
                constexpr int NT = TMW * 2;
                v16i d[2];
                d[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[0], bv[0], bias, 0, 0, 0);
#pragma unroll
                for (int k = 0; k < NT; k++) {
                    if (k + 1 < NT)
                        d[(k + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[(k + 1) >> 1], bv[(k + 1) & 1],
                                                                               bias, 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    const int tm = k >> 1, tn = k & 1;
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const float f = __int_as_float(d[k & 1][i]);
                        const float term = fmul(__builtin_fmaf(f, wsc[tn], cb[tn]), xv[tm][i >> 2][i & 3]);
                        acc[tm][tn][i] = fadd(acc[tm][tn][i], term);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                continue;
            }
            // the four tiles' dots first (in separate registers), so the f32
            // work of one tile does not wait on the next tile's MFMA
            v16i dots[TMW][2];
#pragma unroll
            for (int tm = 0; tm < TMW; tm++)
#pragma unroll
                for (int tn = 0; tn < 2; tn++) {
                    const v16i zero = {};
                    dots[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[tm], bv[tn], zero, 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int tm = 0; tm < TMW; tm++)
#pragma unroll
                for (int tn = 0; tn < 2; tn++)
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const float term = fmul(fmul((float)dots[tm][tn][i], wsc[tn]), xv[tm][i >> 2][i & 3]);
                        acc[tm][tn][i] = fadd(acc[tm][tn][i], term);
                    }
        }
    }
    return flag;
    };

    init_acc();
    if constexpr (kBias) {
        if (run(std::true_type{})) redo = 1;
        __syncthreads();   // every flag is in; every wavefront is done with the LDS stages
        if (redo) {
            init_acc();
            run(std::false_type{});
        }
    } else {
        run(std::false_type{});
    }

    // epilogues (SwiGLU: TMW * 16 exponentials per lane, with expf's
    // constants in registers)
    [[maybe_unused]] const ExpfK ek = EPI == kEpiSwiglu ? expf_k_regs() : expf_k_imm();
#pragma unroll
    for (int tm = 0; tm < TMW; tm++) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = t0 + WT * wm + 32 * tm + (i & 3) + 8 * (i >> 2) + 4 * lh;
            const bool tok_ok = t < M;
            if constexpr (EPI == kEpiSwiglu) {
                // SwiGLU (forward.rs:220-237) over the 64-row group [32 gate |
                // 32 up] of this wavefront, then the 32-group quantization of h
                const int grp = (c0 + 64 * wn) / 64;
                const bool grp_ok = c0 + 64 * wn < a.o;
                const float g = acc[tm][0][i], u = acc[tm][1][i];
                const float den = fadd(1.0f, expf_rn(-g, ek));
                const float h = fmul(g / den, u);
                if (!a.hq) {   // f32 h only (quantized afterwards in the model's groups)
                    if (tok_ok && grp_ok) a.h_f32[(size_t)t * a.hidden + (size_t)grp * kGroup + li] = h;
                    continue;
                }
                float am = group_max(fabsf(h), 32);
                am = fmaxf(am, 0.0f);
                const float sc = a.h_fmt == kQ4 ? group_scale<kQ4>(am) : group_scale<kQ8>(am);
                const int q = a.h_fmt == kQ4 ? quant_one<kQ4>(h, sc) : quant_one<kQ8>(h, sc);
                if (tok_ok && grp_ok) {
                    const size_t base = (size_t)t * a.hidden + (size_t)grp * kGroup;
                    if (a.h_f32) a.h_f32[base + li] = h;
                    a.hq[base + li] = (int8_t)q;
                    if (li == 0) a.hs[(size_t)t * (a.hidden / kGroup) + grp] = sc;
                }
            } else {
#pragma unroll
                for (int tn = 0; tn < 2; tn++) {
                    const int c = c0 + 64 * wn + 32 * tn + li;
                    const float v = acc[tm][tn][i];
                    if constexpr (EPI == kEpiQkvRope) {
                        // rope_gguf (util.rs:653-718) on q and k pairs (2j, 2j+1):
                        // the pair partner is the neighbouring lane
                        const float other = dpp_mov<0xB1>(v);
                        // (uniform branches on the 32-row block, as in the
                        // initial values)
                        const int cb = c0 + 64 * wn + 32 * tn;
                        const int att = a.att_dim, kv = a.kv_dim, hd = a.head_size;
                        if (cb >= att + kv) {
                            if (tok_ok && cb < a.o) a.v_cache[(size_t)(pos + t) * kv + (c - att - kv)] = v;
                        } else {
                            const int tc = tok_ok ? t : t0;
                            const float cs = a.rope_cos[(size_t)(pos + tc) * (hd >> 1) + qpair[tn]];
                            const float sn = a.rope_sin[(size_t)(pos + tc) * (hd >> 1) + qpair[tn]];
                            const float v0 = (li & 1) ? other : v, v1 = (li & 1) ? v : other;
                            const float r = (li & 1) ? fadd(fmul(v0, sn), fmul(v1, cs)) : fmul(v0, cs) - fmul(v1, sn);
                            if (tok_ok) {
                                if (cb < att) a.q_out[(size_t)t * att + qkcol[tn]] = r;
                                else a.k_cache[(size_t)qkcol[tn] * a.kv_ld + pos + t] = r;
                            }
                        }
                    } else if (tok_ok && c < a.o) {
                        if constexpr (EPI == kEpiStore) a.out[(size_t)t * a.o + c] = v;
                        if constexpr (EPI == kEpiResid) {
                            // residual add (forward.rs:196-204 / 245-253)
                            float* xp = a.x + (size_t)t * a.o + c;
                            *xp = fadd(*xp, v);
                        }
                    }
                }
            }
        }
    }

#endif
}

template <int WF, int EPI, int TM>
static hipError_t launch_gemm_tm(const GemvArgs& a, int M, hipStream_t st) {
    const size_t smem = gemm_lds_bytes_tm<TM>(WF);
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm<WF, EPI, TM>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const dim3 grid((a.o + kGmTN - 1) / kGmTN, (M + TM - 1) / TM);
    hipLaunchKernelGGL((k_gemm<WF, EPI, TM>), grid, dim3(kGmThreads), smem, st, a, M);
    return hipGetLastError();
}

// 64-token tiles when 128-token tiles would give each CU at most one
// workgroup (the f32 rescale is VALU-bound: a second workgroup per CU keeps
// the matrix pipe and the VALU of one SIMD busy from different wavefronts).
// Measured at 2048 tokens: Wo 82.5 -> 62.8 us and down 267 -> 203 us with 64
// (256 -> 512 workgroups), but QKV 108 -> 131 us (384 -> 768), so 1.5
// workgroups per CU keep 128.
int gemm_tile_tokens(int o, int M) {
    const long wg128 = (long)((o + kGmTN - 1) / kGmTN) * ((M + 127) / 128);
    return wg128 <= 256 ? 64 : 128;
}

template <int WF, int EPI>
static hipError_t launch_gemm_k(const GemvArgs& a, int M, hipStream_t st) {
    // Q8 with one f32 scale per 4 blocks keeps a group's int32 dots of four
    // tiles in registers besides the accumulators: at 128 tokens that does
    // not fit in 256 registers (spills), so it always takes 64-token tiles
    if constexpr (WF == kQ8S128) return launch_gemm_tm<WF, EPI, 64>(a, M, st);
    else
        return gemm_tile_tokens(a.o, M) == 64 ? launch_gemm_tm<WF, EPI, 64>(a, M, st)
                                              : launch_gemm_tm<WF, EPI, 128>(a, M, st);
}

bool gemm_supported(const GemvArgs& a, int wfmt, int epi, int M) {
    if (M < 1 || a.n % 32 || a.nb != a.n / 32 || a.nb % kGmBK) return false;
    if (wfmt != kQ8 && wfmt != kQ4 && wfmt != kQ8S && wfmt != kQ8S64 && wfmt != kQ8S128) return false;
    if ((wfmt == kQ8S64 && a.nb % 2) || (wfmt == kQ8S128 && a.nb % 4)) return false;
    if (epi == kEpiSwiglu && !a.hq && !a.h_f32) return false;
    if (epi == kEpiSwiglu && (a.o % 64 || a.hidden * 2 != a.o)) return false;
    if (epi == kEpiQkvRope && (a.head_size % 2 || a.att_dim % 32 || a.kv_dim % 32)) return false;
    return true;
}

hipError_t launch_gemm(const GemvArgs& a, int wfmt, int epi, int M, hipStream_t st) {
    if (!gemm_supported(a, wfmt, epi, M)) return hipErrorInvalidValue;
#define YL_GEMM_EPI(WF)                                                        \
    switch (epi) {                                                             \
    case kEpiStore: return launch_gemm_k<WF, kEpiStore>(a, M, st);            \
    case kEpiQkvRope: return launch_gemm_k<WF, kEpiQkvRope>(a, M, st);        \
    case kEpiResid: return launch_gemm_k<WF, kEpiResid>(a, M, st);            \
    case kEpiSwiglu: return launch_gemm_k<WF, kEpiSwiglu>(a, M, st);          \
    default: return hipErrorInvalidValue;                                      \
    }
    if (wfmt == kQ8) { YL_GEMM_EPI(kQ8) }
    if (wfmt == kQ8S) { YL_GEMM_EPI(kQ8S) }
    if (wfmt == kQ8S64) { YL_GEMM_EPI(kQ8S64) }
    if (wfmt == kQ8S128) { YL_GEMM_EPI(kQ8S128) }
    YL_GEMM_EPI(kQ4)
#undef YL_GEMM_EPI
}

}  // namespace yl
