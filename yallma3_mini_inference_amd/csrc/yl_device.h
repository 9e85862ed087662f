// yl_device.h -- device-side arithmetic shared by every kernel.
//
// Bit-exactness contract: the forward path reproduces the reference's f32
// operation order (products and sums rounded one at a time, no fused
// multiply-add).  All HIP sources are compiled with -ffp-contract=off;
// the helpers below spell each rounding step out so the order is visible.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "yl_internal.h"

namespace yl {

constexpr int kGroup = 32;        // block size of Q8_0/Q4_0 (transformer_llama_gguf.rs:281)

// Native 4-float vector for register arrays: copies of HIP's float4 (a
// struct) lower to memcpy, which can keep an array out of registers.
typedef float vf4 __attribute__((ext_vector_type(4)));
typedef float vf2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float fadd(float a, float b) { return a + b; }
__device__ __forceinline__ float fmul(float a, float b) { return a * b; }

// IEEE binary16 bits -> binary32 (exact; v_cvt_f32_f16 keeps f16 subnormals).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// wide::f32x8::reduce_add as built without AVX (forward.rs:340,391,273;
// util.rs:406): each f32x4 half summed left to right, then the halves added.
__device__ __forceinline__ float reduce_add8(const float l[8]) {
    float a = fadd(fadd(fadd(l[0], l[1]), l[2]), l[3]);
    float b = fadd(fadd(fadd(l[4], l[5]), l[6]), l[7]);
    return fadd(a, b);
}

// exp evaluated in binary64, rounded once to binary32: x*log2(e) -> k
// (nearest), r = (x - k*ln2_hi) - k*ln2_lo with the fdlibm split of ln2,
// e^r by the degree-13 Taylor polynomial (Horner, one fused multiply-add per
// degree, as in the oracle), scaled by 2^k.  It is the
// correctly rounded expf except with probability ~1e-9 per input; it stands
// in for f32::exp in the softmax (forward.rs:358) and wide::f32x8::exp in
// SwiGLU (forward.rs:230).
// Its binary64 constants (the polynomial's 1/2 and 1s are inline operands).
// f64 operations take no 64-bit literal, so an immediate constant is moved
// into a register pair at each use (two moves per Horner step ahead of a
// v_fmac_f64).  A kernel that evaluates many exponentials takes the
// constants into registers once (expf_k_regs) and passes them to
// expf_rn(x, k), whose steps are then register-operand FMAs: the same
// operations on the same values, so the same results.
struct ExpfK {
    double log2e, ln2_hi, ln2_lo;
    double c[11];   // Horner coefficients of degrees 13 .. 3
};
__device__ __forceinline__ constexpr ExpfK expf_k_imm() {
    return ExpfK{0x1.71547652b82fep+0, 0x1.62e42fee00000p-1, 0x1.a39ef35793c76p-33,
                 {0x1.6124613a86d09p-33, 0x1.1eed8eff8d898p-29, 0x1.ae64567f544e4p-26, 0x1.27e4fb7789f5cp-22,
                  0x1.71de3a556c734p-19, 0x1.a01a01a01a01ap-16, 0x1.a01a01a01a01ap-13, 0x1.6c16c16c16c17p-10,
                  0x1.1111111111111p-7, 0x1.5555555555555p-5, 0x1.5555555555555p-3}};
}
// the constants in registers, opaque to the compiler (so not re-materialized)
__device__ __forceinline__ ExpfK expf_k_regs() {
    ExpfK k = expf_k_imm();
    asm volatile("" : "+v"(k.log2e), "+v"(k.ln2_hi), "+v"(k.ln2_lo));
#pragma unroll
    for (int i = 0; i < 11; i++) asm volatile("" : "+v"(k.c[i]));
    return k;
}
__device__ __forceinline__ float expf_rn(float xf, const ExpfK& k) {
    if (xf != xf) return xf;
    if (xf > 88.8f) return __builtin_inff();
    if (xf < -104.0f) return 0.0f;
    const double x = (double)xf;
    const double kd = __builtin_rint(x * k.log2e);
    const double r = (x - kd * k.ln2_hi) - kd * k.ln2_lo;
    double p = k.c[0];
#pragma unroll
    for (int i = 1; i < 11; i++) p = __builtin_fma(p, r, k.c[i]);
    p = __builtin_fma(p, r, 0x1.0000000000000p-1);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return (float)__builtin_amdgcn_ldexp(p, (int)kd);
}
__device__ __forceinline__ float expf_rn(float xf) { return expf_rn(xf, expf_k_imm()); }

// Rust `(v).round() as i8`: half away from zero, saturating, NaN -> 0
// (written with selects only, no branches).
__device__ __forceinline__ int round_to_i8(float v) {
    float r = __builtin_roundf(v);
    r = __builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
    return v != v ? 0 : (int)r;
}

// One group of 32 activations -> quantized values and scale.
//   Q8_0: quantization.rs:29-52  (scale = absmax/127, q = round(x/scale))
//   Q4_0: weight_type.rs:52-74   (scale = absmax/7,  then clamp to +-7)
// `absmax` follows the reference's `if val > wmax` scan from 0 (NaN never
// wins), which equals fmaxf over |x| and 0.
template <int FMT>
__device__ __forceinline__ float group_scale(float absmax) {
    return FMT == kQ4 ? absmax / 7.0f : absmax / 127.0f;
}
template <int FMT>
__device__ __forceinline__ int quant_one(float x, float scale) {
    int q = round_to_i8(x / scale);
    if (FMT == kQ4) q = q < -7 ? -7 : (q > 7 ? 7 : q);
    return q;
}

// quant_one over 8 values of one group, without a division per value.
// y = x * fl(1/scale) is within |x/scale| * 2^-23 <= 2^-16 of x/scale (the
// quotient never exceeds 127 * (1 + 2^-23) in magnitude), and so is the
// reference's fl(x/scale).  When y lies more than 2^-14 from every
// half-integer, both round to rint(y); otherwise (and for NaN, an infinite
// or zero reciprocal, or a scale below 2^-100) the lane takes quant_one's
// exact division.  Ties therefore always go through the exact path.
template <int FMT>
__device__ __forceinline__ void quant8(const float v[8], float scale, int q[8]) {
    const float rinv = 1.0f / scale;
    bool slow = !(rinv <= 0x1p100f);
    constexpr float lo = FMT == kQ4 ? -7.0f : -128.0f, hi = FMT == kQ4 ? 7.0f : 127.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float y = v[k] * rinv;
        const float r = __builtin_rintf(y);
        slow = slow || !(__builtin_fabsf(y - r) <= 0.5f - 0x1p-14f);
        q[k] = (int)__builtin_fminf(__builtin_fmaxf(r, lo), hi);
    }
    if (slow) {
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = quant_one<FMT>(v[k], scale);
    }
}

// Lane permutation by DPP (a VALU operand modifier, no LDS round trip).
// Lanes whose source is out of range keep their own value.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    const int i = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(i, i, CTRL, 0xF, 0xF, false));
}

// Maximum over aligned groups of P consecutive lanes (P = 1, 2, ..., 32,
// uniform across the wavefront).  Every lane of the wavefront must be active.
// After the quad steps each quad holds its maximum, so mirroring within
// half-rows (8 lanes) and rows (16 lanes) pairs each lane with the other
// half; the last step crosses rows.
__device__ __forceinline__ float group_max(float v, int P) {
    if (P >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));    // quad_perm [1,0,3,2]
    if (P >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));    // quad_perm [2,3,0,1]
    if (P >= 8) v = fmaxf(v, dpp_mov<0x141>(v));   // row_half_mirror
    if (P >= 16) v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
    if (P >= 32) v = fmaxf(v, __shfl_xor(v, 16, 32));
    return v;
}

// Maximum over the 64 lanes of a wavefront (every lane active), returned to
// every lane: the 16-lane row maxima by DPP, then the four rows' by
// readlane, with no LDS round trip.  fmaxf keeps the larger non-NaN operand,
// so the order of the reduction does not change the result.
__device__ __forceinline__ float wave_max(float v) {
    v = group_max(v, 16);
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// DPP move with out-of-row (or masked-off) lanes reading 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_zero(float v) {
    const int i = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, i, CTRL, ROW_MASK, 0xF, true));
}

// Inclusive prefix sum over the 64 lanes (every lane active): shifts by 1,
// 2, 4, 8 within each row of 16, then row 0's total into row 1 and row 2's
// into row 3 (row_bcast:15), then lane 31's total into rows 2 and 3
// (row_bcast:31).  Exact when every partial sum is an integer below 2^24.
__device__ __forceinline__ float wave_scan_add(float x) {
    x = x + dpp_zero<0x111, 0xF>(x);   // row_shr:1
    x = x + dpp_zero<0x112, 0xF>(x);   // row_shr:2
    x = x + dpp_zero<0x114, 0xF>(x);   // row_shr:4
    x = x + dpp_zero<0x118, 0xF>(x);   // row_shr:8
    x = x + dpp_zero<0x142, 0xA>(x);   // row_bcast:15 into rows 1, 3
    x = x + dpp_zero<0x143, 0xC>(x);   // row_bcast:31 into rows 2, 3
    return x;
}

// Workgroup barrier ordering LDS traffic only: waits for this wavefront's
// LDS operations, but not for its global loads or LDS DMA in flight (a
// __syncthreads() is a release fence, and on this target waits for both).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 32-bit LDS offset of a pointer into shared memory
__device__ __forceinline__ unsigned lds_addr(const float* p) {
    return (unsigned)(size_t)(const __attribute__((address_space(3))) float*)p;
}

// rows O and O + 1 (64 floats apart) at LDS offset a, untracked by the
// compiler's waits: the caller waits with lgkm_wait_tie before the use
template <int O>
__device__ __forceinline__ vf2 lds_read2st64(unsigned a) {
    static_assert(O >= 0 && O + 1 < 256, "offset field");
    vf2 r;
    asm volatile("ds_read2st64_b32 %0, %1 offset0:%2 offset1:%3" : "=v"(r) : "v"(a), "n"(O), "n"(O + 1) : "memory");
    return r;
}

// 16 bytes at LDS offset a + O (a broadcast when a is uniform), untracked
template <int O>
__device__ __forceinline__ vf4 lds_read_b128(unsigned a) {
    static_assert(O >= 0 && O < 65536, "offset field");
    vf4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(O) : "memory");
    return r;
}

// s_waitcnt lgkmcnt(N), tied to the registers it makes valid so that no use
// of them is scheduled above it.  The untracked reads are safe only while
// their results stay in the registers the reads name until this wait (the
// generated code is checked for copies in between).
template <int N>
__device__ __forceinline__ void lgkm_wait_tie(vf2& a, vf2& b, vf2& c, vf2& d, vf4& e, vf4& f) {
    static_assert(N >= 0 && N < 16, "lgkmcnt field");
    asm volatile("s_waitcnt lgkmcnt(%6)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f) : "n"(N) : "memory");
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// vmcnt <= k * D for a run-time k in [0, 7]
template <int D>
__device__ __forceinline__ void wait_vm_slots(int k) {
    switch (k) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<D>(); break;
    case 2: wait_vm<2 * D>(); break;
    case 3: wait_vm<3 * D>(); break;
    case 4: wait_vm<4 * D>(); break;
    case 5: wait_vm<5 * D>(); break;
    case 6: wait_vm<6 * D>(); break;
    default: wait_vm<7 * D>(); break;
    }
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// The serial f32 sum ((0 + v[0]) + v[1]) + ... + v[n-1] of n nonnegative
// values, bit-identical to the one-at-a-time loop, computed by one whole
// wavefront (all 64 lanes active, the same n and values on every lane); the
// values are read as get(i), 0 <= i < n, in any layout.
//
// While the running sum s stays inside one binade it is a multiple of the
// binade's ulp u, and the step fl(s + v) equals s + rn_u(v) -- v rounded to
// the nearest multiple of u -- unless v/u lies exactly halfway between two
// integers (the tie is broken by the last bit of s).  The first 32 values
// are added one at a time: the early sum crosses a binade every few values.
// Then the wavefront takes super-rows of 64 lanes x KV consecutive values:
// r = rint(v/u) (integers below 2^24), each lane's running sums of its own
// r, a DPP scan of the lane totals, and the candidates s + prefix*u (all
// exact).  Candidates never decrease, so a super-row whose values hold no
// tie and none at or above the binade's top B, and whose last candidate per
// lane stays below B, is taken whole.  Otherwise the first offending value
// in order is added by one ordinary f32 add onto the exact sum before it,
// and the same super-row (still in registers) is scanned again from the
// next value with the new binade.  A zero sum takes the next nonzero value
// exactly (0 + v = v).  A softmax denominator over n positions costs about
// n/512 super-row passes plus one pass per binade crossed after the 32nd
// value (a handful).
constexpr int kSerialSumPrologue = 32;

// s is +inf or NaN and values from `start` on are still to be added: adding
// nonnegative values keeps +inf, and a NaN among them gives NaN
template <class Get>
__device__ __forceinline__ float serial_sum_nonfinite(Get get, int n, int start, float s) {
    if (s != s) return s;
    bool nan = false;
    for (int i = start + (int)(threadIdx.x & 63); i < n; i += 64) {
        const float v = get(i);
        nan = nan || v != v;
    }
    return __ballot(nan) ? __builtin_nanf("") : s;
}

// `s0` is the running sum before v[0] (0 for a whole row; a long row can be
// summed in segments, each continuing from the previous segment's result).
template <int KV = 8, class Get>
__device__ __forceinline__ float wave_serial_sum_at(Get get, int n, float s0 = 0.0f) {
    const int lane = threadIdx.x & 63;
    const int np0 = n < kSerialSumPrologue ? n : kSerialSumPrologue;
    const float x0 = lane < np0 ? get(lane) : 0.0f;
    float s = s0;
#pragma unroll
    for (int i = 0; i < kSerialSumPrologue; i++)
        if (i < np0) s = fadd(s, lane_value(x0, i));
    int start = np0;   // the first value not yet added
    constexpr int W = 64 * KV;
    for (int t0 = (start / W) * W; start < n; t0 += W) {
        const int base = t0 + KV * lane;   // index of this lane's x[0]
        float x[KV];
#pragma unroll
        for (int i = 0; i < KV; i++) x[i] = base + i < n ? get(base + i) : 0.0f;
        const int end = n < t0 + W ? n : t0 + W;
        while (start < end) {
            if (!(s <= 0x1.fffffep127f)) return serial_sum_nonfinite(get, n, start, s);
            if (s == 0.0f) {
                int fi = KV;
                float fv = 0.0f;
#pragma unroll
                for (int i = KV - 1; i >= 0; i--)
                    if (base + i >= start && x[i] != 0.0f) { fi = i; fv = x[i]; }
                const unsigned long long m = __ballot(fi < KV);
                if (m == 0ull) { start = end; break; }
                const int L = __builtin_ctzll(m);
                s = lane_value(fv, L);
                start = t0 + KV * L + __builtin_amdgcn_readlane(fi, L) + 1;
                continue;
            }
            // s = m * 2^ex with m in [0.5, 1): u = 2^k, binade top B
            const int ex = __builtin_amdgcn_frexp_expf(s);
            const int k = ex - 24 > -149 ? ex - 24 : -149;
            const float B = ex - 1 >= -126 ? __builtin_amdgcn_ldexpf(1.0f, ex) : 0x1p-126f;
            float P[KV];
            bool bad1[KV];
            float run = 0.0f;
            bool any1 = false;
#pragma unroll
            for (int i = 0; i < KV; i++) {
                const bool live = base + i >= start;
                const float q = __builtin_amdgcn_ldexpf(x[i], -k);
                const float r = __builtin_rintf(q);
                bad1[i] = live && (!(x[i] < B) || __builtin_fabsf(q - r) == 0.5f);
                run += live && !bad1[i] ? r : 0.0f;
                P[i] = run;
                any1 = any1 || bad1[i];
            }
            const float incl = wave_scan_add(run);
            const float cand_last = s + __builtin_amdgcn_ldexpf(incl, k);
            const unsigned long long m = __ballot(any1 || !(cand_last < B));
            if (m == 0ull) {
                s = lane_value(cand_last, 63);
                start = end;
                break;
            }
            // the first offending value of each lane (lane L's is the one)
            const int L = __builtin_ctzll(m);
            const float E = incl - run;
            float prev = s + __builtin_amdgcn_ldexpf(E, k);
            int fb = KV;
            float sp = 0.0f, xv = 0.0f;
#pragma unroll
            for (int i = 0; i < KV; i++) {
                const float cand = s + __builtin_amdgcn_ldexpf(E + P[i], k);
                const bool b = bad1[i] || (base + i >= start && !(cand < B));
                if (fb == KV && b) { fb = i; sp = prev; xv = x[i]; }
                prev = cand;
            }
            s = fadd(lane_value(sp, L), lane_value(xv, L));
            start = t0 + KV * L + __builtin_amdgcn_readlane(fb, L) + 1;
        }
    }
    if (!(s <= 0x1.fffffep127f)) return serial_sum_nonfinite(get, n, n, s);
    return s;
}
__device__ __forceinline__ float wave_serial_sum(const float* v, int n, float s0 = 0.0f) {
    return wave_serial_sum_at([v](int i) { return v[i]; }, n, s0);
}

// Orderable 64-bit argmax key: larger key = larger value, ties broken toward
// the smaller index (Sampler::sample_argmax keeps the first maximum,
// sampler.rs:67-79).  The reference starts from row 0 and replaces the
// maximum only on `p > max`, so a NaN in row 0 is never replaced (the
// result is 0) and a NaN elsewhere never wins: row 0's NaN takes the largest
// key, any other NaN the smallest.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    if (v != v) return idx == 0 ? ~0ull : 0ull;
    if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal in the reference
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

}  // namespace yl
