// Shared device helpers for the muon_sr_amd HIP kernels (gfx950 / CDNA4).
//
// bf16 values are handled as raw 16-bit patterns; fp32 arithmetic is IEEE
// binary32 with one rounding per operation (the library is compiled with
// -ffp-contract=off and the default correctly rounded division and sqrt).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/muon_sr_amd.h"

namespace msr {

// ---------------------------------------------------------------------------
// Status plumbing
// ---------------------------------------------------------------------------

// Error codes are the MSR_ERR_* macros of the public header.
constexpr int MSR_OK = 0;

void set_error(const char *fmt, ...);
int check_launch(const char *what);

// ---------------------------------------------------------------------------
// bf16 helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// low half of a packed pair / high half of a packed pair
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Stochastic rounding: add 16 noise bits to the fp32 pattern (wrapping) and keep the high half.
__device__ __forceinline__ uint32_t sr_bf16(float x, uint32_t noise16) {
    return (__float_as_uint(x) + noise16) >> 16;
}

// Round-to-nearest-even fp32 -> bf16 (quiet NaN for NaN inputs).
__device__ __forceinline__ uint32_t rne_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo16, uint32_t hi16) { return (lo16 & 0xffffu) | (hi16 << 16); }

// Two fp32 values rounded to bf16 (nearest even) and packed, lo in bits 0-15:
// one v_cvt_pk_bf16_f32.  Equal to pack2(rne_bf16(lo), rne_bf16(hi)) for every
// fp32 bit pattern, NaNs included (msr_fastmath_check kind 3 tests all 2^32).
typedef __bf16 msr_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float msr_f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t rne_bf16x2(float lo, float hi) {
    const msr_f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, msr_bf16x2_t));
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11), the generator Triton's tl.randint uses.
// ---------------------------------------------------------------------------

constexpr uint32_t PHILOX_KA = 0x9E3779B9u, PHILOX_KB = 0xBB67AE85u;
constexpr uint32_t PHILOX_RA = 0xD2511F53u, PHILOX_RB = 0xCD9E8D57u;

// a ^ b ^ k.  With a wave-uniform key (UKEY) k is taken from an SGPR into one
// v_bitop3_b32; the compiler's two v_xor_b32 would read the SGPR at the slow
// issue rate as well.  A per-lane key (UKEY false) uses plain XORs.
template <bool UKEY>
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t k) {
    if constexpr (UKEY) {
        uint32_t r;
        asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "s"(k));
        return r;
    } else {
        return a ^ b ^ k;
    }
}

template <bool UKEY = true>
__device__ __forceinline__ void philox10(uint32_t &c0, uint32_t &c1, uint32_t &c2, uint32_t &c3,
                                         uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        uint64_t pa = (uint64_t)PHILOX_RA * c0;
        uint64_t pb = (uint64_t)PHILOX_RB * c2;
        uint32_t n0 = xor3<UKEY>((uint32_t)(pb >> 32), c1, k0);
        uint32_t n2 = xor3<UKEY>((uint32_t)(pa >> 32), c3, k1);
        c1 = (uint32_t)pb;
        c3 = (uint32_t)pa;
        c0 = n0;
        c2 = n2;
        k0 += PHILOX_KA;
        k1 += PHILOX_KB;
    }
}

// Word 0 of Philox(ctr = (c0, 0, 0, 0), key).  With c1 = c2 = c3 = 0 the first
// round reduces to c0' = k0, c2' = hi(RA*c0) ^ k1, c1' = 0, c3' = lo(RA*c0).
template <bool UKEY = true>
__device__ __forceinline__ uint32_t philox_w0(uint32_t ctr, uint32_t k0, uint32_t k1) {
    uint64_t pa = (uint64_t)PHILOX_RA * ctr;
    uint32_t c0 = k0, c1 = 0u, c2 = (uint32_t)(pa >> 32) ^ k1, c3 = (uint32_t)pa;
    k0 += PHILOX_KA;
    k1 += PHILOX_KB;
#pragma unroll
    for (int r = 1; r < 9; ++r) {
        uint64_t qa = (uint64_t)PHILOX_RA * c0;
        uint64_t qb = (uint64_t)PHILOX_RB * c2;
        uint32_t n0 = xor3<UKEY>((uint32_t)(qb >> 32), c1, k0);
        uint32_t n2 = xor3<UKEY>((uint32_t)(qa >> 32), c3, k1);
        c1 = (uint32_t)qb;
        c3 = (uint32_t)qa;
        c0 = n0;
        c2 = n2;
        k0 += PHILOX_KA;
        k1 += PHILOX_KB;
    }
    // last round: only word 0 is needed
    return xor3<UKEY>((uint32_t)(((uint64_t)PHILOX_RB * c2) >> 32), c1, k0);
}

// Philox key of Triton's `SEED + k` stream.  A compiled Triton launch types an
// int argument i32 in [-2^31, 2^31) and i64 in [2^31, 2^63); SEED + k is
// evaluated in that type, then widened to u64 (sign-extended for i32) and split
// into (lo, hi) (triton/language/random.py:49-60).
struct PhiloxKey {
    uint32_t lo, hi;
};

__host__ __device__ inline PhiloxKey seed_key(uint32_t seed, uint32_t k) {
    PhiloxKey key;
    if (seed < 0x80000000u) {
        key.lo = seed + k;
        key.hi = (key.lo >= 0x80000000u) ? 0xffffffffu : 0u;
    } else {
        uint64_t v = (uint64_t)seed + k;
        key.lo = (uint32_t)v;
        key.hi = (uint32_t)(v >> 32);
    }
    return key;
}

// ---------------------------------------------------------------------------
// Noise sources for one stochastic-rounding stream
// ---------------------------------------------------------------------------

enum NoiseMode : int {
    NOISE_TRITON = 0,   // word 0 of Philox((offset mod 2^32, 0, 0, 0), key): the reference's noise
    NOISE_PHILOX8 = 1,  // one Philox call per 8 consecutive offsets, 16-bit lane (offset & 7)
    NOISE_INJECT = 2    // caller-provided uint16 noise, indexed by offset (tests)
};

struct Noise {
    PhiloxKey key;
    const uint16_t *inject;
};

// 16 noise bits for each of the 8 offsets o0 .. o0+7 (o0 a multiple of 8 when
// MODE == NOISE_PHILOX8).  `valid` counts the offsets that exist (<= 8).
// UKEY: the key is the same in every lane of the wave.
template <int MODE, bool UKEY = true>
__device__ __forceinline__ void noise8(const Noise &ns, int64_t o0, int valid, uint32_t out[8]) {
    if constexpr (MODE == NOISE_TRITON) {
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = philox_w0<UKEY>((uint32_t)(o0 + j), ns.key.lo, ns.key.hi) & 0xffffu;
    } else if constexpr (MODE == NOISE_PHILOX8) {
        uint64_t o = (uint64_t)o0;
        uint32_t c0 = (uint32_t)(o >> 3), c1 = (uint32_t)(o >> 35), c2 = 0u, c3 = 0u;
        philox10<UKEY>(c0, c1, c2, c3, ns.key.lo, ns.key.hi);
        out[0] = c0 & 0xffffu; out[1] = c0 >> 16;
        out[2] = c1 & 0xffffu; out[3] = c1 >> 16;
        out[4] = c2 & 0xffffu; out[5] = c2 >> 16;
        out[6] = c3 & 0xffffu; out[7] = c3 >> 16;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (j < valid) ? (uint32_t)ns.inject[o0 + j] : 0u;
    }
}

// Noise for a single offset (scalar fallback paths).
template <int MODE, bool UKEY = true>
__device__ __forceinline__ uint32_t noise1(const Noise &ns, int64_t o) {
    if constexpr (MODE == NOISE_TRITON) {
        return philox_w0<UKEY>((uint32_t)o, ns.key.lo, ns.key.hi) & 0xffffu;
    } else if constexpr (MODE == NOISE_PHILOX8) {
        uint64_t u = (uint64_t)o;
        uint32_t c0 = (uint32_t)(u >> 3), c1 = (uint32_t)(u >> 35), c2 = 0u, c3 = 0u;
        philox10<UKEY>(c0, c1, c2, c3, ns.key.lo, ns.key.hi);
        uint32_t lane = (uint32_t)(u & 7u);
        uint32_t w = (lane < 2) ? c0 : (lane < 4) ? c1 : (lane < 6) ? c2 : c3;
        return (w >> (16u * (lane & 1u))) & 0xffffu;
    } else {
        return ns.inject[o];
    }
}

// ---------------------------------------------------------------------------
// Muon momentum (muon_sr/triton_muon_sr.py:37-42): the new momentum nb (stored with
// SR) and the pre-Newton-Schulz update (stored RNE), in the reference's fp32 order.
// ---------------------------------------------------------------------------
template <bool NEST>
__device__ __forceinline__ void muon_momentum(float g, float b, float beta, float one_m_beta, float &nb,
                                              float &upd) {
    nb = b + one_m_beta * (g - b);            // :37
    upd = NEST ? g + beta * (nb - g) : nb;    // :39-42
}

// ---------------------------------------------------------------------------
// 8-bit quantizer
// ---------------------------------------------------------------------------

// The reference quantizer search (muon_sr/triton_adamw_8bit.py:27-53): seven
// halvings from pivot 127 against the sorted codebook Q, then the midpoint rule
// with the last bounds (initial bounds -1/0 and +1), then the sign fix for the
// signed map.  Compiled for host (table construction) and device.
__host__ __device__ inline uint32_t quantize_search(float x, const float *Q, bool is_signed) {
    int pivot = 127, lower_pivot = 0, upper_pivot = 255;
    float lower = is_signed ? -1.0f : 0.0f;
    float upper = 1.0f;
    float val = Q[pivot];
#pragma unroll
    for (int shift = 0; shift < 7; ++shift) {
        const int delta = 64 >> shift;
        const bool right = x > val;
        lower_pivot = right ? pivot : lower_pivot;
        upper_pivot = right ? upper_pivot : pivot;
        lower = right ? val : lower;
        upper = right ? upper : val;
        pivot += right ? delta : -delta;
        val = Q[pivot];
    }
    int result;
    if (x > val) result = (x > (upper + val) * 0.5f) ? upper_pivot : pivot;
    else result = (x < (lower + val) * 0.5f) ? lower_pivot : pivot;
    if (is_signed) {
        const float decoded = Q[result];
        const bool mismatch = (decoded < 0.0f) != (x < 0.0f);
        result += mismatch ? ((x > 0.0f) ? 1 : -1) : 0;
    }
    return (uint32_t)result & 0xffu;
}

// Bucketed threshold table equivalent to quantize_search for one pair of
// codebooks (built by msr_quant_table_build).  For a float x with bit pattern
// u (|x| <= 1 or NaN), map base mb (0: signed map, 512: unsigned map), the
// octave word o = oct[mb + (u >> 23)] (sign and exponent) and
//     b = (o >> 8) + ((u & 0x7fffff) >> (o & 31)),
//     code = ((u & 0x7fffffff) >= bkt[b].x) ? bkt[b].y >> 8 : bkt[b].y & 0xff.
// Each bucket holds at most one point where the code changes; exponent 255
// (NaN) points at a bucket holding the search's NaN code.
constexpr int QT_OCT = 2 * 512;
constexpr int QT_MAX_BKT = 2048;

// One-level table for the fast kernel (standard codebooks).  A quotient x with
// bit pattern u, |x| <= 1, is looked up through w = (u ^ s) >> 16 and the low
// half (u ^ s) & 0xffff, where s = 0 for x >= 0 and all ones for x < 0: for
// x >= 0, w is the bucket key (exponent and 7 mantissa bits); for x < 0 both
// are complemented, so w = 0x7fff - key and the codes (which fall as |x|
// grows) rise with w and with the low half.  Entry idx = min(max(w - LO1, 0),
// QF_SCAP) with LO1 = QF_LO_KEY - 1:
//   signed plane   [0, QF_N)            x >= 0: key - LO1 (0: x < 2^-23)
//                  [QF_NEG0, QF_SCAP)   x < 0, |x| >= 2^-23: 0x7fff - key - LO1
//                  QF_SCAP              x < 0, |x| < 2^-23
//   unsigned plane [0, QF_N)            key - LO1 (0: x < 2^-23)
// Each bucket holds at most one code change (checked when the table is
// built), so an entry is
//     bits 0-15: c = 0x10000 - (low half at the change point), or 0
//     bits 16-23: code at the bucket's low end
// and code = ((low half + entry) >> 16) & 0xff: the carry adds the step.
constexpr uint32_t QF_LO_KEY = 104u << 7;                         // 2^-23
constexpr uint32_t QF_LO1 = QF_LO_KEY - 1u;
constexpr int QF_N = (int)((127u << 7) - QF_LO1) + 1;            // 2946 (1.0 is the last key)
constexpr int QF_NEG0 = (int)(0x7fffu - (127u << 7) - QF_LO1);   // 3200
constexpr int QF_SCAP = (int)(0x7fffu - QF_LO_KEY - QF_LO1) + 1; // 6145
constexpr int QF_SIGNED = QF_SCAP + 1;                           // signed plane entries
constexpr int QF_TOTAL = QF_SIGNED + QF_N;                       // both planes

struct QuantTable {
    uint32_t n_bkt;
    uint32_t pad[3];
    uint32_t oct[QT_OCT];
    uint2 bkt[QT_MAX_BKT];
    uint32_t flat[QF_TOTAL];
};

__host__ __device__ inline uint32_t quantize_lookup(float x, const uint32_t *oct, const uint2 *bkt, bool is_signed) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t o = oct[(is_signed ? 0u : 512u) + (u >> 23)];
    const uint2 en = bkt[(o >> 8) + ((u & 0x7fffffu) >> (o & 31u))];
    return (en.y >> (((u & 0x7fffffffu) >= en.x) ? 8u : 0u)) & 0xffu;
}

// m / d for the signed map: x = RN_f32(m / d) up to the distinction the
// signed codebook cannot make (every nonzero |x| < FLT_MIN of one sign codes
// alike), for d > 0 (or +inf), rd = RN_f64(1 / d) and dlim = min(d * 2^-150, DBL_MAX).
// In the normal range (float)(m * rd) is exact: an fp32 quotient is never an
// fp32 rounding midpoint (a midpoint needs 25 significant bits) and its
// distance to one (>= 2^-50 relative) exceeds the double product's error
// (<= 2^-52 relative).  Whether RN_f32(m / d) is zero is decided exactly:
// |m| <= d * 2^-150 (ties go to the even zero).
__device__ __forceinline__ float quotient_signed(float m, double rd, double dlim) {
    const float x = (float)((double)m * rd);
    const bool nz = !(fabs((double)m) <= dlim);  // true for NaN and for inf / inf
    const float tiny = copysignf(0x1p-149f, m);
    return nz ? ((x == 0.0f) ? tiny : x) : 0.0f;
}

// v / d for the unsigned map (v >= 0): below FLT_MIN every value, zero
// included, codes to 0, so the double product alone decides the code.
__device__ __forceinline__ float quotient_unsigned(float v, double rd) { return (float)((double)v * rd); }

// ---------------------------------------------------------------------------
// Correctly rounded fp32 building blocks for a stated input range.
//
// Measured on gfx950 (ns per wave64 instruction per SIMD): fp32 add/mul/fma and
// integer add/and/or/xor/shift-right issue at ~1.05; any instruction with an
// SGPR operand, max/min, compares, selects, v_perm, SDWA forms and f64 at
// ~1.8; v_sqrt_f32/v_rcp_f32 at 3.4.  These sequences use the fast class where
// the IEEE library sequences use compares, selects and range scaling.  Each is
// checked against the IEEE operation over its whole input range on the GPU
// (msr_fastmath_check).
// ---------------------------------------------------------------------------

// Work-group b of a grid of g -> its place in the work order.  Consecutive work-groups
// are dispatched over the 8 XCDs in turn; each run of 8 K work-groups takes 8 runs of K
// consecutive places, one run per XCD, so neighbouring work is done from one XCD's L2
// (K = 0: places in dispatch order; work-groups past the last whole run keep theirs).
__device__ __forceinline__ int64_t xcd_place(int64_t b, int64_t g, int64_t K) {
    if (K <= 0 || b >= g / (8 * K) * (8 * K)) return b;
    const int64_t r = b % (8 * K);
    return b - r + (r & 7) * K + (r >> 3);
}

// Opaque VGPR copy of a wave-uniform value, so arithmetic with it keeps the
// fast issue rate (the compiler would otherwise read kernel arguments as SGPRs).
__device__ __forceinline__ float vgpr(float x) {
    float r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}
__device__ __forceinline__ uint32_t vgpr(uint32_t x) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}

// sqrt(v) correctly rounded, for v == +0 or v in [2^-149, 2^62].  v_sqrt_f32
// (within 1 ulp) runs on v * 2^64, which is >= 2^-85, where the residuals
// fma(s -+ 1ulp, s, -v) are exact; the root moves down a step when
// v <= (s - 1ulp) * s and up a step when v > (s + 1ulp) * s, as in the IEEE
// sequence, read off the residuals' sign bits.  At v = 0, s - 1ulp saturates to
// 0 and both residuals are +0.  sqrt_rn_x2p32 returns the root of v * 2^64,
// i.e. 2^32 * sqrt(v), whose unscaling by 2^-32 is exact (the root of v * 2^64
// is 0 or >= 2^-42.5): fma(sqrt_rn_x2p32(v), 2^-32, e) == sqrt_rn(v) + e.
__device__ __forceinline__ float sqrt_rn_x2p32(float v) {
    const float vs = v * 0x1p64f;
    const float s = __builtin_amdgcn_sqrtf(vs);
    const uint32_t sb = __float_as_uint(s);
    const uint32_t sdn = __builtin_elementwise_sub_sat(sb, 1u);
    const float rdn = __builtin_fmaf(__uint_as_float(sdn), s, -vs);
    const float rup = __builtin_fmaf(__uint_as_float(sb + 1u), s, -vs);
    return __uint_as_float(sdn + (__float_as_uint(rdn) >> 31) + (__float_as_uint(rup) >> 31));
}
__device__ __forceinline__ float sqrt_rn(float v) { return sqrt_rn_x2p32(v) * 0x1p-32f; }

// RN(1/d) for d in [2^-60, 2^32): v_rcp_f32 and one Newton step.
__device__ __forceinline__ float rcp_rn(float d) {
    const float r0 = __builtin_amdgcn_rcpf(d);
    const float e = __builtin_fmaf(-d, r0, 1.0f);
    return __builtin_fmaf(e, r0, r0);
}

// RN(m/d) from y = RN(1/d) (Markstein): q0 = RN(m*y) is within an ulp of m/d,
// the remainder m - d*q0 is exact while it is a normal number, and
// RN(q0 + r*y) is then the rounded quotient: for d in [2^-60, 2) and
// |m| in [2^-100, d].  For smaller |m| the quotient keeps m's sign and is +0
// for m = +-0, which is all the codes need there: with d >= 2^-60 such an
// |x| = |m/d| is below 2^-23, where every x of one sign codes alike.
__device__ __forceinline__ float div_rn(float m, float d, float y) {
    const float q0 = m * y;
    const float r = __builtin_fmaf(-q0, d, m);
    return __builtin_fmaf(r, y, q0);
}

// RN(n/d) for the update's quotient, for d in [2^-60, 2^32) and n = +-0 or
// |n| in [2^-90, 2^60] (so the quotient is a normal number or zero).  With
// y = RN(1/d) and q0 = RN(n*y) within an ulp of n/d, the negated remainder
// d*q0 - n is exact (|n| >= 2^-90 keeps it out of the subnormal range) and
// RN(q0 - (d*q0 - n)*y) is the rounded quotient (Markstein's theorem).  The
// negated form also gives the IEEE sign of a zero quotient: for n = -0 it is
// -0 (the plain remainder n - d*q0 = +0 would turn it into +0).
__device__ __forceinline__ float div_upd(float n, float d) {
    const float y = rcp_rn(d);
    const float q0 = n * y;
    const float rn = __builtin_fmaf(d, q0, -n);
    return __builtin_fmaf(-rn, y, q0);
}

// Signed code of x = RN(m/d) for the fast kernel (x != -0, |x| <= 1), as the
// entry sum whose bits 16-23 are the code; `tab` is the signed plane, lo1 and
// scap are VGPR copies of QF_LO1 and QF_SCAP (an SGPR or literal operand of the
// saturating subtract would take the slow issue rate).
__device__ __forceinline__ uint32_t qf_signed(float x, const uint32_t *tab, uint32_t lo1, uint32_t scap) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t uc = u ^ (uint32_t)((int32_t)u >> 31);
    const uint32_t idx = min(__builtin_elementwise_sub_sat(uc >> 16, lo1), scap);
    return (uc & 0xffffu) + tab[idx];
}

// Unsigned code of x in [0, 1] (x != -0); `tab` is the unsigned plane.
__device__ __forceinline__ uint32_t qf_unsigned(float x, const uint32_t *tab, uint32_t lo1) {
    const uint32_t u = __float_as_uint(x);
    return (u & 0xffffu) + tab[__builtin_elementwise_sub_sat(u >> 16, lo1)];
}

// Bytes 2 of four entry sums, packed into one little-endian code word.
__device__ __forceinline__ uint32_t pack_codes(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3) {
    const uint32_t lo = __builtin_amdgcn_perm(r1, r0, 0x0c0c0602u);   // [r0.b2, r1.b2, 0, 0]
    const uint32_t hi = __builtin_amdgcn_perm(r3, r2, 0x06020c0cu);   // [0, 0, r2.b2, r3.b2]
    return lo | hi;
}

// Maxima of two non-negative, NaN-free fp32 values over each 32-lane half of a
// wave64 (integer order equals float order there).  Rows of 16 lanes reduce
// with DPP (quad_perm [1,0,3,2] and [2,3,0,1], row_ror 4 and 8); then
// v_permlane16_swap(a, b) returns rows (a0, b0, a2, b2) and (a1, b1, a3, b3), so
// one swap and a max leave rows (A01, B01, A23, B23), and a swap of that value
// with itself spreads A and B over both rows of their half.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t x) {
    return max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, true));
}

__device__ __forceinline__ void halfwave_max2(float &a, float &b) {
    uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
    x = dpp_max_u32<0xB1>(x); y = dpp_max_u32<0xB1>(y);
    x = dpp_max_u32<0x4E>(x); y = dpp_max_u32<0x4E>(y);
    x = dpp_max_u32<0x124>(x); y = dpp_max_u32<0x124>(y);
    x = dpp_max_u32<0x128>(x); y = dpp_max_u32<0x128>(y);
    const auto s = __builtin_amdgcn_permlane16_swap(x, y, false, false);
    const uint32_t c = max((uint32_t)s[0], (uint32_t)s[1]);
    const auto t = __builtin_amdgcn_permlane16_swap(c, c, false, false);
    a = __uint_as_float(t[0]);
    b = __uint_as_float(t[1]);
}

inline bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Host-side race check: the byte ranges [a, a + na) and [b, b + nb) overlap
// without being the same buffer.  Identical ranges are in-place use, which the
// element-wise kernels allow (each element is read before it is written by the
// same thread); any other overlap would let one element's write race another's
// read.
inline bool partial_overlap(const void *a, size_t na, const void *b, size_t nb) {
    if (!a || !b || na == 0 || nb == 0) return false;
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    if (x == y && na == nb) return false;
    return x < y + nb && y < x + na;
}


// Grid size for a grid-stride loop over `work` items with `threads` per block.
inline unsigned grid_for(int64_t work, int threads, int64_t cap = 256 * 32) {
    int64_t b = (work + threads - 1) / threads;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return (unsigned)b;
}

}  // namespace msr

// Noise-mode dispatch for a templated launcher.
#define MSR_DISPATCH_NOISE(mode, M, ...)                                        \
    switch (mode) {                                                             \
    case msr::NOISE_TRITON: { constexpr int M = msr::NOISE_TRITON; __VA_ARGS__; break; } \
    case msr::NOISE_PHILOX8: { constexpr int M = msr::NOISE_PHILOX8; __VA_ARGS__; break; } \
    case msr::NOISE_INJECT: { constexpr int M = msr::NOISE_INJECT; __VA_ARGS__; break; } \
    default: msr::set_error("unknown noise mode %d", (int)(mode)); return MSR_ERR_ARG; \
    }
