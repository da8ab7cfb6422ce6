// 8-bit blockwise AdamW for gfx950 (muon_sr/triton_adamw_8bit.py:27-99): the fused
// quantized step, the bf16-moment step of excluded tensors, the quantizer
// diagnostics and the quantizer tables.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <utility>
#include <vector>

#include "common.hpp"
#include "vecio.hpp"
#include "../../include/muon_sr_amd.h"

namespace msr {

// ---------------------------------------------------------------------------
// 8-bit blockwise AdamW   (muon_sr/triton_adamw_8bit.py:27-99)
// ---------------------------------------------------------------------------

struct Adam8Args {
    uint16_t *p;
    const uint16_t *g;
    void *s1;
    void *s2;
    float *absmax1;
    float *absmax2;
    const float *qmap1;
    const float *qmap2;
    const QuantTable *qtable;
    int64_t n;
    int64_t qb0;   // first quantization block this launch handles (the rest of the tensor is done elsewhere)
    float lr, b1, b2, eps, wd, bc1, bc2;
    Noise ns_p, ns_m, ns_v;
};

struct Adam8Consts {
    float one_m_b1, one_m_b2, step_c, eps_c, decay;
};

__device__ __forceinline__ Adam8Consts adam8_consts(const Adam8Args &a) {
    Adam8Consts c;
    c.one_m_b1 = 1.0f - a.b1;
    c.one_m_b2 = 1.0f - a.b2;
    const float sqrt_bc2 = sqrtf(a.bc2);
    c.step_c = (a.lr * sqrt_bc2) / a.bc1;     // :74  LR * sqrt(BC2) / BC1
    c.eps_c = sqrt_bc2 * a.eps;               // :74  sqrt(BC2) * EPS
    c.decay = 1.0f - a.lr * a.wd;             // :74  (1 - LR * WD)
    return c;
}

// Threads per quantization block: BLOCK/8.  Work-group size: max(256, BLOCK/8).
// QTAB: requantize through the bucketed threshold table (standard codebooks),
// else through the reference search; both give the search's codes.
template <int MODE, int BLOCK, bool VEC, bool QTAB>
__global__ __launch_bounds__((BLOCK / 8 > THREADS) ? BLOCK / 8 : THREADS) void adamw8bit_quant_kernel(Adam8Args a) {
    constexpr int TPB = BLOCK / 8;
    constexpr int WG = TPB > THREADS ? TPB : THREADS;
    constexpr int QB_PER_WG = WG / TPB;
    constexpr int NWAVES = WG / 64;
    __shared__ float q1s[256], q2s[256];
    __shared__ float red_m[NWAVES], red_v[NWAVES];
    __shared__ uint32_t s_oct[QTAB ? QT_OCT : 1];
    __shared__ uint2 s_bkt[QTAB ? QT_MAX_BKT : 1];
    for (int i = threadIdx.x; i < 256; i += WG) {
        q1s[i] = a.qmap1[i];
        q2s[i] = a.qmap2[i];
    }
    if constexpr (QTAB) {
        const uint32_t nb = a.qtable->n_bkt;
        for (int i = threadIdx.x; i < QT_OCT; i += WG) s_oct[i] = a.qtable->oct[i];
        for (uint32_t i = threadIdx.x; i < nb; i += WG) s_bkt[i] = a.qtable->bkt[i];
    }
    __syncthreads();
    const Adam8Consts c = adam8_consts(a);
    uint8_t *m8 = static_cast<uint8_t *>(a.s1);
    uint8_t *v8 = static_cast<uint8_t *>(a.s2);
    const int64_t nblocks = (a.n + BLOCK - 1) / BLOCK;
    const int sub = threadIdx.x / TPB;       // quant block within the work-group
    const int lane_q = threadIdx.x % TPB;    // thread within the quant block
    const int64_t stride = (int64_t)gridDim.x * QB_PER_WG;

    // raw inputs of one 8-element group; the next group is fetched while the
    // current one is computed
    struct Raw {
        uint32_t wp[4], wg[4];
        uint2 mc, vc;
        float ms, vs;
    };
    auto fetch = [&](int64_t qb, Raw &r) {
        const bool ok = qb < nblocks;
        const int64_t o0 = qb * BLOCK + lane_q * 8;
        const int valid = ok ? clamp_valid(a.n, o0) : 0;
        load_bf16x8<VEC>(a.p, o0, valid, r.wp);
        load_bf16x8<VEC>(a.g, o0, valid, r.wg);
        if (VEC && valid == 8) {
            const u32x2_t mc = ld_nt2(m8 + o0), vc = ld_nt2(v8 + o0);
            r.mc = make_uint2(mc.x, mc.y);
            r.vc = make_uint2(vc.x, vc.y);
        } else {
            uint32_t cm[8], cv[8];
            load_u8x8<false>(m8, o0, valid, 127u, cm);
            load_u8x8<false>(v8, o0, valid, 0u, cv);
            r.mc = make_uint2(cm[0] | cm[1] << 8 | cm[2] << 16 | cm[3] << 24, cm[4] | cm[5] << 8 | cm[6] << 16 | cm[7] << 24);
            r.vc = make_uint2(cv[0] | cv[1] << 8 | cv[2] << 16 | cv[3] << 24, cv[4] | cv[5] << 8 | cv[6] << 16 | cv[7] << 24);
        }
        r.ms = ok ? a.absmax1[qb] : 0.0f;
        r.vs = ok ? a.absmax2[qb] : 0.0f;
    };

    int64_t qb = a.qb0 + (int64_t)blockIdx.x * QB_PER_WG + sub;
    Raw nxt;
    fetch(qb, nxt);
    for (int64_t qb0 = a.qb0 + (int64_t)blockIdx.x * QB_PER_WG; qb0 < nblocks; qb0 += stride, qb += stride) {
        const Raw cur = nxt;
        if (qb0 + stride < nblocks) fetch(qb + stride, nxt);
        const bool qb_ok = qb < nblocks;
        const int64_t o0 = qb * BLOCK + lane_q * 8;
        const int valid = qb_ok ? clamp_valid(a.n, o0) : 0;
        float p[8], g[8], m[8], v[8];
        unpack8(cur.wp, p);
        unpack8(cur.wg, g);
        uint32_t rp[8];
        noise8<MODE>(a.ns_p, o0, valid, rp);
        float mmax = 0.0f, vmax = 0.0f;
        uint32_t op[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t mcj = ((j < 4 ? cur.mc.x : cur.mc.y) >> (8 * (j & 3))) & 0xffu;
            const uint32_t vcj = ((j < 4 ? cur.vc.x : cur.vc.y) >> (8 * (j & 3))) & 0xffu;
            float mj = q1s[mcj] * cur.ms;                                 // :65
            float vj = q2s[vcj] * cur.vs;                                 // :66
            const bool fin = fabsf(g[j]) < __builtin_huge_valf();         // :70
            mj = fin ? a.b1 * mj + c.one_m_b1 * g[j] : 0.0f;              // :71
            vj = fin ? a.b2 * vj + (c.one_m_b2 * g[j]) * g[j] : 0.0f;     // :72
            const float upd = (p[j] - (c.step_c * mj) / (sqrtf(vj) + c.eps_c)) * c.decay;  // :74
            const uint32_t pin = (j & 1) ? (cur.wp[j >> 1] >> 16) : (cur.wp[j >> 1] & 0xffffu);
            op[j] = fin ? sr_bf16(upd, rp[j]) : pin;                      // :75-78
            m[j] = mj;
            v[j] = vj;
            if (j < valid) {
                mmax = fmaxf(mmax, fabsf(mj));
                vmax = fmaxf(vmax, fabsf(vj));
            }
        }
        uint32_t wo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) wo[j] = pack2(op[2 * j], op[2 * j + 1]);
        store_bf16x8<VEC>(a.p, o0, valid, wo);

        // block absmax (:80-81): shuffles inside the wave, LDS across waves
#pragma unroll
        for (int off = (TPB < 64 ? TPB : 64) / 2; off >= 1; off >>= 1) {
            mmax = fmaxf(mmax, __shfl_xor(mmax, off, 64));
            vmax = fmaxf(vmax, __shfl_xor(vmax, off, 64));
        }
        if constexpr (TPB > 64) {
            constexpr int WPQ = TPB / 64;  // waves per quant block
            const int wave = threadIdx.x / 64;
            if ((threadIdx.x & 63) == 0) {
                red_m[wave] = mmax;
                red_v[wave] = vmax;
            }
            __syncthreads();
            const int w0 = (wave / WPQ) * WPQ;
            mmax = red_m[w0];
            vmax = red_v[w0];
#pragma unroll
            for (int w = 1; w < WPQ; ++w) {
                mmax = fmaxf(mmax, red_m[w0 + w]);
                vmax = fmaxf(vmax, red_v[w0 + w]);
            }
            __syncthreads();
        }
        const float md = mmax > 0.0f ? mmax : 1.0f;                       // :82
        const float vd = vmax > 0.0f ? vmax : 1.0f;                       // :83
        const double rmd = 1.0 / (double)md;
        const double rvd = 1.0 / (double)vd;
        const double mlim = fmin((double)md * 0x1p-150, 1.7976931348623157e308);
        uint32_t mc[8], vc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float xm = quotient_signed(m[j], rmd, mlim);            // m / md, :82
            const float xv = quotient_unsigned(v[j], rvd);                // v / vd, :83
            if constexpr (QTAB) {
                mc[j] = quantize_lookup(xm, s_oct, s_bkt, true);          // :84
                vc[j] = quantize_lookup(xv, s_oct, s_bkt, false);         // :85
            } else {
                mc[j] = quantize_search(xm, q1s, true);
                vc[j] = quantize_search(xv, q2s, false);
            }
        }
        store_u8x8<VEC>(m8, o0, valid, mc);
        store_u8x8<VEC>(v8, o0, valid, vc);
        if (qb_ok && lane_q == 0) {
            a.absmax1[qb] = mmax;                                         // :86
            a.absmax2[qb] = vmax;                                         // :87
        }
    }
}

// ---------------------------------------------------------------------------
// Fast 8-bit step: block 256, standard codebooks, full 16-byte-aligned blocks.
//
// A wave owns two quantization blocks (64 lanes x 8 elements) per iteration
// and walks the tensor in a grid-stride loop, fetching its next pair while it
// computes the current one.  Per pair the wave first forms the new moments and
// the two block maxima, then takes one of two branches, uniformly:
//  * fast: every gradient finite, max v' < 2^62, both block divisors in
//    [2^-60, 2) and every update numerator |step_c * m'| zero or in
//    [2^-90, 2^60).  The update uses sqrt_rn and div_upd, the requantization
//    quotients use rcp_rn/div_rn and the codes come from the flat table; all of
//    these equal the IEEE operations on these ranges (see common.hpp);
//  * exact: anything else (non-finite gradients, extreme moments) goes through
//    the reference arithmetic with IEEE sqrt/division, the double-precision
//    quotients and the reference search, as in adamw8bit_quant_kernel.
// Both branches produce the reference's bits; the fast one with about half
// the VALU work.
// ---------------------------------------------------------------------------

#ifndef MSR_F8_WAVES
#define MSR_F8_WAVES 4
#endif
#ifndef MSR_F8_NP
#define MSR_F8_NP 1
#endif
constexpr int F8_THREADS = 64 * MSR_F8_WAVES;
constexpr int F8_NP = MSR_F8_NP;             // adjacent pairs a wave takes per iteration
constexpr int F8_PAIR = 512;                 // elements of a pair (2 blocks of 256: 64 lanes x 8)
constexpr int F8_DEFER = 64;                 // pairs a wave defers to its exact pass before flushing

struct Raw8 {
    u32x4_t p, g;
    u32x2_t mc, vc;
    float ms, vs;
};

__device__ __forceinline__ uint32_t byte_of(u32x2_t w, int j) { return ((j < 4 ? w.x : w.y) >> (8 * (j & 3))) & 0xffu; }
__device__ __forceinline__ float bf16_at(u32x4_t w, int j) {
    const uint32_t x = (j >> 1) == 0 ? w.x : (j >> 1) == 1 ? w.y : (j >> 1) == 2 ? w.z : w.w;
    return (j & 1) ? bf16_hi(x) : bf16_lo(x);
}

// Word k (0..3) of a 4-word vector, and the vector with word k replaced, for a
// loop index k: selects, so the rolled loops below keep everything in registers.
__device__ __forceinline__ uint32_t word_at(u32x4_t w, int k) { return k == 0 ? w.x : k == 1 ? w.y : k == 2 ? w.z : w.w; }
__device__ __forceinline__ u32x4_t with_word(u32x4_t w, int k, uint32_t x) {
    w.x = k == 0 ? x : w.x;
    w.y = k == 1 ? x : w.y;
    w.z = k == 2 ? x : w.z;
    w.w = k == 3 ? x : w.w;
    return w;
}

// The reference arithmetic for one full pair: the rare branch of the fast
// kernel.  Element loops stay rolled and the moments are recomputed for the
// requantization pass, so this branch needs fewer registers than the fast one
// and does not lower the kernel's occupancy.
template <int MODE>
__device__ __forceinline__ void adam8_pair_exact(const Adam8Args &a, const Raw8 &cur, int64_t o0, int64_t qb,
                                                 const float *q1s, const float *q2s) {
    const Adam8Consts c = adam8_consts(a);
    uint8_t *m8 = static_cast<uint8_t *>(a.s1);
    uint8_t *v8 = static_cast<uint8_t *>(a.s2);
    // moments of element j, with non-finite gradients masked (:65-72)
    auto moments = [&](int j, float &mj, float &vj, float &gj, bool &fin) {
        const uint32_t gw = word_at(cur.g, j >> 1);
        gj = (j & 1) ? bf16_hi(gw) : bf16_lo(gw);
        mj = q1s[byte_of(cur.mc, j)] * cur.ms;                               // :65
        vj = q2s[byte_of(cur.vc, j)] * cur.vs;                               // :66
        fin = fabsf(gj) < __builtin_huge_valf();                             // :70
        mj = fin ? a.b1 * mj + c.one_m_b1 * gj : 0.0f;                       // :71
        vj = fin ? a.b2 * vj + (c.one_m_b2 * gj) * gj : 0.0f;                // :72
    };
    float mmax = 0.0f, vmax = 0.0f;
    u32x4_t pout = cur.p;
#pragma unroll 1
    for (int j = 0; j < 8; ++j) {
        float mj, vj, gj;
        bool fin;
        moments(j, mj, vj, gj, fin);
        const uint32_t pw = word_at(cur.p, j >> 1);
        const float pj = (j & 1) ? bf16_hi(pw) : bf16_lo(pw);
        const float upd = (pj - (c.step_c * mj) / (sqrtf(vj) + c.eps_c)) * c.decay;   // :74
        const uint32_t op = fin ? sr_bf16(upd, noise1<MODE>(a.ns_p, o0 + j)) : ((pw >> (16 * (j & 1))) & 0xffffu);  // :75-78
        const uint32_t ow = word_at(pout, j >> 1);
        pout = with_word(pout, j >> 1, (j & 1) ? ((ow & 0xffffu) | (op << 16)) : ((ow & 0xffff0000u) | op));
        mmax = fmaxf(mmax, fabsf(mj));
        vmax = fmaxf(vmax, fabsf(vj));
    }
    st_nt4(a.p + o0, pout);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {                                // :80-81
        mmax = fmaxf(mmax, __shfl_xor(mmax, off, 64));
        vmax = fmaxf(vmax, __shfl_xor(vmax, off, 64));
    }
    const float md = mmax > 0.0f ? mmax : 1.0f;                              // :82
    const float vd = vmax > 0.0f ? vmax : 1.0f;                              // :83
    const double rmd = 1.0 / (double)md, rvd = 1.0 / (double)vd;
    const double mlim = fmin((double)md * 0x1p-150, 1.7976931348623157e308);
    uint32_t mc0 = 0, mc1 = 0, vc0 = 0, vc1 = 0;
#pragma unroll 1
    for (int j = 0; j < 8; ++j) {
        float mj, vj, gj;
        bool fin;
        moments(j, mj, vj, gj, fin);
        const uint32_t mc = quantize_search(quotient_signed(mj, rmd, mlim), q1s, true);     // :82,84
        const uint32_t vc = quantize_search(quotient_unsigned(vj, rvd), q2s, false);        // :83,85
        const uint32_t sh = 8u * (uint32_t)(j & 3);
        if (j < 4) { mc0 |= mc << sh; vc0 |= vc << sh; } else { mc1 |= mc << sh; vc1 |= vc << sh; }
    }
    st_nt2(m8 + o0, u32x2_t{mc0, mc1});
    st_nt2(v8 + o0, u32x2_t{vc0, vc1});
    if ((threadIdx.x & 31) == 0) {
        a.absmax1[qb] = mmax;                                                // :86
        a.absmax2[qb] = vmax;                                                // :87
    }
}

// Wave-uniform constants of the fast branch, held in VGPRs (see vgpr()).
struct F8Consts {
    float b1, omb1, b2, omb2, step_c, eps_c, decay, step_abs;
    uint32_t lo1, scap;
    int32_t tm1;
};

__device__ __forceinline__ F8Consts f8_consts(const Adam8Args &a) {
    const Adam8Consts c = adam8_consts(a);
    F8Consts k;
    k.b1 = vgpr(a.b1); k.omb1 = vgpr(c.one_m_b1); k.b2 = vgpr(a.b2); k.omb2 = vgpr(c.one_m_b2);
    k.step_c = vgpr(c.step_c); k.eps_c = vgpr(c.eps_c); k.decay = vgpr(c.decay);
    k.lo1 = vgpr(QF_LO1); k.scap = vgpr((uint32_t)QF_SCAP);
    // div_upd(step_c * m, den) needs |step_c * m| = 0 or in [2^-90, 2^60]: nonzero |m| below
    // tm = 2^-90 / |step_c| (tm1 = bits(tm) - 1) or |step_c| * max |m| >= 2^60 take the exact
    // branch (den is in [2^-60, 2^32): eps_c is checked by the launcher, v' < 2^62 below)
    k.step_abs = vgpr(fabsf(c.step_c));
    k.tm1 = (int32_t)vgpr(c.step_c != 0.0f ? __float_as_uint(0x1p-90f / fabsf(c.step_c)) - 1u : 0u);
    return k;
}

// NP adjacent pairs of quantization blocks (pair pr0 + q: the wave's 64 lanes x 8 elements)
// on the fast branch.  Returns the mask of the pairs done; a pair whose bit is clear needs
// the exact arithmetic in some lane and has written nothing (the caller defers it to
// adam8_pair_exact).  The pairs' instruction chains are independent, so with NP > 1 the
// scheduler interleaves them: one wave keeps NP pairs of latency in flight.
template <int MODE, int NP>
__device__ __forceinline__ uint32_t adam8_pairs_fast(const Adam8Args &a, const F8Consts &k, const Raw8 (&raw)[NP],
                                                     int64_t pr0, uint32_t lane, const float *q1s, const float *q2s,
                                                     const uint32_t *s_flat) {
    float p[NP][8], m[NP][8], v[NP][8], mx[NP], vx[NP];
    int32_t neg[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        float g[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            p[q][j] = bf16_at(raw[q].p, j);
            g[j] = bf16_at(raw[q].g, j);
        }
        // a sum of the 8 gradients is finite iff all of them are (or it overflows: exact)
        const float gsum = ((g[0] + g[1]) + (g[2] + g[3])) + ((g[4] + g[5]) + (g[6] + g[7]));
        float mxq = 0.0f, vxq = 0.0f;
        uint32_t mnz = 0xffffffffu;   // min of 2 bits(|m|) - 2: (bits of the smallest nonzero |m|) - 1, times 2
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float mq = q1s[byte_of(raw[q].mc, j)] * raw[q].ms;               // :65
            const float vq = q2s[byte_of(raw[q].vc, j)] * raw[q].vs;               // :66
            m[q][j] = k.b1 * mq + k.omb1 * g[j];                                   // :71
            v[q][j] = k.b2 * vq + (k.omb2 * g[j]) * g[j];                          // :72
            mxq = fmaxf(mxq, fabsf(m[q][j]));
            vxq = fmaxf(vxq, v[q][j]);
            mnz = min(mnz, (__float_as_uint(m[q][j]) << 1) - 2u);                  // +-0 gives 0xfffffffe
        }
        halfwave_max2(mxq, vxq);                                                   // :80-81
        mx[q] = mxq;
        vx[q] = vxq;
        const float md = mxq > 0.0f ? mxq : 1.0f;                                  // :82
        const float vd = vxq > 0.0f ? vxq : 1.0f;                                  // :83
        // Fast-branch conditions as sign bits of differences of non-negative bit patterns:
        // finite gradients and block scales, vs >= +0 (then m' is finite or +-inf and v' >= 0
        // finite or +inf, never NaN, so the maxima above are exact), max v' < 2^62, both
        // divisors in [2^-60, 2) and the update's numerators |step_c * m'| zero or in
        // [2^-90, 2^60) (the block maximum of |m'| bounds them from above).
        const int32_t FMAX = 0x7f7fffff, DLO = 0x21800000, DHI = 0x3fffffff, VXHI = 0x5e7fffff;
        const int32_t NHI = 0x5d7fffff;   // bits(2^60) - 1
        const int32_t gsb = (int32_t)(__float_as_uint(gsum) & 0x7fffffffu);
        const int32_t msb = (int32_t)(__float_as_uint(raw[q].ms) & 0x7fffffffu);
        const int32_t vsb = (int32_t)__float_as_uint(raw[q].vs), vxb = (int32_t)__float_as_uint(vxq);
        const int32_t mdb = (int32_t)__float_as_uint(md), vdb = (int32_t)__float_as_uint(vd);
        const int32_t nxb = (int32_t)__float_as_uint(k.step_abs * mxq), mnb = (int32_t)(mnz >> 1);
        neg[q] = (FMAX - gsb) | (FMAX - msb) | vsb | (FMAX - vsb) | (VXHI - vxb) | (mdb - DLO) |
                 (DHI - mdb) | (vdb - DLO) | (DHI - vdb) | (NHI - nxb) | (mnb - k.tm1);
    }
    uint32_t ok = 0;
#pragma unroll
    for (int q = 0; q < NP; ++q)
        if (__builtin_amdgcn_ballot_w64(neg[q] < 0) == 0) ok |= 1u << q;
    // the update, its SR store and the requantization of pair q
    auto finish = [&](int q) {
        const int64_t o0 = (pr0 + q) * F8_PAIR + lane * 8;
        uint32_t rp[8], w[8];
        noise8<MODE>(a.ns_p, o0, 8, rp);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float den = __builtin_fmaf(sqrt_rn_x2p32(v[q][j]), 0x1p-32f, k.eps_c);   // :74 sqrt(v) + eps
            const float upd = (p[q][j] - div_upd(k.step_c * m[q][j], den)) * k.decay;
            w[j] = __float_as_uint(upd) + rp[j];                                           // :75-78 (SR)
        }
        stu_nt4(a.p + (pr0 + q) * F8_PAIR, lane * 16u,
                u32x4_t{__builtin_amdgcn_perm(w[1], w[0], 0x07060302u), __builtin_amdgcn_perm(w[3], w[2], 0x07060302u),
                        __builtin_amdgcn_perm(w[5], w[4], 0x07060302u), __builtin_amdgcn_perm(w[7], w[6], 0x07060302u)});
        const float md = mx[q] > 0.0f ? mx[q] : 1.0f, vd = vx[q] > 0.0f ? vx[q] : 1.0f;
        const float ym = rcp_rn(md), yv = rcp_rn(vd);
        uint32_t rm[8], rv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            rm[j] = qf_signed(div_rn(m[q][j], md, ym), s_flat, k.lo1, k.scap);            // :82,84
            rv[j] = qf_unsigned(div_rn(v[q][j], vd, yv), s_flat + QF_SIGNED, k.lo1);     // :83,85
        }
        stu_nt2(static_cast<uint8_t *>(a.s1) + (pr0 + q) * F8_PAIR, lane * 8u,
                u32x2_t{pack_codes(rm[0], rm[1], rm[2], rm[3]), pack_codes(rm[4], rm[5], rm[6], rm[7])});
        stu_nt2(static_cast<uint8_t *>(a.s2) + (pr0 + q) * F8_PAIR, lane * 8u,
                u32x2_t{pack_codes(rv[0], rv[1], rv[2], rv[3]), pack_codes(rv[4], rv[5], rv[6], rv[7])});
        if ((lane & 31) == 0) {
            stu_f32(a.absmax1 + (pr0 + q) * 2, (lane >> 5) * 4u, mx[q]);         // :86
            stu_f32(a.absmax2 + (pr0 + q) * 2, (lane >> 5) * 4u, vx[q]);         // :87
        }
    };
    constexpr uint32_t ALL = (1u << NP) - 1u;
    if (ok == ALL) {
#pragma unroll
        for (int q = 0; q < NP; ++q) finish(q);
    } else {
#pragma unroll
        for (int q = 0; q < NP; ++q)
            if ((ok >> q) & 1u) finish(q);
    }
    return ok;
}

// Raw inputs of pair pr (wave-uniform), loaded into VGPRs: buffer loads from the pair's
// base address, so the address arithmetic runs on the scalar unit.
__device__ __forceinline__ Raw8 fetch_pair(const Adam8Args &a, int64_t pr, uint32_t lane) {
    Raw8 r;
    r.p = ldu_nt4(a.p + pr * F8_PAIR, lane * 16u);
    r.g = ldu_nt4(a.g + pr * F8_PAIR, lane * 16u);
    r.mc = ldu_nt2(static_cast<const uint8_t *>(a.s1) + pr * F8_PAIR, lane * 8u);
    r.vc = ldu_nt2(static_cast<const uint8_t *>(a.s2) + pr * F8_PAIR, lane * 8u);
    r.ms = ldu_f32(a.absmax1 + pr * 2, (lane >> 5) * 4u);
    r.vs = ldu_f32(a.absmax2 + pr * 2, (lane >> 5) * 4u);
    return r;
}

// The pairs a wave walks: pr, pr + stride, ... below end (groups of np adjacent pairs).
// The work-groups of one XCD take runs of MSR_F8_XCD_RUN consecutive places of the
// grid-stride order (-1: a run of g / 8, the XCD's whole share of each sweep).  A run of 4
// work-groups is 16 pairs, one 128-byte line of each block-scale array, which is then
// written from one XCD's L2 rather than from four.  Measured on 2^28 elements (A/B in one
// process, bit-exact): the step 2.4 % faster than places in dispatch order (runs of 32
// and g / 8: 1.4 % and 0 %), the access-pattern probe at 16 waves per CU 8.5 % faster.
#ifndef MSR_F8_XCD_RUN
#define MSR_F8_XCD_RUN 4
#endif
struct F8Walk {
    int64_t pr, end, stride;
};
__device__ __forceinline__ F8Walk f8_walk(int64_t npairs, int wave, int np) {
    const int64_t b = blockIdx.x, g = gridDim.x;
    constexpr int W = F8_THREADS / 64;
    const int64_t run = MSR_F8_XCD_RUN >= 0 ? MSR_F8_XCD_RUN : ((g & 7) == 0 ? g / 8 : 0);
    F8Walk w;
    w.pr = (xcd_place(b, g, run) * W + wave) * np;
    w.end = npairs;
    w.stride = g * W * np;
    return w;
}

// Four waves per SIMD (16 per CU) hide the branch's latency chains: at most 128 VGPRs.
#ifndef MSR_F8_MIN_WAVES
#define MSR_F8_MIN_WAVES 4
#endif
template <int MODE>
__global__ __launch_bounds__(F8_THREADS, MSR_F8_MIN_WAVES) void adamw8bit_fast_kernel(Adam8Args a, int64_t npairs) {
    __shared__ float q1s[256], q2s[256];
    __shared__ uint32_t s_flat[QF_TOTAL];
    __shared__ uint32_t s_deferred[F8_THREADS / 64][F8_DEFER];
    for (int i = threadIdx.x; i < 256; i += F8_THREADS) {
        q1s[i] = a.qmap1[i];
        q2s[i] = a.qmap2[i];
    }
    for (int i = threadIdx.x; i < QF_TOTAL; i += F8_THREADS) s_flat[i] = a.qtable->flat[i];
    __syncthreads();
    const F8Consts k = f8_consts(a);
    const uint32_t lane = threadIdx.x & 63u;
    // the pair index is wave-uniform: addresses are a scalar base plus a fixed lane offset.
    // Each wave takes F8_NP adjacent pairs per iteration (npairs is a multiple of F8_NP).
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const F8Walk walk = f8_walk(npairs, wave, F8_NP);
    const int64_t wstride = walk.stride, pend = walk.end;
    int64_t pr = walk.pr;
    uint32_t *deferred = s_deferred[wave];
    for (;;) {
        int ndef = 0;
        Raw8 nxt[F8_NP];
        if (pr < pend) {
#pragma unroll
            for (int q = 0; q < F8_NP; ++q) nxt[q] = fetch_pair(a, pr + q, lane);
        }
        for (; pr < pend; pr += wstride) {
            Raw8 raw[F8_NP];
#pragma unroll
            for (int q = 0; q < F8_NP; ++q) raw[q] = nxt[q];
            if (pr + wstride < pend) {
#pragma unroll
                for (int q = 0; q < F8_NP; ++q) nxt[q] = fetch_pair(a, pr + wstride + q, lane);
            }
            const uint32_t ok = adam8_pairs_fast<MODE, F8_NP>(a, k, raw, pr, lane, q1s, q2s, s_flat);
            if (ok == (1u << F8_NP) - 1u) continue;
#pragma unroll
            for (int q = 0; q < F8_NP; ++q) {
                if ((ok >> q) & 1u) continue;
                if (lane == 0) deferred[ndef] = (uint32_t)(pr + q);
                ++ndef;
            }
            if (ndef > F8_DEFER - F8_NP) {
                pr += wstride;
                break;
            }
        }
        __builtin_amdgcn_wave_barrier();   // lane 0's list writes precede the wave's reads
        for (int i = 0; i < ndef; ++i) {
            const int64_t pe = (int64_t)__builtin_amdgcn_readfirstlane(deferred[i]);
            adam8_pair_exact<MODE>(a, fetch_pair(a, pe, lane), pe * F8_PAIR + lane * 8, pe * 2 + (lane >> 5), q1s, q2s);
        }
        if (pr >= pend) break;
    }
}

// Streaming probe of the fast kernel's memory accesses (a measurement aid, no counterpart
// in the reference): the same pair walk, loads and stores as adamw8bit_fast_kernel (read p,
// g 16 B and the m, v codes 8 B per lane, and the two block scales; write p, m, v and the
// scales), with one integer operation per word in place of the arithmetic.  Its rate is what
// the memory system delivers for this pattern at a given grid and occupancy (set by the
// dynamic LDS of each work-group); the step cannot stream faster.
__global__ __launch_bounds__(F8_THREADS) void stream8_probe_kernel(Adam8Args a, int64_t npairs) {
    extern __shared__ uint32_t occupancy_pad[];
    const uint32_t lane = threadIdx.x & 63u;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const F8Walk walk = f8_walk(npairs, wave, 1);
    const int64_t wstride = walk.stride, pend = walk.end;
    int64_t pr = walk.pr;
    if (pr >= pend) return;
    Raw8 nxt = fetch_pair(a, pr, lane);
    for (; pr < pend; pr += wstride) {
        const Raw8 raw = nxt;
        if (pr + wstride < pend) nxt = fetch_pair(a, pr + wstride, lane);
        const int64_t o0 = pr * F8_PAIR + lane * 8;
        const u32x4_t pw = raw.p ^ raw.g;
        st_nt4(a.p + o0, pw);
        st_nt2(static_cast<uint8_t *>(a.s1) + o0, u32x2_t{raw.mc.x ^ 0x01010101u, raw.mc.y ^ 0x01010101u});
        st_nt2(static_cast<uint8_t *>(a.s2) + o0, u32x2_t{raw.vc.x + 0x01010101u, raw.vc.y + 0x01010101u});
        if ((lane & 31) == 0) {
            const int64_t qb = pr * 2 + (lane >> 5);
            a.absmax1[qb] = raw.ms + 1.0f;
            a.absmax2[qb] = raw.vs * 0.5f;
        }
    }
}

// Excluded tensors: bf16 moments with SR on both moment stores (:90-99).
template <int MODE, bool VEC>
__global__ __launch_bounds__(THREADS) void adamw8bit_bf16_kernel(Adam8Args a) {
    const Adam8Consts c = adam8_consts(a);
    uint16_t *m16 = static_cast<uint16_t *>(a.s1);
    uint16_t *v16 = static_cast<uint16_t *>(a.s2);
    const int64_t groups = (a.n + 7) >> 3;
    for (int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x; t < groups; t += (int64_t)gridDim.x * THREADS) {
        const int64_t o0 = t << 3;
        const int valid = clamp_valid(a.n, o0);
        uint32_t wp[4], wg[4], wm[4], wv[4];
        load_bf16x8<VEC>(a.p, o0, valid, wp);
        load_bf16x8<VEC>(a.g, o0, valid, wg);
        load_bf16x8<VEC>(m16, o0, valid, wm);
        load_bf16x8<VEC>(v16, o0, valid, wv);
        float p[8], g[8], m[8], v[8];
        unpack8(wp, p); unpack8(wg, g); unpack8(wm, m); unpack8(wv, v);
        uint32_t rp[8], rm[8], rv[8];
        noise8<MODE>(a.ns_p, o0, valid, rp);
        noise8<MODE>(a.ns_m, o0, valid, rm);
        noise8<MODE>(a.ns_v, o0, valid, rv);
        uint32_t op[8], om[8], ov[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool fin = fabsf(g[j]) < __builtin_huge_valf();
            const float mj = fin ? a.b1 * m[j] + c.one_m_b1 * g[j] : 0.0f;
            const float vj = fin ? a.b2 * v[j] + (c.one_m_b2 * g[j]) * g[j] : 0.0f;
            const float upd = (p[j] - (c.step_c * mj) / (sqrtf(vj) + c.eps_c)) * c.decay;
            const uint32_t pin = (j & 1) ? (wp[j >> 1] >> 16) : (wp[j >> 1] & 0xffffu);
            op[j] = fin ? sr_bf16(upd, rp[j]) : pin;
            om[j] = sr_bf16(mj, rm[j]);
            ov[j] = sr_bf16(vj, rv[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            wp[j] = pack2(op[2 * j], op[2 * j + 1]);
            wm[j] = pack2(om[2 * j], om[2 * j + 1]);
            wv[j] = pack2(ov[2 * j], ov[2 * j + 1]);
        }
        store_bf16x8<VEC>(a.p, o0, valid, wp);
        store_bf16x8<VEC>(m16, o0, valid, wm);
        store_bf16x8<VEC>(v16, o0, valid, wv);
    }
}


__global__ __launch_bounds__(THREADS) void quantize_kernel(const float *x, uint8_t *out, int64_t n,
                                                          const float *qmap, int is_signed, const QuantTable *qt) {
    __shared__ float q[256];
    __shared__ uint32_t s_oct[QT_OCT];
    __shared__ uint2 s_bkt[QT_MAX_BKT];
    for (int i = threadIdx.x; i < 256; i += THREADS) q[i] = qmap[i];
    if (qt) {
        for (int i = threadIdx.x; i < QT_OCT; i += THREADS) s_oct[i] = qt->oct[i];
        for (uint32_t i = threadIdx.x; i < qt->n_bkt; i += THREADS) s_bkt[i] = qt->bkt[i];
    }
    __syncthreads();
    for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * THREADS)
        out[i] = (uint8_t)(qt ? quantize_lookup(x[i], s_oct, s_bkt, is_signed != 0)
                              : quantize_search(x[i], q, is_signed != 0));
}

// Counts, per work-group, the floats x = bits(u) for u in [lo, hi] where the
// table disagrees with the search: signed map at x and -x, unsigned map at x.
__global__ __launch_bounds__(THREADS) void quant_table_check_kernel(const QuantTable *qt, const float *q1,
                                                                    const float *q2, uint32_t lo, uint32_t hi,
                                                                    uint32_t *counts) {
    __shared__ float s1[256], s2[256];
    __shared__ uint32_t s_oct[QT_OCT];
    __shared__ uint2 s_bkt[QT_MAX_BKT];
    __shared__ uint32_t s_flat[QF_TOTAL];
    __shared__ uint32_t red[THREADS];
    for (int i = threadIdx.x; i < 256; i += THREADS) { s1[i] = q1[i]; s2[i] = q2[i]; }
    for (int i = threadIdx.x; i < QT_OCT; i += THREADS) s_oct[i] = qt->oct[i];
    for (uint32_t i = threadIdx.x; i < qt->n_bkt; i += THREADS) s_bkt[i] = qt->bkt[i];
    for (int i = threadIdx.x; i < QF_TOTAL; i += THREADS) s_flat[i] = qt->flat[i];
    __syncthreads();
    uint32_t bad = 0;
    const uint64_t span = (uint64_t)hi - lo + 1;
    for (uint64_t i = (uint64_t)blockIdx.x * THREADS + threadIdx.x; i < span; i += (uint64_t)gridDim.x * THREADS) {
        const float x = __uint_as_float(lo + (uint32_t)i);
        const uint32_t cp = quantize_search(x, s1, true), cn = quantize_search(-x, s1, true);
        const uint32_t cu = quantize_search(x, s2, false);
        bad += quantize_lookup(x, s_oct, s_bkt, true) != cp;
        bad += quantize_lookup(-x, s_oct, s_bkt, true) != cn;
        bad += quantize_lookup(x, s_oct, s_bkt, false) != cu;
        // flat table (fast kernel): every x in [0, 1] and x in [-1, 0) (never -0)
        bad += ((qf_signed(x, s_flat, QF_LO1, QF_SCAP) >> 16) & 0xffu) != cp;
        if (x != 0.0f) bad += ((qf_signed(-x, s_flat, QF_LO1, QF_SCAP) >> 16) & 0xffu) != cn;
        bad += ((qf_unsigned(x, s_flat + QF_SIGNED, QF_LO1) >> 16) & 0xffu) != cu;
    }
    red[threadIdx.x] = bad;
    __syncthreads();
    for (int w = THREADS / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) counts[blockIdx.x] = red[0];
}

// Counts, per work-group, mismatches between a fast building block and the IEEE
// operation over the float bit patterns u in [lo, hi]:
//   kind 0: sqrt_rn(x) vs sqrtf(x), and fma(sqrt_rn_x2p32(x), 2^-32, e) vs sqrtf(x) + e
//           for a hashed e in [0, 2)            (x in [0, 2^62])
//   kind 1: rcp_rn(d) vs 1/d                  (d in [2^-60, 2))
//   kind 2: div_rn(m, d, rcp_rn(d)) vs m/d    (d in [2^-60, 2), 16 hashed m per d with
//           2^-63 d <= |m| <= d; for |m| < 2^-100 only the sign and zero-ness must agree)
//   kind 3: rne_bf16x2 (hardware conversion) vs rne_bf16 (any u; both halves)
//   kind 4: div_upd(n, d) vs n/d              (d in [2^-60, 2^32), 16 n per d: +-0 and
//           15 hashed n with |n| in [2^-90, 2^60], spread over the quotient's range)
__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16;
    return x;
}

__global__ __launch_bounds__(THREADS) void fastmath_check_kernel(int kind, uint32_t lo, uint32_t hi, uint32_t *counts) {
    __shared__ uint32_t red[THREADS];
    uint32_t bad = 0;
    const uint64_t span = (uint64_t)hi - lo + 1;
    for (uint64_t i = (uint64_t)blockIdx.x * THREADS + threadIdx.x; i < span; i += (uint64_t)gridDim.x * THREADS) {
        const uint32_t u = lo + (uint32_t)i;
        const float x = __uint_as_float(u);
        if (kind == 0) {
            const float r = sqrtf(x), e = __uint_as_float(mix32(u) & 0x3fffffffu);
            bad += __float_as_uint(sqrt_rn(x)) != __float_as_uint(r);
            bad += __float_as_uint(__builtin_fmaf(sqrt_rn_x2p32(x), 0x1p-32f, e)) != __float_as_uint(r + e);
        } else if (kind == 1) {
            bad += __float_as_uint(rcp_rn(x)) != __float_as_uint(1.0f / x);
        } else if (kind == 3) {
            const float x2 = __uint_as_float(~u);
            bad += rne_bf16x2(x, x2) != pack2(rne_bf16(x), rne_bf16(x2));
        } else if (kind == 4) {
            for (uint32_t k = 0; k < 16; ++k) {
                const uint32_t h = mix32(u * 16u + k);
                // |n| = 2^t * (1 + f), t in [-90, 59]; k = 0 is a signed zero
                const int t = (int)(h % 150u) - 90;
                float n = k == 0 ? 0.0f : ldexpf(1.0f + (float)(mix32(h) >> 8) * 0x1p-24f, t);
                if (h & 0x80000000u) n = -n;
                bad += __float_as_uint(div_upd(n, x)) != __float_as_uint(n / x);
            }
        } else {
            const float y = rcp_rn(x);
            for (uint32_t k = 0; k < 16; ++k) {
                const uint32_t h = mix32(u * 16u + k);
                // |m| = d * 2^-s * (1 + f), s in [0, 63], clamped to d: covers the whole quotient range
                const uint32_t s = h & 63u;
                float m = ldexpf(x, -(int)s) * (1.0f + (float)(mix32(h) >> 8) * 0x1p-24f);
                if (m > x) m = x;
                if (h & 0x80000000u) m = -m;
                const float q = div_rn(m, x, y), e = m / x;
                if (fabsf(m) >= 0x1p-100f) bad += __float_as_uint(q) != __float_as_uint(e);
                else bad += (signbit(q) != signbit(e)) || ((q == 0.0f) != (m == 0.0f));
            }
        }
    }
    red[threadIdx.x] = bad;
    __syncthreads();
    for (int w = THREADS / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) counts[blockIdx.x] = red[0];
}

}  // namespace msr

using namespace msr;

static inline Noise make_noise(uint32_t seed, uint32_t k, const uint16_t *inject, int64_t stream_stride) {
    Noise ns;
    ns.key = seed_key(seed, k);
    ns.inject = inject ? inject + (int64_t)k * stream_stride : nullptr;
    return ns;
}

#define MSR_CHECK_MODE(mode, inject)                                                         \
    do {                                                                                     \
        if ((mode) < 0 || (mode) > 2) { set_error("noise_mode %d is not 0, 1 or 2", (int)(mode)); return MSR_ERR_ARG; } \
        if ((mode) == NOISE_INJECT && !(inject)) { set_error("noise_mode INJECT needs an inject buffer"); return MSR_ERR_ARG; } \
    } while (0)

template <int MODE, int BLOCK>
static void launch_quant_mode(bool vec, bool qtab, const Adam8Args &a, hipStream_t s, unsigned grid, int wg) {
    if (qtab) {
        if (vec) hipLaunchKernelGGL((adamw8bit_quant_kernel<MODE, BLOCK, true, true>), dim3(grid), dim3(wg), 0, s, a);
        else hipLaunchKernelGGL((adamw8bit_quant_kernel<MODE, BLOCK, false, true>), dim3(grid), dim3(wg), 0, s, a);
    } else {
        if (vec) hipLaunchKernelGGL((adamw8bit_quant_kernel<MODE, BLOCK, true, false>), dim3(grid), dim3(wg), 0, s, a);
        else hipLaunchKernelGGL((adamw8bit_quant_kernel<MODE, BLOCK, false, false>), dim3(grid), dim3(wg), 0, s, a);
    }
}

template <int BLOCK>
static void launch_quant(int mode, bool vec, const Adam8Args &a, hipStream_t s, int64_t nblocks) {
    constexpr int TPB = BLOCK / 8;
    constexpr int WG = TPB > THREADS ? TPB : THREADS;
    constexpr int QB_PER_WG = WG / TPB;
    const unsigned grid = grid_for(nblocks - a.qb0, QB_PER_WG, 256 * 8);
    const bool qtab = a.qtable != nullptr;
    if (mode == NOISE_TRITON) launch_quant_mode<NOISE_TRITON, BLOCK>(vec, qtab, a, s, grid, WG);
    else if (mode == NOISE_PHILOX8) launch_quant_mode<NOISE_PHILOX8, BLOCK>(vec, qtab, a, s, grid, WG);
    else launch_quant_mode<NOISE_INJECT, BLOCK>(vec, qtab, a, s, grid, WG);
}

#ifndef MSR_F8_GRID_CAP
#define MSR_F8_GRID_CAP 2048   // twice the resident work-groups (4 per CU on 256 CUs): measured best
#endif

// Fast kernel over the first 2 * npairs blocks (block 256); returns blocks done.
static int64_t launch_fast8(int mode, const Adam8Args &a, hipStream_t s, int64_t nfull) {
    const int64_t npairs = nfull / (2 * F8_NP) * F8_NP;   // whole groups of F8_NP pairs; the rest goes to the general kernel
    if (npairs == 0 || npairs >= ((int64_t)1 << 31)) return 0;   // deferred pairs are recorded as int32
    // the update's divisor sqrt(v') + eps_c must lie in [2^-60, 2^32) (sqrt(v') < 2^31 is
    // checked per pair), and step_c must be finite: the same fp32 arithmetic as adam8_consts
    const float sqrt_bc2 = sqrtf(a.bc2), eps_c = sqrt_bc2 * a.eps, step_c = (a.lr * sqrt_bc2) / a.bc1;
    if (!(eps_c >= 0x1p-60f && eps_c <= 0x1p30f) || !std::isfinite(step_c)) return 0;
    const unsigned grid = grid_for(npairs / F8_NP, F8_THREADS / 64, MSR_F8_GRID_CAP);
    if (mode == NOISE_TRITON) hipLaunchKernelGGL((adamw8bit_fast_kernel<NOISE_TRITON>), dim3(grid), dim3(F8_THREADS), 0, s, a, npairs);
    else if (mode == NOISE_PHILOX8) hipLaunchKernelGGL((adamw8bit_fast_kernel<NOISE_PHILOX8>), dim3(grid), dim3(F8_THREADS), 0, s, a, npairs);
    else hipLaunchKernelGGL((adamw8bit_fast_kernel<NOISE_INJECT>), dim3(grid), dim3(F8_THREADS), 0, s, a, npairs);
    return 2 * npairs;
}

extern "C" {

int msr_adamw8bit_step(uint16_t *p, const uint16_t *g, void *state1, void *state2, float *absmax1, float *absmax2,
                       const float *qmap1, const float *qmap2, const void *qtable, int64_t n, int32_t block,
                       int32_t quantized, float lr,
                       float beta1, float beta2, float eps, float weight_decay, float bc1, float bc2, uint32_t seed,
                       int32_t noise_mode, const uint16_t *inject, msr_stream_t stream) {
    if (n < 0 || (n > 0 && (!p || !g || !state1 || !state2))) { set_error("msr_adamw8bit_step: bad arguments"); return MSR_ERR_ARG; }
    if (block < 32 || block > 4096 || (block & (block - 1))) {
        set_error("msr_adamw8bit_step: block %d is not a power of two in [32, 4096]", (int)block);
        return MSR_ERR_ARG;
    }
    if (quantized && (!absmax1 || !absmax2 || !qmap1 || !qmap2)) { set_error("msr_adamw8bit_step: quantized state needs absmax and qmaps"); return MSR_ERR_ARG; }
    MSR_CHECK_MODE(noise_mode, inject);
    if (n == 0) return MSR_OK;
    {
        const size_t sb = (quantized ? 1 : 2) * (size_t)n, ab = 4 * (size_t)((n + block - 1) / block);
        const void *ops[6] = {p, g, state1, state2, quantized ? absmax1 : nullptr, quantized ? absmax2 : nullptr};
        const size_t len[6] = {2 * (size_t)n, 2 * (size_t)n, sb, sb, ab, ab};
        for (int i = 0; i < 6; ++i)
            for (int j = i + 1; j < 6; ++j)
                if (partial_overlap(ops[i], len[i], ops[j], len[j])) {
                    set_error("msr_adamw8bit_step: operands %d and %d overlap", i, j);
                    return MSR_ERR_OVERLAP;
                }
    }
    Adam8Args a;
    a.p = p; a.g = g; a.s1 = state1; a.s2 = state2; a.absmax1 = absmax1; a.absmax2 = absmax2;
    a.qmap1 = qmap1; a.qmap2 = qmap2; a.n = n; a.qb0 = 0;
    a.qtable = static_cast<const QuantTable *>(qtable);
    if (a.qtable && !aligned(a.qtable, 16)) { set_error("msr_adamw8bit_step: qtable must be 16-byte aligned"); return MSR_ERR_ALIGN; }
    a.lr = lr; a.b1 = beta1; a.b2 = beta2; a.eps = eps; a.wd = weight_decay; a.bc1 = bc1; a.bc2 = bc2;
    a.ns_p = make_noise(seed, 0, inject, n);
    a.ns_m = make_noise(seed, 1, inject, n);
    a.ns_v = make_noise(seed, 2, inject, n);
    hipStream_t s = (hipStream_t)stream;
    if (quantized) {
        const bool vec = aligned(p, 16) && aligned(g, 16) && aligned(state1, 8) && aligned(state2, 8);
        const int64_t nblocks = (n + block - 1) / block;
        // standard codebooks, block 256, aligned: the fast kernel takes the full block pairs
        if (block == 256 && a.qtable && vec) a.qb0 = launch_fast8(noise_mode, a, s, n / 256);
        if (a.qb0 == nblocks) return check_launch("msr_adamw8bit_step");
        switch (block) {
        case 32: launch_quant<32>(noise_mode, vec, a, s, nblocks); break;
        case 64: launch_quant<64>(noise_mode, vec, a, s, nblocks); break;
        case 128: launch_quant<128>(noise_mode, vec, a, s, nblocks); break;
        case 256: launch_quant<256>(noise_mode, vec, a, s, nblocks); break;
        case 512: launch_quant<512>(noise_mode, vec, a, s, nblocks); break;
        case 1024: launch_quant<1024>(noise_mode, vec, a, s, nblocks); break;
        case 2048: launch_quant<2048>(noise_mode, vec, a, s, nblocks); break;
        default: launch_quant<4096>(noise_mode, vec, a, s, nblocks); break;
        }
    } else {
        const bool vec = aligned(p, 16) && aligned(g, 16) && aligned(state1, 16) && aligned(state2, 16);
        const unsigned grid = grid_for((n + 7) / 8, THREADS);
        if (vec) { MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((adamw8bit_bf16_kernel<M, true>), dim3(grid), dim3(THREADS), 0, s, a)); }
        else { MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((adamw8bit_bf16_kernel<M, false>), dim3(grid), dim3(THREADS), 0, s, a)); }
    }
    return check_launch("msr_adamw8bit_step");
}

int msr_stream_probe8(uint16_t *p, const uint16_t *g, uint8_t *state1, uint8_t *state2, float *absmax1,
                      float *absmax2, int64_t n, int32_t grid, int32_t lds_bytes, msr_stream_t stream) {
    if (n <= 0 || n % F8_PAIR || !p || !g || !state1 || !state2 || !absmax1 || !absmax2) {
        set_error("msr_stream_probe8: n must be a positive multiple of %d and every pointer set", F8_PAIR);
        return MSR_ERR_ARG;
    }
    if (!aligned(p, 16) || !aligned(g, 16) || !aligned(state1, 8) || !aligned(state2, 8)) {
        set_error("msr_stream_probe8: p, g need 16-byte and the codes 8-byte alignment");
        return MSR_ERR_ALIGN;
    }
    if (grid < 1 || grid > (1 << 20) || lds_bytes < 0 || lds_bytes > (64 << 10)) {
        set_error("msr_stream_probe8: grid %d not in [1, 2^20] or lds_bytes %d not in [0, 64 KiB]", (int)grid, (int)lds_bytes);
        return MSR_ERR_ARG;
    }
    Adam8Args a = {};
    a.p = p; a.g = g; a.s1 = state1; a.s2 = state2; a.absmax1 = absmax1; a.absmax2 = absmax2; a.n = n;
    hipLaunchKernelGGL(stream8_probe_kernel, dim3((unsigned)grid), dim3(F8_THREADS), (unsigned)lds_bytes,
                       (hipStream_t)stream, a, n / F8_PAIR);
    return check_launch("msr_stream_probe8");
}

int msr_quantize(const float *x, uint8_t *out, int64_t n, const float *qmap, int32_t is_signed, const void *qtable,
                 msr_stream_t stream) {
    if (n < 0 || (n > 0 && (!x || !out || !qmap))) { set_error("msr_quantize: bad arguments"); return MSR_ERR_ARG; }
    if (n == 0) return MSR_OK;
    hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(n, THREADS)), dim3(THREADS), 0, (hipStream_t)stream, x, out, n,
                       qmap, is_signed, static_cast<const QuantTable *>(qtable));
    return check_launch("msr_quantize");
}

size_t msr_quant_table_bytes(void) { return sizeof(QuantTable); }

int msr_quant_table_build(const float *qmap_signed, const float *qmap_unsigned, void *table, size_t table_bytes) {
    if (!qmap_signed || !qmap_unsigned || !table || table_bytes < sizeof(QuantTable)) {
        set_error("msr_quant_table_build: need host codebooks and a host buffer of %zu bytes", sizeof(QuantTable));
        return MSR_ERR_ARG;
    }
    QuantTable *t = static_cast<QuantTable *>(table);
    memset(t, 0, sizeof(QuantTable));
    const uint32_t ONE = 0x3f800000u;
    uint32_t nb = 0;
    // three sides: signed map x >= 0, signed map x < 0, unsigned map x >= 0
    for (int side = 0; side < 3; ++side) {
        const float *Q = side < 2 ? qmap_signed : qmap_unsigned;
        const bool sgn = side < 2;
        const bool neg = side == 1;
        const uint32_t oct_base = (side == 2 ? 512u : 0u) + (neg ? 256u : 0u);
        auto f = [&](uint32_t a) {
            const float x = __builtin_bit_cast(float, a | (neg ? 0x80000000u : 0u));
            return quantize_search(x, Q, sgn);
        };
        // change points of the monotone code over |x| bits a in [0, ONE], by bisection
        std::vector<uint32_t> tr;
        std::vector<std::pair<uint32_t, uint32_t>> stack{{0u, ONE}};
        while (!stack.empty()) {
            auto [lo, hi] = stack.back();
            stack.pop_back();
            if (f(lo) == f(hi)) continue;
            if (hi == lo + 1) { tr.push_back(hi); continue; }
            const uint32_t mid = lo + (hi - lo) / 2;
            stack.push_back({mid, hi});
            stack.push_back({lo, mid});
        }
        std::sort(tr.begin(), tr.end());
        for (uint32_t e = 0; e < 128; ++e) {
            const uint32_t base = e << 23;
            std::vector<uint32_t> te;
            for (uint32_t x : tr)
                if ((x >> 23) == e) te.push_back(x);
            int sh = 23;
            auto ok = [&](int s) {
                for (size_t i = 1; i < te.size(); ++i)
                    if ((te[i] >> s) == (te[i - 1] >> s)) return false;
                return true;
            };
            while (sh > 0 && !ok(sh)) --sh;
            if (!ok(sh)) { set_error("msr_quant_table_build: two code changes one ulp apart"); return MSR_ERR_ARG; }
            const uint32_t cnt = 1u << (23 - sh);
            if (nb + cnt + 1 > (uint32_t)QT_MAX_BKT) { set_error("msr_quant_table_build: more than %d buckets", QT_MAX_BKT); return MSR_ERR_ARG; }
            t->oct[oct_base + e] = (nb << 8) | (uint32_t)sh;
            for (uint32_t k = 0; k < cnt; ++k) {
                const uint32_t a0 = base + (k << sh);
                const uint32_t a1 = a0 + (1u << sh) - 1;
                uint32_t thr = 0xffffffffu;
                for (uint32_t x : te)
                    if (x > a0 && x <= a1) thr = x;
                const uint32_t lo_code = a0 <= ONE ? f(a0) : f(ONE);
                const uint32_t hi_code = thr != 0xffffffffu ? f(thr) : lo_code;
                t->bkt[nb + k] = make_uint2(thr, lo_code | (hi_code << 8));
            }
            nb += cnt;
        }
        // exponents 128..255 (|x| > 1 cannot occur; 255 is NaN): the search's NaN code
        const uint32_t nan_code = quantize_search(__builtin_bit_cast(float, 0x7fc00000u), Q, sgn);
        t->bkt[nb] = make_uint2(0xffffffffu, nan_code | (nan_code << 8));
        for (uint32_t e = 128; e < 256; ++e) t->oct[oct_base + e] = (nb << 8) | 23u;
        nb += 1;
    }
    // the unsigned map never sees x < 0 (v >= 0); point that half at its NaN bucket
    for (uint32_t e = 0; e < 256; ++e) t->oct[512 + 256 + e] = t->oct[512 + 255];
    t->n_bkt = nb;

    // flat table of the fast kernel (layout in common.hpp)
    for (int i = 0; i < QF_TOTAL; ++i) t->flat[i] = 0;
    for (int plane = 0; plane < 3; ++plane) {          // signed x >= 0, signed x < 0, unsigned
        const float *Q = plane < 2 ? qmap_signed : qmap_unsigned;
        const bool sgn = plane < 2;
        const uint32_t sign = plane == 1 ? 0x80000000u : 0u;
        uint32_t *dst = t->flat + (plane == 2 ? QF_SIGNED : 0);
        for (int k = 0; k < QF_N; ++k) {
            const uint32_t key = QF_LO1 + (uint32_t)k;   // k = 0: every |x| < 2^-23
            // code at lookup variable w (low 16 bits, complemented on the negative plane)
            auto code_at = [&](uint32_t w) {
                const uint32_t low = sign ? 0xffffu - w : w;
                return quantize_search(__builtin_bit_cast(float, sign | (key << 16) | low), Q, sgn);
            };
            uint32_t entry;
            if (k == 0) {
                // one code per sign (the fast kernel never forms x = -0)
                entry = quantize_search(__builtin_bit_cast(float, sign | 1u), Q, sgn) << 16;
            } else if (key == (127u << 7)) {
                // [1, 1 + 2^-7): only |x| = 1 occurs
                entry = quantize_search(__builtin_bit_cast(float, sign | ONE), Q, sgn) << 16;
            } else {
                const uint32_t c0 = code_at(0), c1 = code_at(0xffffu);
                if (c0 == c1) {
                    entry = c0 << 16;
                } else {
                    if (c1 != c0 + 1) { set_error("msr_quant_table_build: codes jump by %d in one bucket", (int)(c1 - c0)); return MSR_ERR_ARG; }
                    uint32_t lo = 0, hi = 0xffffu;   // code_at(lo) == c0, code_at(hi) == c1
                    while (hi - lo > 1) {
                        const uint32_t mid = (lo + hi) / 2;
                        if (code_at(mid) == c0) lo = mid; else hi = mid;
                    }
                    entry = (c0 << 16) | (0x10000u - hi);
                }
            }
            const int idx = plane == 1 ? (k == 0 ? QF_SCAP : (int)(0x7fffu - key - QF_LO1)) : k;
            dst[idx] = entry;
        }
    }
    return MSR_OK;
}

int msr_quant_table_check(const void *qtable, const float *qmap_signed, const float *qmap_unsigned, uint32_t bits_lo,
                          uint32_t bits_hi, uint32_t *counts, int32_t n_counts, msr_stream_t stream) {
    if (!qtable || !qmap_signed || !qmap_unsigned || !counts || n_counts <= 0 || bits_hi < bits_lo ||
        bits_hi > 0x3f800000u) {
        set_error("msr_quant_table_check: bad arguments");
        return MSR_ERR_ARG;
    }
    hipLaunchKernelGGL(quant_table_check_kernel, dim3((unsigned)n_counts), dim3(THREADS), 0, (hipStream_t)stream,
                       static_cast<const QuantTable *>(qtable), qmap_signed, qmap_unsigned, bits_lo, bits_hi, counts);
    return check_launch("msr_quant_table_check");
}

int msr_fastmath_check(int32_t kind, uint32_t bits_lo, uint32_t bits_hi, uint32_t *counts, int32_t n_counts,
                       msr_stream_t stream) {
    const uint32_t SQRT_HI = 0x5e800000u, RCP_LO = 0x21800000u, RCP_HI = 0x3fffffffu;   // 2^62, 2^-60, 2 - ulp
    const uint32_t UPD_HI = 0x4f7fffffu;                                                 // 2^32 - ulp
    const bool range_ok = kind == 0 ? bits_hi <= SQRT_HI
                        : kind == 3 ? true
                        : kind == 2 ? bits_lo >= RCP_LO && bits_hi <= RCP_HI
                                    : (kind == 1 || kind == 4) && bits_lo >= RCP_LO && bits_hi <= UPD_HI;
    if (!counts || n_counts <= 0 || bits_hi < bits_lo || !range_ok) {
        set_error("msr_fastmath_check: bad arguments (kind %d, range %08x..%08x)", (int)kind, bits_lo, bits_hi);
        return MSR_ERR_ARG;
    }
    hipLaunchKernelGGL(fastmath_check_kernel, dim3((unsigned)n_counts), dim3(THREADS), 0, (hipStream_t)stream, (int)kind,
                       bits_lo, bits_hi, counts);
    return check_launch("msr_fastmath_check");
}

}  // extern "C"
