// Memory-bound optimizer kernels for gfx950: SR gradient accumulation, bf16-
// moment AdamW, 8-bit blockwise AdamW and the Muon momentum/update passes.
//
// Each thread owns 8 consecutive elements (one 16-byte bf16 vector), so a
// wave64 streams 1 KiB of every bf16 operand per access.  The quantized AdamW
// kernel assigns block/8 consecutive threads to one quantization block and
// reduces the block absmax with cross-lane shuffles (LDS across waves for
// blocks above 512 elements).
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <utility>
#include <vector>

#include "common.hpp"
#include "../../include/muon_sr_amd.h"

namespace msr {

static thread_local char g_err[512];

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return (int)e;
    }
    return MSR_OK;
}

constexpr int THREADS = 256;

// ---------------------------------------------------------------------------
// 8-element vector I/O (aligned fast path, masked scalar path at tails or for
// unaligned views)
// ---------------------------------------------------------------------------

// Streaming accesses: every element-wise kernel touches each byte once, so the
// aligned vector paths use non-temporal loads and stores (measured: the SR
// accumulate over 7.8 GB goes from 5.2 to 5.6 TB/s).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4_t ld_nt4(const void *p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p)); }
__device__ __forceinline__ u32x2_t ld_nt2(const void *p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p)); }
__device__ __forceinline__ f32x4_t ld_nt4f(const void *p) { return __builtin_nontemporal_load(reinterpret_cast<const f32x4_t *>(p)); }
__device__ __forceinline__ void st_nt4(void *p, u32x4_t v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t *>(p)); }
__device__ __forceinline__ void st_nt2(void *p, u32x2_t v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x2_t *>(p)); }

template <bool VEC>
__device__ __forceinline__ void load_bf16x8(const uint16_t *base, int64_t o0, int valid, uint32_t w[4]) {
    if (VEC && valid == 8) {
        const u32x4_t v = ld_nt4(base + o0);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t lo = (2 * j < valid) ? base[o0 + 2 * j] : 0u;
            uint32_t hi = (2 * j + 1 < valid) ? base[o0 + 2 * j + 1] : 0u;
            w[j] = lo | (hi << 16);
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void store_bf16x8(uint16_t *base, int64_t o0, int valid, const uint32_t w[4]) {
    if (VEC && valid == 8) {
        st_nt4(base + o0, u32x4_t{w[0], w[1], w[2], w[3]});
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (2 * j < valid) base[o0 + 2 * j] = (uint16_t)(w[j] & 0xffffu);
            if (2 * j + 1 < valid) base[o0 + 2 * j + 1] = (uint16_t)(w[j] >> 16);
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void load_f32x8(const float *base, int64_t o0, int valid, float f[8]) {
    if (VEC && valid == 8) {
        const f32x4_t a = ld_nt4f(base + o0);
        const f32x4_t b = ld_nt4f(base + o0 + 4);
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = (j < valid) ? base[o0 + j] : 0.0f;
    }
}

template <bool VEC>
__device__ __forceinline__ void load_u8x8(const uint8_t *base, int64_t o0, int valid, uint32_t fill,
                                          uint32_t c[8]) {
    if (VEC && valid == 8) {
        const u32x2_t v = ld_nt2(base + o0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            c[j] = (v.x >> (8 * j)) & 0xffu;
            c[j + 4] = (v.y >> (8 * j)) & 0xffu;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = (j < valid) ? (uint32_t)base[o0 + j] : fill;
    }
}

template <bool VEC>
__device__ __forceinline__ void store_u8x8(uint8_t *base, int64_t o0, int valid, const uint32_t c[8]) {
    if (VEC && valid == 8) {
        uint32_t x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
        uint32_t y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
        st_nt2(base + o0, u32x2_t{x, y});
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < valid) base[o0 + j] = (uint8_t)c[j];
    }
}

__device__ __forceinline__ void unpack8(const uint32_t w[4], float f[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_lo(w[j]);
        f[2 * j + 1] = bf16_hi(w[j]);
    }
}

__device__ __forceinline__ int clamp_valid(int64_t n, int64_t o0) {
    int64_t r = n - o0;
    return r <= 0 ? 0 : (r >= 8 ? 8 : (int)r);
}

// ---------------------------------------------------------------------------
// (c) SR gradient accumulation   (muon_sr/triton_adamw.py:206-229)
// ---------------------------------------------------------------------------

// One 8-element group of acc <- SR(acc + grad): offsets o0 .. o0+7 of a tensor
// of n elements (valid = how many exist).
template <int MODE, bool GF32, bool ZERO, bool VEC>
__device__ __forceinline__ void accum_group(uint16_t *__restrict__ acc, const void *__restrict__ grad,
                                            const Noise &ns, int64_t o0, int valid) {
    float a[8], g[8];
    if constexpr (ZERO) {
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = 0.0f;
    } else {
        uint32_t w[4];
        load_bf16x8<VEC>(acc, o0, valid, w);
        unpack8(w, a);
    }
    if constexpr (GF32) {
        load_f32x8<VEC>(static_cast<const float *>(grad), o0, valid, g);
    } else {
        uint32_t w[4];
        load_bf16x8<VEC>(static_cast<const uint16_t *>(grad), o0, valid, w);
        unpack8(w, g);
    }
    uint32_t r[8];
    noise8<MODE>(ns, o0, valid, r);
    uint32_t out[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        out[j] = pack2(sr_bf16(a[2 * j] + g[2 * j], r[2 * j]), sr_bf16(a[2 * j + 1] + g[2 * j + 1], r[2 * j + 1]));
    store_bf16x8<VEC>(acc, o0, valid, out);
}

template <int MODE, bool GF32, bool ZERO, bool VEC>
__global__ __launch_bounds__(THREADS) void sr_accum_kernel(uint16_t *__restrict__ acc, const void *__restrict__ grad,
                                                          int64_t n, Noise ns) {
    const int64_t groups = (n + 7) >> 3;
    for (int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x; t < groups; t += (int64_t)gridDim.x * THREADS) {
        const int64_t o0 = t << 3;
        accum_group<MODE, GF32, ZERO, VEC>(acc, grad, ns, o0, clamp_valid(n, o0));
    }
}

// Many tensors in one launch (the hooks of a backward pass, deferred).  Tensor
// t owns groups [gstart[t], gstart[t+1]) of the launch's group space; its
// offsets, and so its noise counters, start at 0, so the result equals one
// sr_accum_kernel launch per tensor.
constexpr int ACC_MAXT = 80;
constexpr uint32_t ACC_ZERO = 1, ACC_F32 = 2, ACC_VEC = 4;
struct AccumMultiArgs {
    int count;
    int64_t gstart[ACC_MAXT + 1];
    uint16_t *acc[ACC_MAXT];
    const void *grad[ACC_MAXT];
    int64_t n[ACC_MAXT];
    PhiloxKey key[ACC_MAXT];
    uint32_t flags[ACC_MAXT];
};

template <int MODE>
__global__ __launch_bounds__(THREADS) void sr_accum_multi_kernel(AccumMultiArgs a) {
    __shared__ int64_t s_start[ACC_MAXT + 1];
    for (int i = threadIdx.x; i <= a.count; i += THREADS) s_start[i] = a.gstart[i];
    __syncthreads();
    const int64_t total = s_start[a.count];
    for (int64_t gi = (int64_t)blockIdx.x * THREADS + threadIdx.x; gi < total; gi += (int64_t)gridDim.x * THREADS) {
        int lo = 0, hi = a.count - 1;   // last t with s_start[t] <= gi
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_start[mid] <= gi) lo = mid; else hi = mid - 1;
        }
        const int t = lo;
        const int64_t o0 = (gi - s_start[t]) << 3;
        const int valid = clamp_valid(a.n[t], o0);
        Noise ns;
        ns.key = a.key[t];
        ns.inject = nullptr;
        uint16_t *acc = a.acc[t];
        const void *grad = a.grad[t];
        switch (a.flags[t]) {
            case 0: accum_group<MODE, false, false, false>(acc, grad, ns, o0, valid); break;
            case ACC_ZERO: accum_group<MODE, false, true, false>(acc, grad, ns, o0, valid); break;
            case ACC_F32: accum_group<MODE, true, false, false>(acc, grad, ns, o0, valid); break;
            case ACC_F32 | ACC_ZERO: accum_group<MODE, true, true, false>(acc, grad, ns, o0, valid); break;
            case ACC_VEC: accum_group<MODE, false, false, true>(acc, grad, ns, o0, valid); break;
            case ACC_VEC | ACC_ZERO: accum_group<MODE, false, true, true>(acc, grad, ns, o0, valid); break;
            case ACC_VEC | ACC_F32: accum_group<MODE, true, false, true>(acc, grad, ns, o0, valid); break;
            default: accum_group<MODE, true, true, true>(acc, grad, ns, o0, valid); break;
        }
    }
}

// ---------------------------------------------------------------------------
// BF16-moment AdamW   (muon_sr/triton_adamw.py:9-72)
// ---------------------------------------------------------------------------

struct AdamWArgs {
    uint16_t *p;
    const uint16_t *g;
    uint16_t *ema;
    uint16_t *ema_sq;
    int64_t n;
    float lr, beta1, beta2, eps, wd, bc, bcs;
    Noise ns_ema, ns_ema_sq, ns_p;
};

template <int MODE, bool VEC>
__global__ __launch_bounds__(THREADS) void adamw_bf16_kernel(AdamWArgs a) {
    const float one_m_b1 = 1.0f - a.beta1;
    const float one_m_b2 = 1.0f - a.beta2;
    const float step_size = a.lr / a.bc;
    const float decay = 1.0f - a.lr * a.wd;
    const int64_t groups = (a.n + 7) >> 3;
    for (int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x; t < groups; t += (int64_t)gridDim.x * THREADS) {
        const int64_t o0 = t << 3;
        const int valid = clamp_valid(a.n, o0);
        uint32_t wp[4], wg[4], we[4], ws[4];
        load_bf16x8<VEC>(a.p, o0, valid, wp);
        load_bf16x8<VEC>(a.g, o0, valid, wg);
        load_bf16x8<VEC>(a.ema, o0, valid, we);
        load_bf16x8<VEC>(a.ema_sq, o0, valid, ws);
        float p[8], g[8], e[8], s[8];
        unpack8(wp, p); unpack8(wg, g); unpack8(we, e); unpack8(ws, s);
        uint32_t re[8], rs[8], rp[8];
        noise8<MODE>(a.ns_ema, o0, valid, re);
        noise8<MODE>(a.ns_ema_sq, o0, valid, rs);
        noise8<MODE>(a.ns_p, o0, valid, rp);
        uint32_t oe[8], os[8], op[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float ej = a.beta1 * e[j] + one_m_b1 * g[j];
            float sj = a.beta2 * s[j] + (one_m_b2 * g[j]) * g[j];
            float denom = sqrtf(sj) / a.bcs + a.eps;
            float pj = p[j] * decay;
            pj = pj - (step_size * ej) / denom;
            oe[j] = sr_bf16(ej, re[j]);
            os[j] = sr_bf16(sj, rs[j]);
            op[j] = sr_bf16(pj, rp[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            we[j] = pack2(oe[2 * j], oe[2 * j + 1]);
            ws[j] = pack2(os[2 * j], os[2 * j + 1]);
            wp[j] = pack2(op[2 * j], op[2 * j + 1]);
        }
        store_bf16x8<VEC>(a.ema, o0, valid, we);
        store_bf16x8<VEC>(a.ema_sq, o0, valid, ws);
        store_bf16x8<VEC>(a.p, o0, valid, wp);
    }
}

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

    int64_t qb = (int64_t)blockIdx.x * QB_PER_WG + sub;
    Raw nxt;
    fetch(qb, nxt);
    for (int64_t qb0 = (int64_t)blockIdx.x * QB_PER_WG; qb0 < nblocks; qb0 += stride, qb += stride) {
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

// ---------------------------------------------------------------------------
// Muon prepare / apply   (muon_sr/triton_muon_sr.py:18-80)
// ---------------------------------------------------------------------------

constexpr int MAX_TABLE = 240;  // pointers per launch (kernel-argument table)

struct PrepareArgs {
    const uint16_t *grads[MAX_TABLE];
    uint16_t *buf;       // stack base (already offset to the first matrix of this launch)
    uint16_t *out;
    int64_t numel;
    int64_t stack_off0;  // stack offset of matrix 0 of this launch (noise counter base)
    float beta;
    Noise ns;
};

template <int MODE, bool NEST, bool VEC>
__global__ __launch_bounds__(THREADS) void muon_prepare_kernel(PrepareArgs a) {
    const int i = blockIdx.y;
    const uint16_t *g = a.grads[i];
    uint16_t *buf = a.buf + (int64_t)i * a.numel;
    uint16_t *out = a.out + (int64_t)i * a.numel;
    const int64_t base = a.stack_off0 + (int64_t)i * a.numel;
    const float one_m_beta = 1.0f - a.beta;
    const int64_t groups = (a.numel + 7) >> 3;
    for (int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x; t < groups; t += (int64_t)gridDim.x * THREADS) {
        const int64_t o0 = t << 3;
        const int valid = clamp_valid(a.numel, o0);
        uint32_t wg[4], wb[4];
        load_bf16x8<VEC>(g, o0, valid, wg);
        load_bf16x8<VEC>(buf, o0, valid, wb);
        float gf[8], bf[8];
        unpack8(wg, gf);
        unpack8(wb, bf);
        uint32_t r[8];
        if (VEC || MODE != NOISE_PHILOX8) {
            noise8<MODE>(a.ns, base + o0, valid, r);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = (j < valid) ? noise1<MODE>(a.ns, base + o0 + j) : 0u;
        }
        uint32_t ob[8], ou[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float nb = bf[j] + one_m_beta * (gf[j] - bf[j]);        // :37
            const float upd = NEST ? gf[j] + a.beta * (nb - gf[j]) : nb;  // :39-42
            ob[j] = sr_bf16(nb, r[j]);                                    // :44-49
            ou[j] = rne_bf16(upd);                                        // :50
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            wb[j] = pack2(ob[2 * j], ob[2 * j + 1]);
            wg[j] = pack2(ou[2 * j], ou[2 * j + 1]);
        }
        store_bf16x8<VEC>(buf, o0, valid, wb);
        store_bf16x8<VEC>(out, o0, valid, wg);
    }
}

struct ApplyArgs {
    uint16_t *params[MAX_TABLE];
    uint32_t seeds[MAX_TABLE];
    const uint16_t *upd;  // [count][numel] for this launch
    int64_t numel;
    float lr, wd, scale;
    const uint16_t *inject;  // [count][numel] for this launch (NOISE_INJECT)
};

template <int MODE, bool VEC>
__global__ __launch_bounds__(THREADS) void muon_apply_kernel(ApplyArgs a) {
    const int i = blockIdx.y;
    uint16_t *p = a.params[i];
    const uint16_t *u = a.upd + (int64_t)i * a.numel;
    Noise ns;
    ns.key = seed_key(a.seeds[i], 0);
    ns.inject = a.inject ? a.inject + (int64_t)i * a.numel : nullptr;
    const float decay = 1.0f - a.lr * a.wd;                               // :72
    const int64_t groups = (a.numel + 7) >> 3;
    for (int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x; t < groups; t += (int64_t)gridDim.x * THREADS) {
        const int64_t o0 = t << 3;
        const int valid = clamp_valid(a.numel, o0);
        uint32_t wp[4], wu[4];
        load_bf16x8<VEC>(p, o0, valid, wp);
        load_bf16x8<VEC>(u, o0, valid, wu);
        float pf[8], uf[8];
        unpack8(wp, pf);
        unpack8(wu, uf);
        uint32_t r[8];
        noise8<MODE>(ns, o0, valid, r);
        uint32_t op[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float t1 = uf[j] * a.scale;                             // :70
            float pj = pf[j] * decay;                                     // :72
            pj = pj - a.lr * t1;                                          // :73
            op[j] = sr_bf16(pj, r[j]);                                    // :75-80
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) wp[j] = pack2(op[2 * j], op[2 * j + 1]);
        store_bf16x8<VEC>(p, o0, valid, wp);
    }
}

// ---------------------------------------------------------------------------
// Diagnostics
// ---------------------------------------------------------------------------

template <int MODE>
__global__ __launch_bounds__(THREADS) void noise_fill_kernel(uint16_t *out, int64_t n, int64_t off0, Noise ns) {
    for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * THREADS)
        out[i] = (uint16_t)noise1<MODE>(ns, off0 + i);
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
    __shared__ uint32_t red[THREADS];
    for (int i = threadIdx.x; i < 256; i += THREADS) { s1[i] = q1[i]; s2[i] = q2[i]; }
    for (int i = threadIdx.x; i < QT_OCT; i += THREADS) s_oct[i] = qt->oct[i];
    for (uint32_t i = threadIdx.x; i < qt->n_bkt; i += THREADS) s_bkt[i] = qt->bkt[i];
    __syncthreads();
    uint32_t bad = 0;
    const uint64_t span = (uint64_t)hi - lo + 1;
    for (uint64_t i = (uint64_t)blockIdx.x * THREADS + threadIdx.x; i < span; i += (uint64_t)gridDim.x * THREADS) {
        const float x = __uint_as_float(lo + (uint32_t)i);
        bad += quantize_lookup(x, s_oct, s_bkt, true) != quantize_search(x, s1, true);
        bad += quantize_lookup(-x, s_oct, s_bkt, true) != quantize_search(-x, s1, true);
        bad += quantize_lookup(x, s_oct, s_bkt, false) != quantize_search(x, s2, false);
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
    const unsigned grid = grid_for(nblocks, QB_PER_WG, 256 * 8);
    const bool qtab = a.qtable != nullptr;
    if (mode == NOISE_TRITON) launch_quant_mode<NOISE_TRITON, BLOCK>(vec, qtab, a, s, grid, WG);
    else if (mode == NOISE_PHILOX8) launch_quant_mode<NOISE_PHILOX8, BLOCK>(vec, qtab, a, s, grid, WG);
    else launch_quant_mode<NOISE_INJECT, BLOCK>(vec, qtab, a, s, grid, WG);
}

extern "C" {

int msr_version(void) { return 100; }

const char *msr_last_error(void) { return g_err; }

int msr_sr_accum(uint16_t *acc, const void *grad, int32_t grad_is_f32, int64_t n, uint32_t seed, int32_t zero_init,
                 int32_t noise_mode, const uint16_t *inject, msr_stream_t stream) {
    if (n < 0 || (n > 0 && (!acc || !grad))) { set_error("msr_sr_accum: bad arguments"); return MSR_ERR_ARG; }
    MSR_CHECK_MODE(noise_mode, inject);
    if (n == 0) return MSR_OK;
    const Noise ns = make_noise(seed, 0, inject, n);
    const bool vec = aligned(acc, 16) && aligned(grad, 16);
    const unsigned grid = grid_for((n + 7) / 8, THREADS);
    hipStream_t s = (hipStream_t)stream;
#define LAUNCH_ACC(GF, Z, V)                                                                                   \
    MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((sr_accum_kernel<M, GF, Z, V>), dim3(grid), dim3(THREADS), 0, s, acc, grad, n, ns))
    if (grad_is_f32) {
        if (zero_init) { if (vec) { LAUNCH_ACC(true, true, true); } else { LAUNCH_ACC(true, true, false); } }
        else { if (vec) { LAUNCH_ACC(true, false, true); } else { LAUNCH_ACC(true, false, false); } }
    } else {
        if (zero_init) { if (vec) { LAUNCH_ACC(false, true, true); } else { LAUNCH_ACC(false, true, false); } }
        else { if (vec) { LAUNCH_ACC(false, false, true); } else { LAUNCH_ACC(false, false, false); } }
    }
#undef LAUNCH_ACC
    return check_launch("msr_sr_accum");
}

int msr_sr_accum_multi(const msr_accum_item *items, int32_t count, int32_t noise_mode, msr_stream_t stream) {
    if (count < 0 || (count > 0 && !items)) { set_error("msr_sr_accum_multi: bad arguments"); return MSR_ERR_ARG; }
    if (noise_mode != NOISE_TRITON && noise_mode != NOISE_PHILOX8) {
        set_error("msr_sr_accum_multi: noise_mode must be TRITON or PHILOX8 (got %d)", (int)noise_mode);
        return MSR_ERR_ARG;
    }
    for (int32_t i = 0; i < count; ++i) {
        const msr_accum_item &it = items[i];
        if (it.n < 0 || (it.n > 0 && (!it.acc || !it.grad)) ||
            (it.flags & ~(MSR_ACCUM_ZERO_INIT | MSR_ACCUM_GRAD_F32))) {
            set_error("msr_sr_accum_multi: bad item %d", (int)i);
            return MSR_ERR_ARG;
        }
    }
    hipStream_t s = (hipStream_t)stream;
    int32_t i = 0;
    while (i < count) {
        AccumMultiArgs a;
        a.count = 0;
        int64_t g = 0;
        for (; i < count && a.count < ACC_MAXT; ++i) {
            const msr_accum_item &it = items[i];
            if (it.n == 0) continue;
            const int t = a.count++;
            const bool f32 = (it.flags & MSR_ACCUM_GRAD_F32) != 0;
            a.gstart[t] = g;
            a.acc[t] = it.acc;
            a.grad[t] = it.grad;
            a.n[t] = it.n;
            a.key[t] = seed_key(it.seed, 0);
            a.flags[t] = ((it.flags & MSR_ACCUM_ZERO_INIT) ? ACC_ZERO : 0u) | (f32 ? ACC_F32 : 0u) |
                         ((aligned(it.acc, 16) && aligned(it.grad, 16)) ? ACC_VEC : 0u);
            g += (it.n + 7) / 8;
        }
        if (a.count == 0) break;
        a.gstart[a.count] = g;
        const unsigned grid = grid_for(g, THREADS);
        if (noise_mode == NOISE_TRITON)
            hipLaunchKernelGGL((sr_accum_multi_kernel<NOISE_TRITON>), dim3(grid), dim3(THREADS), 0, s, a);
        else
            hipLaunchKernelGGL((sr_accum_multi_kernel<NOISE_PHILOX8>), dim3(grid), dim3(THREADS), 0, s, a);
        const int rc = check_launch("msr_sr_accum_multi");
        if (rc) return rc;
    }
    return MSR_OK;
}

int msr_adamw_bf16_step(uint16_t *p, const uint16_t *g, uint16_t *ema, uint16_t *ema_sq, int64_t n, float lr,
                        float beta1, float beta2, float eps, float weight_decay, float bias_correction,
                        float bias_correction_sqrt, uint32_t seed, int32_t noise_mode, const uint16_t *inject,
                        msr_stream_t stream) {
    if (n < 0 || (n > 0 && (!p || !g || !ema || !ema_sq))) { set_error("msr_adamw_bf16_step: bad arguments"); return MSR_ERR_ARG; }
    MSR_CHECK_MODE(noise_mode, inject);
    if (n == 0) return MSR_OK;
    AdamWArgs a;
    a.p = p; a.g = g; a.ema = ema; a.ema_sq = ema_sq; a.n = n;
    a.lr = lr; a.beta1 = beta1; a.beta2 = beta2; a.eps = eps; a.wd = weight_decay;
    a.bc = bias_correction; a.bcs = bias_correction_sqrt;
    a.ns_ema = make_noise(seed, 0, inject, n);
    a.ns_ema_sq = make_noise(seed, 1, inject, n);
    a.ns_p = make_noise(seed, 2, inject, n);
    const bool vec = aligned(p, 16) && aligned(g, 16) && aligned(ema, 16) && aligned(ema_sq, 16);
    const unsigned grid = grid_for((n + 7) / 8, THREADS);
    hipStream_t s = (hipStream_t)stream;
    if (vec) { MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((adamw_bf16_kernel<M, true>), dim3(grid), dim3(THREADS), 0, s, a)); }
    else { MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((adamw_bf16_kernel<M, false>), dim3(grid), dim3(THREADS), 0, s, a)); }
    return check_launch("msr_adamw_bf16_step");
}

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
    Adam8Args a;
    a.p = p; a.g = g; a.s1 = state1; a.s2 = state2; a.absmax1 = absmax1; a.absmax2 = absmax2;
    a.qmap1 = qmap1; a.qmap2 = qmap2; a.n = n;
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

int msr_muon_prepare(const uint16_t *const *grads, uint16_t *buf, uint16_t *out, int64_t numel_each, int32_t count,
                     float beta, int32_t nesterov, uint32_t seed, int32_t noise_mode, const uint16_t *inject,
                     msr_stream_t stream) {
    if (numel_each < 0 || count < 0 || (numel_each > 0 && count > 0 && (!grads || !buf || !out))) {
        set_error("msr_muon_prepare: bad arguments");
        return MSR_ERR_ARG;
    }
    MSR_CHECK_MODE(noise_mode, inject);
    if (numel_each == 0 || count == 0) return MSR_OK;
    hipStream_t s = (hipStream_t)stream;
    const bool rows_aligned = (numel_each % 8) == 0 && aligned(buf, 16) && aligned(out, 16);
    for (int32_t c0 = 0; c0 < count; c0 += MAX_TABLE) {
        const int32_t cnt = (count - c0) < MAX_TABLE ? (count - c0) : MAX_TABLE;
        PrepareArgs a;
        bool vec = rows_aligned;
        for (int32_t i = 0; i < cnt; ++i) {
            if (!grads[c0 + i]) { set_error("msr_muon_prepare: null gradient pointer %d", (int)(c0 + i)); return MSR_ERR_ARG; }
            a.grads[i] = grads[c0 + i];
            vec = vec && aligned(grads[c0 + i], 16);
        }
        a.buf = buf + (int64_t)c0 * numel_each;
        a.out = out + (int64_t)c0 * numel_each;
        a.numel = numel_each;
        a.stack_off0 = (int64_t)c0 * numel_each;
        a.beta = beta;
        a.ns = make_noise(seed, 0, inject, 0);
        const unsigned gx = grid_for((numel_each + 7) / 8, THREADS, (256 * 32 + cnt - 1) / cnt);
        const dim3 grid(gx, (unsigned)cnt);
#define LAUNCH_PREP(NEST, V) MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((muon_prepare_kernel<M, NEST, V>), grid, dim3(THREADS), 0, s, a))
        if (nesterov) { if (vec) { LAUNCH_PREP(true, true); } else { LAUNCH_PREP(true, false); } }
        else { if (vec) { LAUNCH_PREP(false, true); } else { LAUNCH_PREP(false, false); } }
#undef LAUNCH_PREP
        int rc = check_launch("msr_muon_prepare");
        if (rc) return rc;
    }
    return MSR_OK;
}

int msr_muon_apply(uint16_t *const *params, const uint16_t *upd, int64_t numel_each, int32_t count, float lr,
                   float weight_decay, float scale, const uint32_t *seeds, int32_t noise_mode, const uint16_t *inject,
                   msr_stream_t stream) {
    if (numel_each < 0 || count < 0 || (numel_each > 0 && count > 0 && (!params || !upd || !seeds))) {
        set_error("msr_muon_apply: bad arguments");
        return MSR_ERR_ARG;
    }
    MSR_CHECK_MODE(noise_mode, inject);
    if (numel_each == 0 || count == 0) return MSR_OK;
    hipStream_t s = (hipStream_t)stream;
    const bool rows_aligned = (numel_each % 8) == 0 && aligned(upd, 16);
    for (int32_t c0 = 0; c0 < count; c0 += MAX_TABLE) {
        const int32_t cnt = (count - c0) < MAX_TABLE ? (count - c0) : MAX_TABLE;
        ApplyArgs a;
        bool vec = rows_aligned;
        for (int32_t i = 0; i < cnt; ++i) {
            if (!params[c0 + i]) { set_error("msr_muon_apply: null parameter pointer %d", (int)(c0 + i)); return MSR_ERR_ARG; }
            a.params[i] = params[c0 + i];
            a.seeds[i] = seeds[c0 + i];
            vec = vec && aligned(params[c0 + i], 16);
        }
        a.upd = upd + (int64_t)c0 * numel_each;
        a.numel = numel_each;
        a.lr = lr; a.wd = weight_decay; a.scale = scale;
        a.inject = inject ? inject + (int64_t)c0 * numel_each : nullptr;
        const unsigned gx = grid_for((numel_each + 7) / 8, THREADS, (256 * 32 + cnt - 1) / cnt);
        const dim3 grid(gx, (unsigned)cnt);
        if (vec) { MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((muon_apply_kernel<M, true>), grid, dim3(THREADS), 0, s, a)); }
        else { MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((muon_apply_kernel<M, false>), grid, dim3(THREADS), 0, s, a)); }
        int rc = check_launch("msr_muon_apply");
        if (rc) return rc;
    }
    return MSR_OK;
}

int msr_noise_fill(uint16_t *out, int64_t n, int64_t offset0, uint32_t seed, uint32_t k, int32_t noise_mode,
                   msr_stream_t stream) {
    if (n < 0 || (n > 0 && !out) || offset0 < 0) { set_error("msr_noise_fill: bad arguments"); return MSR_ERR_ARG; }
    if (noise_mode != NOISE_TRITON && noise_mode != NOISE_PHILOX8) { set_error("msr_noise_fill: mode must be 0 or 1"); return MSR_ERR_ARG; }
    if (n == 0) return MSR_OK;
    const Noise ns = make_noise(seed, k, nullptr, 0);
    const unsigned grid = grid_for(n, THREADS);
    hipStream_t s = (hipStream_t)stream;
    if (noise_mode == NOISE_TRITON) hipLaunchKernelGGL((noise_fill_kernel<NOISE_TRITON>), dim3(grid), dim3(THREADS), 0, s, out, n, offset0, ns);
    else hipLaunchKernelGGL((noise_fill_kernel<NOISE_PHILOX8>), dim3(grid), dim3(THREADS), 0, s, out, n, offset0, ns);
    return check_launch("msr_noise_fill");
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

}  // extern "C"
