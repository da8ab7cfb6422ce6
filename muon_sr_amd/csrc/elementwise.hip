// Memory-bound optimizer kernels for gfx950: SR gradient accumulation, bf16-
// moment AdamW and the Muon momentum/update passes (8-bit AdamW: adamw8bit.hip).
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
#include "vecio.hpp"
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


// ---------------------------------------------------------------------------
// (c) SR gradient accumulation   (muon_sr/triton_adamw.py:206-229)
// ---------------------------------------------------------------------------

// Many tensors in one launch (the hooks of a backward pass, deferred).  The
// launch's 8-element groups are cut into tiles of ACC_TILE groups that never
// cross a tensor: tensor t owns tiles [tstart[t], tstart[t+1]).  A work-group
// takes tiles in a grid-stride loop, finds the tile's tensor once (a
// wave-uniform search, so pointers, key and flags are uniform), and each
// thread loads ACC_U groups (one per ACC_THREADS-wide slice of the tile)
// before computing them.  A tensor's offsets, and so its noise counters,
// start at 0: the result equals one sr_accum_kernel launch per tensor.
constexpr int ACC_MAXT = 80;
// Tiles of 128 threads x 2 groups (2048 elements).  Measured on config 3's 217 tensors
// against 256 x 4: the per-hook launches (one per tensor) 7 % faster (256 x 1 and 256 x 2
// within 1 %, 256 x 8 12 % slower), the multi-tensor launch 2.2 % faster (256 x 2 and
// 512 x 2 0.4-1.0 %, 64 x 4 0.3 %).
#ifndef MSR_ACC_U
#define MSR_ACC_U 2
#endif
#ifndef MSR_ACC_THREADS
#define MSR_ACC_THREADS 128
#endif
constexpr int ACC_THREADS = MSR_ACC_THREADS, ACC_U = MSR_ACC_U, ACC_TILE = ACC_THREADS * ACC_U;
constexpr uint32_t ACC_ZERO = 1, ACC_F32 = 2, ACC_VEC = 4;
struct AccumMultiArgs {
    int count;
    int64_t tstart[ACC_MAXT + 1];
    uint16_t *acc[ACC_MAXT];
    const void *grad[ACC_MAXT];
    int64_t n[ACC_MAXT];
    PhiloxKey key[ACC_MAXT];
    uint32_t flags[ACC_MAXT];
};

// ACC_U groups of one tile of one tensor: loads first, then SR sums and stores.
template <int MODE, bool GF32, bool ZERO, bool VEC>
__device__ __forceinline__ void accum_tile(uint16_t *__restrict__ acc, const void *__restrict__ grad, const Noise &ns,
                                           int64_t n, int64_t g0) {
    uint32_t wa[ACC_U][4], wg[ACC_U][4];
    float gf[ACC_U][8];
    int valid[ACC_U];
#pragma unroll
    for (int u = 0; u < ACC_U; ++u) {
        const int64_t o0 = (g0 + u * ACC_THREADS + threadIdx.x) * 8;
        valid[u] = clamp_valid(n, o0);
        if constexpr (!ZERO) load_bf16x8<VEC>(acc, o0, valid[u], wa[u]);
        if constexpr (GF32) load_f32x8<VEC>(static_cast<const float *>(grad), o0, valid[u], gf[u]);
        else load_bf16x8<VEC>(static_cast<const uint16_t *>(grad), o0, valid[u], wg[u]);
    }
#pragma unroll
    for (int u = 0; u < ACC_U; ++u) {
        if (valid[u] == 0) continue;
        const int64_t o0 = (g0 + u * ACC_THREADS + threadIdx.x) * 8;
        float a[8], g[8];
        if constexpr (ZERO) {
#pragma unroll
            for (int j = 0; j < 8; ++j) a[j] = 0.0f;
        } else {
            unpack8(wa[u], a);
        }
        if constexpr (GF32) {
#pragma unroll
            for (int j = 0; j < 8; ++j) g[j] = gf[u][j];
        } else {
            unpack8(wg[u], g);
        }
        uint32_t r[8];
        noise8<MODE>(ns, o0, valid[u], r);
        uint32_t out[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            out[j] = pack2(sr_bf16(a[2 * j] + g[2 * j], r[2 * j]), sr_bf16(a[2 * j + 1] + g[2 * j + 1], r[2 * j + 1]));
        store_bf16x8<VEC>(acc, o0, valid[u], out);
    }
}

// One tensor: tiles of ACC_TILE groups, one work-group per tile (grid-stride
// beyond the launch's grid).
template <int MODE, bool GF32, bool ZERO, bool VEC>
__global__ __launch_bounds__(ACC_THREADS) void sr_accum_kernel(uint16_t *__restrict__ acc, const void *__restrict__ grad,
                                                              int64_t n, Noise ns) {
    const int64_t tiles = ((n + 7) / 8 + ACC_TILE - 1) / ACC_TILE;
    for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x)
        accum_tile<MODE, GF32, ZERO, VEC>(acc, grad, ns, n, tile * ACC_TILE);
}

// The multi-tensor launch takes its tiles in runs of MSR_ACC_XCD consecutive tiles per XCD
// (128 tiles: 512 KiB of bf16 accumulator), 0.7 % faster than tiles in dispatch order (runs
// of 16 tiles 5 % slower, 32 and 64 equal; with 16 KiB tiles of 256 x 4 groups, runs of 32
// measured 1.4 %); bit-exact.  The one-tensor launches of the per-hook path keep the
// dispatch order (runs of 32 tiles of 256 x 4 groups measured 5 % slower there).
#ifndef MSR_ACC_XCD
#define MSR_ACC_XCD 128
#endif

template <int MODE>
__global__ __launch_bounds__(ACC_THREADS) void sr_accum_multi_kernel(AccumMultiArgs a) {
    const int64_t total = a.tstart[a.count];
    for (int64_t tile = xcd_place(blockIdx.x, gridDim.x, MSR_ACC_XCD); tile < total; tile += gridDim.x) {
        int lo = 0, hi = a.count - 1;   // last t with tstart[t] <= tile (uniform)
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (a.tstart[mid] <= tile) lo = mid; else hi = mid - 1;
        }
        const int t = lo;
        const int64_t g0 = (tile - a.tstart[t]) * ACC_TILE;
        Noise ns;
        ns.key = a.key[t];
        ns.inject = nullptr;
        uint16_t *acc = a.acc[t];
        const void *grad = a.grad[t];
        const int64_t n = a.n[t];
        switch (a.flags[t]) {
            case 0: accum_tile<MODE, false, false, false>(acc, grad, ns, n, g0); break;
            case ACC_ZERO: accum_tile<MODE, false, true, false>(acc, grad, ns, n, g0); break;
            case ACC_F32: accum_tile<MODE, true, false, false>(acc, grad, ns, n, g0); break;
            case ACC_F32 | ACC_ZERO: accum_tile<MODE, true, true, false>(acc, grad, ns, n, g0); break;
            case ACC_VEC: accum_tile<MODE, false, false, true>(acc, grad, ns, n, g0); break;
            case ACC_VEC | ACC_ZERO: accum_tile<MODE, false, true, true>(acc, grad, ns, n, g0); break;
            case ACC_VEC | ACC_F32: accum_tile<MODE, true, false, true>(acc, grad, ns, n, g0); break;
            default: accum_tile<MODE, true, true, true>(acc, grad, ns, n, g0); break;
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
// Muon prepare / apply   (muon_sr/triton_muon_sr.py:18-80)
// ---------------------------------------------------------------------------

constexpr int MAX_TABLE = 240;  // pointers per launch (kernel-argument table)

struct PrepareArgs {
    const void *grads[MAX_TABLE];   // bf16, or fp32 (G32)
    uint16_t *buf;       // stack base (already offset to the first matrix of this launch)
    uint16_t *out;
    int64_t numel;
    int64_t stack_off0;  // stack offset of matrix 0 of this launch (noise counter base)
    float beta;
    Noise ns;
};

// G32: fp32 gradients, read as fp32 (the reference's kernel loads the gradient in its
// own dtype, muon_sr/triton_muon_sr.py:34)
template <int MODE, bool NEST, bool VEC, bool G32>
__global__ __launch_bounds__(THREADS) void muon_prepare_kernel(PrepareArgs a) {
    const int i = blockIdx.y;
    const void *g = a.grads[i];
    uint16_t *buf = a.buf + (int64_t)i * a.numel;
    uint16_t *out = a.out + (int64_t)i * a.numel;
    const int64_t base = a.stack_off0 + (int64_t)i * a.numel;
    const float one_m_beta = 1.0f - a.beta;
    const int64_t groups = (a.numel + 7) >> 3;
    for (int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x; t < groups; t += (int64_t)gridDim.x * THREADS) {
        const int64_t o0 = t << 3;
        const int valid = clamp_valid(a.numel, o0);
        uint32_t wg[4], wb[4];
        float gf[8], bf[8];
        if constexpr (G32) {
            load_f32x8<VEC>(static_cast<const float *>(g), o0, valid, gf);
        } else {
            load_bf16x8<VEC>(static_cast<const uint16_t *>(g), o0, valid, wg);
            unpack8(wg, gf);
        }
        load_bf16x8<VEC>(buf, o0, valid, wb);
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
            float nb, upd;
            muon_momentum<NEST>(gf[j], bf[j], a.beta, one_m_beta, nb, upd);   // :37-42
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

#ifndef MSR_ACC_GRID_CAP
#define MSR_ACC_GRID_CAP (1 << 20)   // one work-group per tile: measured best
#endif

extern "C" {

int msr_version(void) { return 100; }

const char *msr_last_error(void) { return g_err; }

int msr_sr_accum(uint16_t *acc, const void *grad, int32_t grad_is_f32, int64_t n, uint32_t seed, int32_t zero_init,
                 int32_t noise_mode, const uint16_t *inject, msr_stream_t stream) {
    if (n < 0 || (n > 0 && (!acc || !grad))) { set_error("msr_sr_accum: bad arguments"); return MSR_ERR_ARG; }
    MSR_CHECK_MODE(noise_mode, inject);
    if (partial_overlap(acc, 2 * (size_t)n, grad, (grad_is_f32 ? 4 : 2) * (size_t)n)) {
        set_error("msr_sr_accum: acc and grad overlap");
        return MSR_ERR_OVERLAP;
    }
    if (n == 0) return MSR_OK;
    const Noise ns = make_noise(seed, 0, inject, n);
    const bool vec = aligned(acc, 16) && aligned(grad, 16);
    const int64_t tiles = ((n + 7) / 8 + ACC_TILE - 1) / ACC_TILE;
    const unsigned grid = (unsigned)(tiles < MSR_ACC_GRID_CAP ? tiles : MSR_ACC_GRID_CAP);
    hipStream_t s = (hipStream_t)stream;
#define LAUNCH_ACC(GF, Z, V)                                                                                   \
    MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((sr_accum_kernel<M, GF, Z, V>), dim3(grid), dim3(ACC_THREADS), 0, s, acc, grad, n, ns))
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
        int64_t g = 0;   // tiles
        for (; i < count && a.count < ACC_MAXT; ++i) {
            const msr_accum_item &it = items[i];
            if (it.n == 0) continue;
            const bool f32 = (it.flags & MSR_ACCUM_GRAD_F32) != 0;
            // items of one launch run concurrently: an accumulator may share memory
            // with no other operand of the launch (its own gradient aside, in place)
            const size_t ab = 2 * (size_t)it.n, gb = (f32 ? 4 : 2) * (size_t)it.n;
            bool race = partial_overlap(it.acc, ab, it.grad, gb);
            for (int u = 0; u < a.count && !race; ++u) {
                const size_t ub = 2 * (size_t)a.n[u];
                const size_t ug = ((a.flags[u] & ACC_F32) ? 4 : 2) * (size_t)a.n[u];
                race = (uintptr_t)it.acc < (uintptr_t)a.acc[u] + ub && (uintptr_t)a.acc[u] < (uintptr_t)it.acc + ab;
                race = race || ((uintptr_t)it.acc < (uintptr_t)a.grad[u] + ug && (uintptr_t)a.grad[u] < (uintptr_t)it.acc + ab);
                race = race || ((uintptr_t)a.acc[u] < (uintptr_t)it.grad + gb && (uintptr_t)it.grad < (uintptr_t)a.acc[u] + ub);
            }
            if (race) {
                set_error("msr_sr_accum_multi: item %d overlaps another operand of its launch", (int)i);
                return MSR_ERR_OVERLAP;
            }
            const int t = a.count++;
            a.tstart[t] = g;
            a.acc[t] = it.acc;
            a.grad[t] = it.grad;
            a.n[t] = it.n;
            a.key[t] = seed_key(it.seed, 0);
            a.flags[t] = ((it.flags & MSR_ACCUM_ZERO_INIT) ? ACC_ZERO : 0u) | (f32 ? ACC_F32 : 0u) |
                         ((aligned(it.acc, 16) && aligned(it.grad, 16)) ? ACC_VEC : 0u);
            g += ((it.n + 7) / 8 + ACC_TILE - 1) / ACC_TILE;
        }
        if (a.count == 0) break;
        a.tstart[a.count] = g;
        const unsigned grid = (unsigned)(g < MSR_ACC_GRID_CAP ? g : MSR_ACC_GRID_CAP);
        if (noise_mode == NOISE_TRITON)
            hipLaunchKernelGGL((sr_accum_multi_kernel<NOISE_TRITON>), dim3(grid), dim3(ACC_THREADS), 0, s, a);
        else
            hipLaunchKernelGGL((sr_accum_multi_kernel<NOISE_PHILOX8>), dim3(grid), dim3(ACC_THREADS), 0, s, a);
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
    {
        const void *ops[4] = {p, g, ema, ema_sq};
        for (int i = 0; i < 4; ++i)
            for (int j = i + 1; j < 4; ++j)
                if (partial_overlap(ops[i], 2 * (size_t)n, ops[j], 2 * (size_t)n)) {
                    set_error("msr_adamw_bf16_step: operands %d and %d overlap", i, j);
                    return MSR_ERR_OVERLAP;
                }
    }
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

int msr_muon_prepare(const void *const *grads, int32_t grad_is_f32, uint16_t *buf, uint16_t *out, int64_t numel_each,
                     int32_t count, float beta, int32_t nesterov, uint32_t seed, int32_t noise_mode,
                     const uint16_t *inject, msr_stream_t stream) {
    if (numel_each < 0 || count < 0 || (numel_each > 0 && count > 0 && (!grads || !buf || !out))) {
        set_error("msr_muon_prepare: bad arguments");
        return MSR_ERR_ARG;
    }
    MSR_CHECK_MODE(noise_mode, inject);
    if (numel_each == 0 || count == 0) return MSR_OK;
    {
        const size_t sb = 2 * (size_t)numel_each * (size_t)count, eb = (grad_is_f32 ? 4 : 2) * (size_t)numel_each;
        bool race = (uintptr_t)buf < (uintptr_t)out + sb && (uintptr_t)out < (uintptr_t)buf + sb;
        for (int32_t i = 0; i < count && !race; ++i)
            race = grads[i] && (partial_overlap(grads[i], eb, buf, sb) || partial_overlap(grads[i], eb, out, sb));
        if (race) { set_error("msr_muon_prepare: gradients, momentum stack and update stack must not overlap"); return MSR_ERR_OVERLAP; }
    }
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
#define LAUNCH_PREP(NEST, V, G) MSR_DISPATCH_NOISE(noise_mode, M, hipLaunchKernelGGL((muon_prepare_kernel<M, NEST, V, G>), grid, dim3(THREADS), 0, s, a))
        if (grad_is_f32) {
            if (nesterov) { if (vec) { LAUNCH_PREP(true, true, true); } else { LAUNCH_PREP(true, false, true); } }
            else { if (vec) { LAUNCH_PREP(false, true, true); } else { LAUNCH_PREP(false, false, true); } }
        } else {
            if (nesterov) { if (vec) { LAUNCH_PREP(true, true, false); } else { LAUNCH_PREP(true, false, false); } }
            else { if (vec) { LAUNCH_PREP(false, true, false); } else { LAUNCH_PREP(false, false, false); } }
        }
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
    {
        // the parameters of one launch are written concurrently: they may share
        // memory neither with each other nor with the update stack
        const size_t eb = 2 * (size_t)numel_each, ub = eb * (size_t)count;
        for (int32_t i = 0; i < count; ++i) {
            if (!params[i]) { set_error("msr_muon_apply: null parameter pointer %d", (int)i); return MSR_ERR_ARG; }
            bool race = (uintptr_t)params[i] < (uintptr_t)upd + ub && (uintptr_t)upd < (uintptr_t)params[i] + eb;
            for (int32_t j = 0; j < i && !race; ++j)
                race = (uintptr_t)params[i] < (uintptr_t)params[j] + eb && (uintptr_t)params[j] < (uintptr_t)params[i] + eb;
            if (race) { set_error("msr_muon_apply: parameter %d overlaps another parameter or the update stack", (int)i); return MSR_ERR_OVERLAP; }
        }
    }
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

}  // extern "C"
