/*
 * oracle.c -- CPU restatement of the muon_sr optimizer-step kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path (muon_sr_amd/) never calls
 * it and has no CPU fallback.
 *
 * Numerical contract: every expression is evaluated in IEEE binary32, one
 * rounding per operation, left to right as written in the reference, with no
 * FMA contraction (build with -ffp-contract=off), correctly rounded / and sqrt,
 * and denormals preserved.  This is the order the Triton interpreter evaluates
 * the reference kernels in, which is how the committed golden vectors were made.
 *
 * Each function names the reference lines it restates.  Paths are relative to
 * the reference checkout (bab2min/muon_sr 0.1.2) and to the installed
 * triton-rocm 3.6.0 package for the Philox generator.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Threads the block loop of orc_adamw8bit runs on. */
int32_t orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* bf16 helpers                                                              */
/* ------------------------------------------------------------------------ */

static inline float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bf16_to_f32(uint16_t h) { return f32_from_bits(((uint32_t)h) << 16); }

/* Round-to-nearest-even fp32 -> bf16 (the default rounding of a Triton
 * fp32->bf16 cast, triton/language/semantic.py:805-809).  NaN maps to a quiet
 * NaN of the same sign. */
uint16_t orc_bf16_rne(float x)
{
    uint32_t u = bits_from_f32(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

/* Stochastic rounding as the reference writes it (e.g.
 * muon_sr/triton_adamw.py:57-59): add the 16 noise bits to the fp32 bit
 * pattern as an int32 (wrapping) and keep the high half. */
static inline uint16_t sr_bf16(float x, uint32_t noise16)
{
    uint32_t u = bits_from_f32(x);
    return (uint16_t)(((u + noise16) & 0xffff0000u) >> 16);
}

/* ------------------------------------------------------------------------ */
/* Philox4x32-10, as triton/language/random.py:12-41 (philox_impl) runs it.   */
/* ------------------------------------------------------------------------ */

static inline uint32_t mulhi32(uint32_t a, uint32_t b)
{
    return (uint32_t)(((uint64_t)a * (uint64_t)b) >> 32);
}

void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4])
{
    const uint32_t KA = 0x9E3779B9u, KB = 0xBB67AE85u;
    const uint32_t RA = 0xD2511F53u, RB = 0xCD9E8D57u;
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; ++r) {
        uint32_t o0 = c0, o2 = c2;
        c0 = mulhi32(RB, o2) ^ c1 ^ k0;
        c2 = mulhi32(RA, o0) ^ c3 ^ k1;
        c1 = RB * o2;
        c3 = RA * o0;
        k0 += KA;
        k1 += KB;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* Seed -> Philox key for the stream `seed + k`.
 * A compiled Triton launch types an integer argument i32 when it lies in
 * [-2^31, 2^31) and i64 when it lies in [2^31, 2^63) (the 'i32'/'i64' of
 * triton.runtime.jit.mangle_type).  `SEED + k` is evaluated in that type and
 * widened to u64 (sign extension for i32), whose halves are the Philox key
 * (triton/language/random.py:49-60).  So an i32 seed that wraps past 2^31-1
 * gets the high word 0xFFFFFFFF, and an i64 seed that passes 2^32-1 gets 1. */
void orc_seed_key(uint32_t seed, uint32_t k, uint32_t key[2])
{
    if (seed < 0x80000000u) {
        uint32_t lo = seed + k;
        key[0] = lo;
        key[1] = (lo >= 0x80000000u) ? 0xffffffffu : 0u;
    } else {
        uint64_t v = (uint64_t)seed + k;
        key[0] = (uint32_t)v;
        key[1] = (uint32_t)(v >> 32);
    }
}

/* A noise source for one SR stream. */
enum { NOISE_TRITON = 0, NOISE_PHILOX8 = 1, NOISE_INJECT = 2 };

typedef struct {
    int32_t mode;          /* NOISE_* */
    uint32_t key_lo;       /* Philox key (from orc_seed_key) */
    uint32_t key_hi;
    const uint16_t *inject;/* NOISE_INJECT: noise[offset] */
} orc_noise_t;

/* 16 noise bits for element `offset` of a launch.
 *  - NOISE_TRITON: word 0 of Philox(ctr=(offset mod 2^32, 0, 0, 0), key), as
 *    tl.randint(seed, offset) with an int32 offset (random.py:76-110); the
 *    reference keeps `& 0xFFFF` of it (e.g. muon_sr/triton_adamw.py:58).
 *  - NOISE_PHILOX8: this library's own counter-based stream: one Philox call
 *    per 8 consecutive elements, counter (offset>>3 low, offset>>35, 0, 0),
 *    16-bit lane (offset & 7) of the 128-bit output.
 *  - NOISE_INJECT: caller-provided noise (tests). */
uint32_t orc_noise16(const orc_noise_t *ns, int64_t offset)
{
    uint32_t key[2] = {ns->key_lo, ns->key_hi};
    uint32_t out[4];
    if (ns->mode == NOISE_INJECT) return ns->inject[offset];
    if (ns->mode == NOISE_TRITON) {
        uint32_t ctr[4] = {(uint32_t)(uint64_t)offset, 0u, 0u, 0u};
        orc_philox4x32_10(ctr, key, out);
        return out[0] & 0xffffu;
    }
    {
        uint64_t o = (uint64_t)offset;
        uint32_t ctr[4] = {(uint32_t)(o >> 3), (uint32_t)(o >> 35), 0u, 0u};
        unsigned lane = (unsigned)(o & 7u);
        orc_philox4x32_10(ctr, key, out);
        return (out[lane >> 1] >> (16u * (lane & 1u))) & 0xffffu;
    }
}

/* ------------------------------------------------------------------------ */
/* SR gradient accumulation: muon_sr/triton_adamw.py:206-229                  */
/* ------------------------------------------------------------------------ */

/* acc <- SR(f32(acc) + f32(grad)).  grad is bf16 (grad_is_f32 = 0) or fp32. */
void orc_sr_accum(uint16_t *acc, const void *grad, int32_t grad_is_f32, int64_t n,
                  const orc_noise_t *ns)
{
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n; ++o) {
        float a = bf16_to_f32(acc[o]);
        float g = grad_is_f32 ? ((const float *)grad)[o] : bf16_to_f32(((const uint16_t *)grad)[o]);
        float s = a + g;
        acc[o] = sr_bf16(s, orc_noise16(ns, o));
    }
}

/* ------------------------------------------------------------------------ */
/* BF16-moment AdamW (PyTorch order): muon_sr/triton_adamw.py:9-72            */
/* ------------------------------------------------------------------------ */

void orc_adamw_bf16(uint16_t *p, const uint16_t *g, uint16_t *ema, uint16_t *ema_sq, int64_t n,
                    float lr, float beta1, float beta2, float eps, float weight_decay,
                    float bias_correction, float bias_correction_sqrt,
                    const orc_noise_t *ns_ema, const orc_noise_t *ns_ema_sq,
                    const orc_noise_t *ns_p)
{
    const float one_m_b1 = 1.0f - beta1;                       /* :37 */
    const float one_m_b2 = 1.0f - beta2;                       /* :38 */
    const float step_size = lr / bias_correction;              /* :41 */
    const float decay = 1.0f - lr * weight_decay;              /* :45 */
    for (int64_t o = 0; o < n; ++o) {
        float pf = bf16_to_f32(p[o]);
        float gf = bf16_to_f32(g[o]);
        float e = bf16_to_f32(ema[o]);
        float s = bf16_to_f32(ema_sq[o]);
        e = beta1 * e + one_m_b1 * gf;                         /* :37 */
        s = beta2 * s + (one_m_b2 * gf) * gf;                  /* :38 */
        float denom = sqrtf(s) / bias_correction_sqrt + eps;   /* :42 */
        pf = pf * decay;                                       /* :45 */
        pf = pf - (step_size * e) / denom;                     /* :48 */
        ema[o] = sr_bf16(e, orc_noise16(ns_ema, o));           /* :52,57-59,70 */
        ema_sq[o] = sr_bf16(s, orc_noise16(ns_ema_sq, o));     /* :53,61-63,71 */
        p[o] = sr_bf16(pf, orc_noise16(ns_p, o));              /* :54,65-67,72 */
    }
}

/* ------------------------------------------------------------------------ */
/* 8-bit blockwise AdamW: muon_sr/triton_adamw_8bit.py:27-99                  */
/* ------------------------------------------------------------------------ */

/* The quantizer search exactly as muon_sr/triton_adamw_8bit.py:27-53 runs it. */
uint8_t orc_quantize_one(float x, const float *Q, int32_t is_signed)
{
    int32_t pivot = 127, lower_pivot = 0, upper_pivot = 255;
    float lower = is_signed ? -1.0f : 0.0f;
    float upper = 1.0f;
    float val = Q[pivot];
    for (int shift = 0; shift < 7; ++shift) {
        int32_t delta = 64 >> shift;
        int right = x > val;
        if (right) { lower_pivot = pivot; lower = val; }
        else { upper_pivot = pivot; upper = val; }
        pivot += right ? delta : -delta;
        val = Q[pivot];
    }
    int32_t result;
    if (x > val) result = (x > (upper + val) * 0.5f) ? upper_pivot : pivot;
    else result = (x < (lower + val) * 0.5f) ? lower_pivot : pivot;
    if (is_signed) {
        float decoded = Q[result];
        int mismatch = (decoded < 0.0f) != (x < 0.0f);
        if (mismatch) result += (x > 0.0f) ? 1 : -1;
    }
    return (uint8_t)result;
}

void orc_quantize(const float *x, int64_t n, const float *Q, int32_t is_signed, uint8_t *out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_quantize_one(x[i], Q, is_signed);
}

/* One optimizer step on one parameter (both QUANTIZED variants).
 * quantized != 0: m8/v8 uint8 codes with absmax1/absmax2 per block, qmaps Q1/Q2.
 * quantized == 0: m16/v16 bf16 moments with SR streams ns_m / ns_v. */
void orc_adamw8bit(uint16_t *p, const uint16_t *g,
                   uint8_t *m8, uint8_t *v8, float *absmax1, float *absmax2,
                   const float *Q1, const float *Q2,
                   uint16_t *m16, uint16_t *v16,
                   int64_t n, int32_t block, int32_t quantized,
                   float LR, float B1, float B2, float EPS, float WD, float BC1, float BC2,
                   const orc_noise_t *ns_p, const orc_noise_t *ns_m, const orc_noise_t *ns_v)
{
    const float one_m_b1 = 1.0f - B1;
    const float one_m_b2 = 1.0f - B2;
    const float sqrt_bc2 = sqrtf(BC2);
    const float step_c = (LR * sqrt_bc2) / BC1;                 /* :81 */
    const float eps_c = sqrt_bc2 * EPS;                         /* :81 */
    const float decay = 1.0f - LR * WD;                         /* :81 */
    int64_t nblocks = (n + block - 1) / block;
    /* blocks are independent (the noise is a function of the element offset) */
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nblocks; ++b) {
        float mnew[4096], vnew[4096];
        float m_max = 0.0f, v_max = 0.0f;
        for (int32_t i = 0; i < block; ++i) {
            int64_t o = b * (int64_t)block + i;
            int valid = o < n;
            float pf = valid ? bf16_to_f32(p[o]) : 0.0f;        /* :60 */
            float gf = valid ? bf16_to_f32(g[o]) : 0.0f;        /* :61 */
            float m, v;
            if (quantized) {
                int32_t mc = valid ? m8[o] : 127;               /* :63 */
                int32_t vc = valid ? v8[o] : 0;                 /* :64 */
                m = Q1[mc] * absmax1[b];                        /* :65 */
                v = Q2[vc] * absmax2[b];                        /* :66 */
            } else {
                m = valid ? bf16_to_f32(m16[o]) : 0.0f;         /* :68 */
                v = valid ? bf16_to_f32(v16[o]) : 0.0f;         /* :69 */
            }
            int finite = fabsf(gf) < INFINITY;                  /* :70 */
            m = finite ? B1 * m + one_m_b1 * gf : 0.0f;         /* :71 */
            v = finite ? B2 * v + (one_m_b2 * gf) * gf : 0.0f;  /* :72 */
            float upd = (pf - (step_c * m) / (sqrtf(v) + eps_c)) * decay;   /* :74 */
            if (valid) {
                uint16_t rounded = sr_bf16(upd, orc_noise16(ns_p, o));      /* :75-77 */
                p[o] = finite ? rounded : p[o];                              /* :78 */
            }
            mnew[i] = m;
            vnew[i] = v;
            if (quantized && valid) {                           /* :80-81 */
                float am = fabsf(m), av = fabsf(v);
                if (am > m_max) m_max = am;
                if (av > v_max) v_max = av;
            }
            if (!quantized && valid) {                          /* :90-99 */
                m16[o] = sr_bf16(m, orc_noise16(ns_m, o));
                v16[o] = sr_bf16(v, orc_noise16(ns_v, o));
            }
        }
        if (quantized) {
            float md = m_max > 0.0f ? m_max : 1.0f;             /* :82 */
            float vd = v_max > 0.0f ? v_max : 1.0f;             /* :83 */
            for (int32_t i = 0; i < block; ++i) {
                int64_t o = b * (int64_t)block + i;
                if (o >= n) break;
                m8[o] = orc_quantize_one(mnew[i] / md, Q1, 1);  /* :82,84 */
                v8[o] = orc_quantize_one(vnew[i] / vd, Q2, 0);  /* :83,85 */
            }
            absmax1[b] = m_max;                                 /* :86 */
            absmax2[b] = v_max;                                 /* :87 */
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Muon elementwise kernels: muon_sr/triton_muon_sr.py:18-80                  */
/* ------------------------------------------------------------------------ */

/* _muon_prepare_kernel (:18-50).  Writes buf <- SR(new_buf) and the pre-NS
 * update both unrounded (out_f32, may be NULL) and RNE-rounded to bf16
 * (out_bf16, may be NULL).  The noise offset is the element's position in the
 * launch (the whole stack in the batched path, :154-159); NOISE_TRITON keeps
 * its low 32 bits as the reference's `offsets.to(tl.int32)` does (:44). */
void orc_muon_prepare(const void *g, int32_t g_is_f32, uint16_t *buf, float *out_f32, uint16_t *out_bf16,
                      int64_t n, float beta, int32_t nesterov, const orc_noise_t *ns)
{
    const float one_m_beta = 1.0f - beta;
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n; ++o) {
        /* the gradient in its own dtype (:34): bf16, or fp32 on the per-parameter path */
        float gf = g_is_f32 ? ((const float *)g)[o] : bf16_to_f32(((const uint16_t *)g)[o]);
        float bf = bf16_to_f32(buf[o]);
        float nb = bf + one_m_beta * (gf - bf);                 /* :37 */
        float upd = nesterov ? gf + beta * (nb - gf) : nb;      /* :39-42 */
        buf[o] = sr_bf16(nb, orc_noise16(ns, o));               /* :44-49 */
        if (out_f32) out_f32[o] = upd;
        if (out_bf16) out_bf16[o] = orc_bf16_rne(upd);          /* :50 */
    }
}

/* _muon_apply_kernel (:53-80). */
void orc_muon_apply(uint16_t *p, const uint16_t *upd, int64_t n, float lr, float weight_decay,
                    float scale, const orc_noise_t *ns)
{
    const float decay = 1.0f - lr * weight_decay;              /* :72 */
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n; ++o) {
        float pf = bf16_to_f32(p[o]);
        float u = bf16_to_f32(upd[o]) * scale;                  /* :70 */
        pf = pf * decay;                                        /* :72 */
        pf = pf - lr * u;                                       /* :73 */
        p[o] = sr_bf16(pf, orc_noise16(ns, o));                 /* :75-80 */
    }
}

/* Vectorised helpers for the Python side of the oracle. */
void orc_noise16_batch(const orc_noise_t *ns, const int64_t *offsets, int64_t n, uint16_t *out)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = (uint16_t)orc_noise16(ns, offsets[i]);
}

void orc_bf16_rne_batch(const float *x, int64_t n, uint16_t *out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_rne(x[i]);
}
