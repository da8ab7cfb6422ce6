/*
 * muon_sr_amd.h -- C ABI of libmuon_sr_amd.so, the MI355X (gfx950) kernels of
 * the muon_sr optimizer-step hot path.
 *
 * Conventions (every entry point):
 *  - All pointers are device pointers unless documented as host arrays; the
 *    library never allocates or frees device memory (workspace comes from the
 *    caller, sized by the matching *_workspace_bytes query).
 *  - bf16 tensors are passed as uint16_t bit patterns, contiguous.
 *  - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the
 *    default stream).  Nothing synchronises.
 *  - Return 0 on success, else a hipError_t or one of the MSR_ERR_* codes
 *    below; msr_last_error() returns a message for the calling thread.
 *  - fp32 scalars are the reference's Python floats rounded to fp32, as a
 *    compiled Triton launch passes them.  Seeds are the reference's 32-bit
 *    seeds; the library derives each stream's Philox key (SEED + k typing).
 *  - noise_mode selects the stochastic-rounding noise source:
 *      MSR_NOISE_TRITON  word 0 of Philox4x32-10 at counter (offset, 0, 0, 0):
 *                        the same bits the reference's tl.randint produces;
 *      MSR_NOISE_PHILOX8 one Philox4x32-10 call per 8 consecutive offsets
 *                        (16 bits each): this library's fast stream;
 *      MSR_NOISE_INJECT  noise read from `inject` (uint16 [streams][n]); tests.
 *  - Entry points keep no global mutable state and are safe to call from
 *    several host threads (autograd hooks run on the engine thread).
 */
#ifndef MUON_SR_AMD_H
#define MUON_SR_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *msr_stream_t; /* == hipStream_t */

#define MSR_NOISE_TRITON 0
#define MSR_NOISE_PHILOX8 1
#define MSR_NOISE_INJECT 2

#define MSR_ERR_ARG 1001
#define MSR_ERR_ALIGN 1002
#define MSR_ERR_LAUNCH 1003
#define MSR_ERR_WORKSPACE 1004
#define MSR_ERR_OVERLAP 1005   /* operands overlap without being the same buffer (a data race) */

/* Library version (major*10000 + minor*100 + patch) and error text. */
int msr_version(void);
const char *msr_last_error(void);

/* ---------------------------------------------------------------------------
 * (c) SR gradient accumulation.
 * Replaces the _grad_accum_kernel launches of TritonSRAccumulator._accum_hook
 * (muon_sr/triton_adamw.py:206-229, launched at :260 and :264).
 *   acc[i] <- SR_bf16(f32(acc[i]) + f32(grad[i])),  noise offset i.
 * grad_is_f32: 0 = bf16 grad, 1 = fp32 grad.
 * zero_init != 0 treats acc as zero on input (fuses the zeros_like at :263);
 * acc is then write-only.  inject: uint16 [n].
 * ------------------------------------------------------------------------- */
int msr_sr_accum(uint16_t *acc, const void *grad, int32_t grad_is_f32, int64_t n, uint32_t seed,
                 int32_t zero_init, int32_t noise_mode, const uint16_t *inject, msr_stream_t stream);

/* (c) SR accumulation fused with the weight-gradient GEMM of a linear layer
 * y = x W^T: the bf16 weight gradient dW = dy^T x that autograd hands the
 * accumulation hook (muon_sr/triton_adamw.py:252-265) is accumulated into acc
 * as the hook's _grad_accum_kernel (:206-229) does, without being written:
 *   acc[o][i] <- SR_bf16( f32(acc[o][i]) + f32(RNE_bf16( sum_t dy[t][o] x[t][i] )) )
 * (fp32 products accumulated in fp32; noise of element offset o * in + i, as
 * msr_sr_accum on the contiguous [out][in] buffer).  No counterpart in the
 * reference, which runs the GEMM and the accumulation separately.
 * x: bf16 [tokens][in] (row stride ldx), dy: bf16 [tokens][out] (ldy), acc:
 * bf16 [out][in] contiguous; in and out multiples of 256, tokens a multiple of
 * 128 (else MSR_ERR_ARG: use the GEMM and msr_sr_accum).  zero_init, seed,
 * noise_mode and inject as msr_sr_accum. */
int msr_linear_wgrad_sr_accum(uint16_t *acc, const uint16_t *x, int64_t ldx, const uint16_t *dy, int64_t ldy,
                              int64_t tokens, int64_t in_features, int64_t out_features, uint32_t seed,
                              int32_t zero_init, int32_t noise_mode, const uint16_t *inject, msr_stream_t stream);

/* (c) SR gradient accumulation of many tensors in one launch.
 * Same arithmetic and noise as one msr_sr_accum call per item (noise offsets
 * restart at 0 in every tensor), for the hooks of one backward pass collected
 * by TritonSRAccumulator (muon_sr/triton_adamw.py:252-265, one launch per
 * parameter in the reference).  items: HOST array; any count (split into
 * launches internally).  noise_mode: MSR_NOISE_TRITON or MSR_NOISE_PHILOX8. */
typedef struct msr_accum_item {
    uint16_t *acc;      /* bf16 accumulator [n] */
    const void *grad;   /* bf16, or fp32 with MSR_ACCUM_GRAD_F32, [n] */
    int64_t n;
    uint32_t seed;
    int32_t flags;      /* MSR_ACCUM_ZERO_INIT | MSR_ACCUM_GRAD_F32 */
} msr_accum_item;
#define MSR_ACCUM_ZERO_INIT 1
#define MSR_ACCUM_GRAD_F32 2
int msr_sr_accum_multi(const msr_accum_item *items, int32_t count, int32_t noise_mode, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * BF16-moment AdamW step (PyTorch order: decay before the update).
 * Replaces _adamw_kernel / _adamw_step (muon_sr/triton_adamw.py:9-114).
 * Streams: ema uses SEED, ema_sq SEED+1, p SEED+2 (inject: uint16 [3][n]).
 * ------------------------------------------------------------------------- */
int msr_adamw_bf16_step(uint16_t *p, const uint16_t *g, uint16_t *ema, uint16_t *ema_sq, int64_t n,
                        float lr, float beta1, float beta2, float eps, float weight_decay,
                        float bias_correction, float bias_correction_sqrt, uint32_t seed,
                        int32_t noise_mode, const uint16_t *inject, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * Gradient centralization of TritonAdamW, on the device.
 * Replaces the host-issued torch ops of muon_sr/triton_adamw.py:179-187
 * (g.to(fp32); g -= g.mean(dims 1..) * c; g.to(bf16)).  g, out: bf16
 * [rows][cols] (rows = dim 0 of a tensor of 2+ dims, else 1); out[r][j] =
 * bf16_rne(g[r][j] - (sum_j g[r][j] / cols) * alpha) with fp32 sums in a fixed
 * order.  workspace: msr_centralize_workspace_bytes(rows, cols) bytes of
 * device memory (the library does not allocate).  out may equal g.
 * ------------------------------------------------------------------------- */
int msr_centralize_workspace_bytes(int64_t rows, int64_t cols, size_t *bytes);
int msr_centralize_bf16(const uint16_t *g, uint16_t *out, int64_t rows, int64_t cols, float alpha,
                        void *workspace, size_t workspace_bytes, msr_stream_t stream);

/* msr_centralize_bf16 without a workspace argument and without allocating.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a static device array of
 * MSR_CENTRALIZE_NOALLOC_SCRATCH_BYTES in the library, one per GPU, held until
 * the process ends; its address is looked up on the first call for a device
 * (the device of `stream`, or the current device for the null stream).  Sizes
 * whose msr_centralize_workspace_bytes exceed it return MSR_ERR_WORKSPACE
 * (4 MiB covers about 500,000 rows of up to 16384 columns, e.g. a 128256 x 4096
 * embedding).  Same results as msr_centralize_bf16, bit for bit.  Calls that
 * overlap in time on one GPU share the array and race: serialise them (one
 * stream, or events). */
#define MSR_CENTRALIZE_NOALLOC_SCRATCH_BYTES (4 << 20)
int msr_centralize_bf16_noalloc(const uint16_t *g, uint16_t *out, int64_t rows, int64_t cols, float alpha,
                                msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * (a) 8-bit blockwise AdamW step (bitsandbytes order: decay after the update).
 * Replaces the _adamw_8bit_kernel launch of TritonAdamW8bit.step
 * (muon_sr/triton_adamw_8bit.py:56-99, launched at :198-204).
 * quantized != 0: state1/state2 are uint8 codes [n], absmax1/absmax2 fp32
 *   [ceil(n/block)], qmap1 (signed) / qmap2 (unsigned) fp32 [256].
 *   qtable: NULL, or a device copy of msr_quant_table_build(qmap1, qmap2)
 *   (16-byte aligned) -- the same codes from a bucketed threshold table.
 *   With block 256, a qtable and 16-byte aligned p/g (8-byte aligned codes),
 *   whole pairs of blocks run through a fast kernel (correctly rounded sqrt and
 *   quotients from fp32 sequences valid on checked ranges, exact fallback
 *   per wave outside them) and the rest through the general kernel; both give
 *   the reference's bits.
 * quantized == 0: state1/state2 are bf16 moments [n]; absmax/qmap unused.
 * block: power of two in [32, 4096].  bc1 = 1-b1^step, bc2 = 1-b2^step.
 * Streams: p uses SEED, bf16 m SEED+1, bf16 v SEED+2 (inject: uint16 [3][n]).
 * ------------------------------------------------------------------------- */
int msr_adamw8bit_step(uint16_t *p, const uint16_t *g, void *state1, void *state2,
                       float *absmax1, float *absmax2, const float *qmap1, const float *qmap2,
                       const void *qtable, int64_t n, int32_t block, int32_t quantized,
                       float lr, float beta1, float beta2, float eps, float weight_decay,
                       float bc1, float bc2, uint32_t seed,
                       int32_t noise_mode, const uint16_t *inject, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * (b) Muon momentum prologue over one shape group.
 * Replaces the grad->stack copy and the _muon_prepare_kernel launch of
 * _triton_muon_batch_step (muon_sr/triton_muon_sr.py:150-159) and, with
 * count == 1, _run_prepare (:88-98).
 *   grads: HOST array of `count` device pointers, each to numel_each bf16
 *          (grad_is_f32 == 0) or fp32 (grad_is_f32 != 0: read as fp32, as the
 *          reference's kernel reads an fp32 gradient on the per-parameter path,
 *          :34; its batched path copies gradients into a bf16 stack first).
 *   buf:   bf16 momentum stack [count][numel_each], updated in place (SR).
 *   out:   bf16 pre-NS update [count][numel_each] (RNE).
 * Noise offset of element j of matrix i: i*numel_each + j (stack offset).
 * inject: uint16 [count*numel_each].
 * ------------------------------------------------------------------------- */
int msr_muon_prepare(const void *const *grads, int32_t grad_is_f32, uint16_t *buf, uint16_t *out,
                     int64_t numel_each, int32_t count, float beta, int32_t nesterov,
                     uint32_t seed, int32_t noise_mode, const uint16_t *inject, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * (b) Muon parameter update over several matrices of one shape.
 * Replaces the per-parameter _muon_apply_kernel launches of
 * _triton_muon_batch_step and _run_apply (muon_sr/triton_muon_sr.py:53-80,
 * 105-113, 167-169).
 *   params: HOST array of `count` device pointers, each to numel_each bf16.
 *   upd:    bf16 Newton-Schulz output [count][numel_each] (parameter layout).
 *   seeds:  HOST array of `count` seeds (salt-1 deterministic seeds).
 *   p <- SR(p*(1-lr*wd) - lr*(f32(upd)*scale)), noise offset j within p.
 * inject: uint16 [count][numel_each].
 * ------------------------------------------------------------------------- */
int msr_muon_apply(uint16_t *const *params, const uint16_t *upd, int64_t numel_each, int32_t count,
                   float lr, float weight_decay, float scale, const uint32_t *seeds,
                   int32_t noise_mode, const uint16_t *inject, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * (b) Batched Newton-Schulz orthogonalisation on bf16 MFMA.
 * Replaces _newton_schulz(G, steps, out_dtype=None) (muon_sr/muon_sr.py:82-98)
 * for a contiguous bf16 stack G [batch][rows][cols]; out has the same shape.
 * The iteration runs on the wide orientation (transposed when rows > cols):
 *   X = G/(||G||_F + 1e-7);  repeat: A = X X^T; B = b A + c A A; X = a X + B X,
 * evaluated as B' = c A A + b A + a I, X = B' X: products accumulate in fp32,
 * A, B' and X are stored in bf16 between GEMMs.  The normalised input is not
 * rounded (G itself, or G scaled by a power of two when ||G||_F is below 2^-17
 * or at least 2^16, is the first iterate, and 1/(||G||_F + 1e-7) goes into the
 * first products' scale factors), and the bf16 rounding residuals of the
 * diagonals of A and B' are carried in fp32 into the next product.  Within
 * 1e-2 relative Frobenius of the exact iteration on Gaussian inputs.
 * steps == 0 returns the reference's bf16 normalisation bf16(G / bf16(bf16(
 * ||G||_F) + 1e-7)).
 * Results do not depend on `batch` (each matrix is computed independently).
 * The workspace holds the iterates and the products' tile counters: calls that
 * may run at the same time (other streams) need workspaces of their own.
 * ------------------------------------------------------------------------- */
int msr_ns_workspace_bytes(int64_t batch, int64_t rows, int64_t cols, size_t *bytes);
int msr_newton_schulz(const uint16_t *in, uint16_t *out, int64_t batch, int64_t rows, int64_t cols,
                      int32_t steps, float a, float b, float c, void *workspace, size_t workspace_bytes,
                      msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * (b) Newton-Schulz and the Muon parameter update in one pass.
 * Replaces the _newton_schulz call and the _run_apply launches of one chunk of
 * _triton_muon_batch_step (muon_sr/triton_muon_sr.py:160-169), and of
 * _triton_muon_step (:116-120) with batch == 1.  Equal, bit for bit, to
 * msr_newton_schulz(upd -> X) followed by msr_muon_apply(params, X, ...), but
 * the last product's store applies the update to the parameters directly: X is
 * never written and the apply pass does not run.
 *   upd:    bf16 pre-NS update stack [batch][rows][cols] (read only)
 *   params: HOST array of `batch` device pointers, each to rows*cols bf16
 *   seeds:  HOST array of `batch` seeds (salt-1 deterministic seeds)
 *   p <- SR(p*(1-lr*wd) - lr*(f32(bf16(X))*scale)), noise offset = element index in p.
 * steps >= 1; workspace as msr_ns_workspace_bytes(batch, rows, cols).
 * inject: uint16 [batch][rows*cols].
 * ------------------------------------------------------------------------- */
int msr_muon_ns_apply(const uint16_t *upd, uint16_t *const *params, const uint32_t *seeds, int64_t batch,
                      int64_t rows, int64_t cols, int32_t steps, float a, float b, float c, float lr,
                      float weight_decay, float scale, int32_t noise_mode, const uint16_t *inject,
                      void *workspace, size_t workspace_bytes, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * (b) The whole Muon step of one chunk: momentum prologue, Newton-Schulz and
 * the parameter update.  Replaces, for one NS chunk of a shape group, the
 * grad->stack copy and _muon_prepare_kernel (muon_sr/triton_muon_sr.py:18-50,
 * 150-159), _newton_schulz (muon_sr/muon_sr.py:82-98) and the _run_apply
 * launches (triton_muon_sr.py:53-80, 160-169); with batch == 1, first == 0,
 * _triton_muon_step (:88-120).  Equal, bit for bit, to msr_muon_prepare over the
 * chunk's rows of the stack, then msr_newton_schulz, then msr_muon_apply (or,
 * with out, without the apply), but the update is made inside the
 * Newton-Schulz prologue, which writes it straight into the first iterate
 * (with its sum of squares): the update stack is never written or read.
 *   grads:  HOST array of `batch` device pointers (bf16, or fp32 with grads_f32)
 *   buf:    bf16 momentum of the chunk's first matrix, [batch][rows][cols],
 *           updated in place (SR); `first` = that matrix's index in its stack:
 *           noise offset of element j of matrix i = (first + i)*rows*cols + j
 *   params/apply_seeds: HOST arrays of `batch` (as msr_muon_ns_apply), or
 *   params == NULL and out: bf16 [batch][rows][cols] receives the NS output.
 * steps >= 1; workspace as msr_ns_workspace_bytes(batch, rows, cols).
 * inject_prepare: uint16 indexed by the stack offset above; inject_apply as
 * msr_muon_ns_apply's.
 * ------------------------------------------------------------------------- */
int msr_muon_fused_step(const void *const *grads, int32_t grads_f32, uint16_t *buf, int64_t first, int64_t batch,
                        int64_t rows, int64_t cols, float beta, int32_t nesterov, uint32_t prepare_seed,
                        int32_t steps, float a, float b, float c, uint16_t *out, uint16_t *const *params,
                        const uint32_t *apply_seeds, float lr, float weight_decay, float scale,
                        int32_t noise_mode, const uint16_t *inject_prepare, const uint16_t *inject_apply,
                        void *workspace, size_t workspace_bytes, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * (b) The whole Muon step of several shape groups in one call: one
 * msr_muon_fused_step per group, with the groups' matrices sharing each
 * Newton-Schulz product launch.  Replaces, for shape groups whose shapes are
 * transposes of each other (a model's tall and wide projections), the
 * per-group loop of muon_sr/triton_muon_sr.py:128-177 (group order does not
 * matter: groups touch disjoint memory).  Equal, bit for bit, to
 * msr_muon_fused_step called once per group with the same arguments (params,
 * apply_seeds and a group's prepare_seed as there); a shared launch only fills
 * the GPU's last round of tiles better than separate ones.
 *   groups: HOST array of n_groups; every group's shape is rows x cols or
 *           cols x rows of group 0's; pointers as in msr_muon_fused_step
 *           (grads, params, apply_seeds: HOST arrays of `batch` entries).
 * noise_mode: MSR_NOISE_TRITON or MSR_NOISE_PHILOX8.  steps >= 1; workspace as
 * msr_ns_workspace_bytes(sum of the groups' batch, rows, cols) of group 0.
 * ------------------------------------------------------------------------- */
typedef struct msr_muon_group {
    const void *const *grads;      /* bf16, or fp32 with grads_f32 */
    uint16_t *buf;                 /* momentum of the group's first matrix, [batch][rows][cols] */
    uint16_t *const *params;
    const uint32_t *apply_seeds;
    int64_t first;                 /* index of buf's first matrix in its stack (noise offsets) */
    int64_t batch, rows, cols;
    uint32_t prepare_seed;
    int32_t grads_f32;
    float scale;                   /* the group's sqrt(max(1, rows/cols)) */
} msr_muon_group;
int msr_muon_fused_steps(const msr_muon_group *groups, int32_t n_groups, float beta, int32_t nesterov,
                         int32_t steps, float a, float b, float c, float lr, float weight_decay,
                         int32_t noise_mode, void *workspace, size_t workspace_bytes, msr_stream_t stream);

/* ---------------------------------------------------------------------------
 * Diagnostics (no counterpart in the reference; used by the parity tests).
 * ------------------------------------------------------------------------- */

/* out[i] = 16-bit noise of stream (seed, k) at offset offset0 + i. */
int msr_noise_fill(uint16_t *out, int64_t n, int64_t offset0, uint32_t seed, uint32_t k,
                   int32_t noise_mode, msr_stream_t stream);

/* Streaming probe of the fused 8-bit step's memory accesses: the pair walk, loads and
 * stores of the fast kernel over n elements (n a multiple of 512; p, g 16-byte and the
 * codes 8-byte aligned; absmax1/2 hold n/256 floats), with the arithmetic replaced by one
 * integer operation per word (every buffer is overwritten).  `grid` work-groups of 256
 * threads, each holding `lds_bytes` (<= 64 KiB) of LDS that sets the work-groups per CU.
 * Measurement aid: no counterpart in the reference. */
int msr_stream_probe8(uint16_t *p, const uint16_t *g, uint8_t *state1, uint8_t *state2, float *absmax1,
                      float *absmax2, int64_t n, int32_t grid, int32_t lds_bytes, msr_stream_t stream);

/* out[i] = quantizer code of x[i] against qmap (reference search rule), or
 * through qtable when it is not NULL. */
int msr_quantize(const float *x, uint8_t *out, int64_t n, const float *qmap, int32_t is_signed,
                 const void *qtable, msr_stream_t stream);

/* Host-side construction of the quantizer table for a (signed, unsigned)
 * codebook pair (HOST pointers, 256 floats each) into a HOST buffer of
 * msr_quant_table_bytes() bytes.  Valid for codebooks on which the reference
 * search is monotone (the bitsandbytes dynamic maps are; proven exhaustively
 * by msr_quant_table_check). */
size_t msr_quant_table_bytes(void);
int msr_quant_table_build(const float *qmap_signed, const float *qmap_unsigned, void *table, size_t table_bytes);

/* Device self-check of a table against the search for every float bit
 * pattern u in [bits_lo, bits_hi] (<= bits(1.0f)): signed map at +x and -x,
 * unsigned map at x, through both the two-level lookup of the general 8-bit
 * kernel and the flat table of the fast one.  counts[i] = mismatches found by
 * work-group i. */
int msr_quant_table_check(const void *qtable, const float *qmap_signed, const float *qmap_unsigned,
                          uint32_t bits_lo, uint32_t bits_hi, uint32_t *counts, int32_t n_counts,
                          msr_stream_t stream);

/* Device self-check of the fast kernel's correctly rounded building blocks
 * against the IEEE operations, over the float bit patterns u in
 * [bits_lo, bits_hi]: kind 0 sqrt, alone and fused into the update's
 * sqrt(v) + eps (u <= bits(2^62)); kind 1 reciprocal
 * (bits(2^-60) <= u < bits(2^32)); kind 2 quotient m/d of the requantization
 * for 16 hashed m per d (bits(2^-60) <= u < bits(2)); kind 3 the hardware
 * fp32->bf16 round-to-nearest-even of the GEMM epilogues against the
 * bit-level rounding (any u); kind 4 the update's quotient n/d for 16 n per d
 * (+-0 and |n| in [2^-90, 2^60]; bits(2^-60) <= u < bits(2^32)).
 * counts[i] = mismatches found by work-group i.  Test support: no
 * counterpart in the reference. */
int msr_fastmath_check(int32_t kind, uint32_t bits_lo, uint32_t bits_hi, uint32_t *counts, int32_t n_counts,
                       msr_stream_t stream);

/* Batched bf16 GEMM  D[b] = alpha * P[b] Q[b]^T + beta * C[b] + diag * I  (fp32 accumulate, RNE
 * bf16 out; the diag term is added where m == n).
 * P: [M][K] (row stride ldp), Q: [N][K] (ldq), C/D: [M][N] (ldc/ldd); C may be NULL when beta == 0.
 * M, N multiples of 256 and K a multiple of 128 (the NS workspace is padded to these). */
int msr_gemm_nt(const uint16_t *P, int64_t ldp, int64_t strideP, const uint16_t *Q, int64_t ldq,
                int64_t strideQ, const uint16_t *C, int64_t ldc, int64_t strideC, uint16_t *D, int64_t ldd,
                int64_t strideD, int64_t M, int64_t N, int64_t K, int64_t batch, float alpha, float beta,
                float diag, msr_stream_t stream);

/* The same with a K-major Q:  D[b] = alpha * P[b] Q[b] + beta * C[b] + diag * I,  Q: [K][N] (row
 * stride ldq).  This is the kernel of Newton-Schulz's X' = B' X.  Test support: no counterpart in
 * the reference. */
int msr_gemm_nn(const uint16_t *P, int64_t ldp, int64_t strideP, const uint16_t *Q, int64_t ldq,
                int64_t strideQ, const uint16_t *C, int64_t ldc, int64_t strideC, uint16_t *D, int64_t ldd,
                int64_t strideD, int64_t M, int64_t N, int64_t K, int64_t batch, float alpha, float beta,
                float diag, msr_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MUON_SR_AMD_H */
