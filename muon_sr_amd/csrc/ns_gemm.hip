// Batched Newton-Schulz orthogonalisation on gfx950 bf16 MFMA.
//
// Every product of the iteration is one GEMM kernel,
//     D[m][n] = alpha * sum_k P[m][k] * Q[n][k] + beta * C[m][n] (+ diag if m == n)
// whose operands are read, per K range, either K-contiguous (one 16-byte LDS
// read per MFMA fragment) or K-major (two 8-byte transposing reads,
// ds_read_b64_tr_b16): "NT" has both K-contiguous, "NN" a K-major Q.  The
// iterate X (m x n, m <= n) is kept row-major:
//     A  = X X^T              NT, P = X,  Q = X   (symmetric: upper tiles only)
//     B' = c A A + b A + a I  NT, P = A,  Q = A   (A symmetric, so A A = A A^T)
//     X' = B' X               NN, P = B', Q = X   (= B X + a X)
// Workspace matrices are zero-padded to multiples of 256.  The padding of X
// and A stays zero through every product (B' carries a on its padded
// diagonal, which meets only zero rows of X), so only the final store is
// bounds-checked.
//
// Kernel shape: 512 threads (8 wave64s in a 2 x 4 grid, two per SIMD), a
// 256x256 output tile per work-group, K staged through LDS in 64-wide slabs,
// double buffered (2 x 64 KiB) and filled by buffer loads that write LDS
// directly, one slab ahead.  Each wave owns a 128x64 sub-tile = 4x2 tiles of
// the 32x32x16 bf16 MFMA (fp32 accumulators); with two waves per SIMD, one
// wave's MFMAs keep the matrix core busy while the other waits at the slab
// barrier.  K-contiguous LDS rows are 128 B; chunk c of row r is stored at
// c ^ ((r >> 1) & 7), so the 16 consecutive rows of one 16-lane quarter of a
// fragment read (256 B) cover all 64 banks once (the K-major layout is
// described at the loads).  Each K substep is one
// scheduling region in which the MFMAs are interleaved with the next
// substep's fragment reads; the next slab's loads are all issued at the start
// of the slab.  Work-groups are persistent, one per CU: each walks its share
// of the tiles, and a tile's epilogue (each wave staging its own sub-tile
// through LDS, no work-group barrier) overlaps the loads of the next tile's
// first slab, and its stores the next tile's first MFMAs.
#include <algorithm>
#include <atomic>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "vecio.hpp"
#include "../../include/muon_sr_amd.h"

namespace msr {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int GEMM_THREADS = 512;

// Muon apply fused into the store of the last Newton-Schulz product
// (msr_muon_ns_apply): matrix b of a launch updates params p[b] with seed[b].
constexpr int APPLY_MAX = 128;   // matrices per launch (kernel-argument table)
struct ApplyTab {
    uint16_t *p[APPLY_MAX];
    uint32_t seed[APPLY_MAX];
    const uint16_t *inject;      // uint16 [count][numel] of this launch (NOISE_INJECT), or null
    int64_t numel;
    float lr, decay, scale;      // decay = 1 - lr * wd
};

struct GemmArgs {
    const uint16_t *P; int64_t ldp, sP;
    const uint16_t *Q; int64_t ldq, sQ;
    const uint16_t *C; int64_t ldc, sC;
    uint16_t *D; int64_t ldd, sD;
    uint16_t *DT; int64_t lddt, sDT;
    int M, N, K;       // padded extents (multiples of 256, 256, 128)
    int Mv, Nv;        // stores are limited to m < Mv, n < Nv
    float alpha, beta;
    float diag;        // added to the elements with m == n
    int tiles_m, tiles_n;
    int symmetric;     // M == N, P == Q: only tiles ti <= tj are computed and stored
    int d_vec;         // D rows allow 16-byte stores (set by launch_gemm)
    int dt_vec;        // DT rows allow 16-byte stores (set by launch_gemm)
    int tiles;         // tiles per matrix
    int total;         // virtual work-groups (tiles) of the launch
    int per_xcd;       // tile order over a multiple of 8 matrices, whole matrices per XCD
    int gm;            // operand layouts by K range (GM_*)
    int sracc;         // 0, or 1 + the noise mode of the SR-accumulating store (D = acc)
    int zero_init;     // SR-accumulating store: acc reads as zero
    Noise ns;          // SR-accumulating store: noise of element offset m * ldd + n
    // Newton-Schulz epilogues (EPI_* below)
    const float *alpha_b;   // per-matrix alpha (replaces alpha when not null)
    float *resid;           // EPI_A, EPI_B: fp32 rounding residual of each diagonal element, [batch][sv]
    const float *rvec;      // EPI_B: residuals of A's diagonal; EPI_X: residuals of B''s diagonal, [batch][sv]
    int64_t sv;             // batch stride of resid and rvec
    int apply1;             // 0, or 1 + the noise mode of the fused apply store (then D / DT only mark the layout)
    ApplyTab ap;            // apply1 > 0: the parameters the D / DT store updates instead of writing
    int *tile_ctr;          // dynamic tile order (see the kernel), or null: [0, 8) per XCD, [8] work-groups done
};

// p[off + j] <- SR(p*(1 - lr*wd) - lr*(f32(u_j)*scale)) for the j < valid bf16 values u
// (packed in u[4]) of one 8-element chunk: the arithmetic and noise of
// muon_apply_kernel (muon_sr/triton_muon_sr.py:53-80); off is the element index in p.
// vec: the chunk is 16-byte aligned and off a multiple of 8.
// The parameter chunk of apply_chunk (loaded ahead so that the loads of a thread's
// chunks overlap).
__device__ __forceinline__ u32x4_t apply_load(const uint16_t *P, int64_t off, int valid, bool vec) {
    if (vec && valid == 8) return ld_nt4(P + off);
    uint32_t wp[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (j < valid) wp[j >> 1] |= (uint32_t)P[off + j] << (16 * (j & 1));
    return u32x4_t{wp[0], wp[1], wp[2], wp[3]};
}

template <int MODE>
__device__ __forceinline__ void apply_chunk(const ApplyTab &ap, uint16_t *P, const Noise &ns, int64_t off, int valid,
                                            bool vec, const uint32_t u[4], u32x4_t pw) {
    const uint32_t wp[4] = {pw.x, pw.y, pw.z, pw.w};
    uint32_t r[8];
    if (vec && valid == 8) {
        noise8<MODE>(ns, off, 8, r);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = j < valid ? noise1<MODE>(ns, off + j) : 0u;
    }
    uint32_t op[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float uf = (j & 1) ? bf16_hi(u[j >> 1]) : bf16_lo(u[j >> 1]);
        const float pf = (j & 1) ? bf16_hi(wp[j >> 1]) : bf16_lo(wp[j >> 1]);
        const float t1 = uf * ap.scale;                                   // :70
        float pj = pf * ap.decay;                                         // :72
        pj = pj - ap.lr * t1;                                             // :73
        op[j] = sr_bf16(pj, r[j]);                                        // :75-80
    }
    if (vec && valid == 8) {
        st_nt4(P + off, u32x4_t{pack2(op[0], op[1]), pack2(op[2], op[3]), pack2(op[4], op[5]), pack2(op[6], op[7])});
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < valid) P[off + j] = (uint16_t)op[j];
    }
}

// Work-group -> (matrix, tile).  Consecutive work-group ids are dispatched
// round-robin over the 8 XCDs (each with its own L2), so tiles that share
// operand row blocks should run on one XCD at the same time:
//  * small matrices (at most PER_XCD_TILES tiles, 192 for X' = B' X) in launches over a multiple
//    of 8 matrices (1-D grid): whole matrices per XCD.  Work-group L runs on
//    XCD L % 8 and takes slot L / 8 of that XCD's list, the tiles of matrices
//    xcd, xcd + 8, xcd + 16, ... in tile order;
//  * otherwise (2-D grid, blockIdx.y = matrix) each XCD takes a contiguous
//    range of one matrix's tile order, so the XCDs work on the same matrices
//    at once and share its operand rows through the Infinity Cache (measured
//    8 % faster on the 4096 x 14336 products than whole matrices per XCD,
//    which suits matrices whose tiles/8 would be too few to share operands).
// Tile order: non-symmetric products go GROUP_M tile-rows at a time, column
// by column inside a group; symmetric ones walk the upper triangle in bands of
// GROUP_M tile-rows, column by column, taking the band's rows ti <= tj of each
// column.  Either way a run of consecutive tiles covers a compact block of
// tile-rows and tile-columns.
constexpr int NXCD = 8;
constexpr int GROUP_M = 4;
constexpr int PER_XCD_TILES = 64;
constexpr int PERSIST_MAX = 32;   // tiles per persistent work-group, at most

__device__ __forceinline__ int xcd_remap(int w, int total) {
    const int per = total / NXCD;          // full rounds
    if (w >= per * NXCD) return w;         // tail keeps its order
    return (w % NXCD) * per + w / NXCD;
}

__device__ __forceinline__ void decode_tile(const GemmArgs &a, int t, int &ti, int &tj) {
    if (a.symmetric) {
        const int T = a.tiles_m;
        int g0 = 0, start = 0, rows = min(GROUP_M, T);
        for (;;) {
            const int cnt = rows * (rows + 1) / 2 + rows * (T - g0 - rows);
            if (t < start + cnt) break;
            start += cnt;
            g0 += rows;
            rows = min(GROUP_M, T - g0);
        }
        int r = t - start;
        const int tri = rows * (rows + 1) / 2;
        if (r < tri) {           // columns g0 .. g0+rows-1 hold 1 .. rows tiles
            int c = 0;
            while ((c + 1) * (c + 2) / 2 <= r) ++c;
            tj = g0 + c;
            ti = g0 + (r - c * (c + 1) / 2);
        } else {                 // full columns of `rows` tiles
            r -= tri;
            tj = g0 + rows + r / rows;
            ti = g0 + r % rows;
        }
    } else {
        const int per_group = GROUP_M * a.tiles_n;
        const int g = t / per_group;
        const int first = g * GROUP_M;
        const int rows = min(GROUP_M, a.tiles_m - first);
        const int r = t - g * per_group;
        ti = first + r % rows;
        tj = r / rows;
    }
}

// Virtual work-group v -> (matrix bz, tile origin m0, n0), per the order above.
__device__ __forceinline__ void locate_tile(const GemmArgs &a, int v, int64_t &bz, int &m0, int &n0) {
    int ti, tj;
    if (a.per_xcd) {
        const int slot = v / NXCD;
        bz = (int64_t)(v % NXCD) + (int64_t)NXCD * (slot / a.tiles);
        decode_tile(a, slot % a.tiles, ti, tj);
    } else {
        bz = v / a.tiles;
        decode_tile(a, xcd_remap(v % a.tiles, a.tiles), ti, tj);
    }
    m0 = ti * BM;
    n0 = tj * BN;
}

// Wait until at most N vector memory operations of this wave are outstanding
// (s_waitcnt: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt at their maxima).
// Vector memory operations complete in issue order, so every operation issued
// before the last N has completed.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef __attribute__((address_space(3))) void lds_void_t;

// LDS: four variables of 32 KiB, one per slab: P stage 0, P stage 1, Q stage
// 0, Q stage 1.  Separate variables tell the compiler that
// the fragment reads of one stage do not alias the direct-to-LDS loads into
// the other stage (it would otherwise wait for those loads before the reads).
// After the K loop the stage-1 variables hold the epilogue's staging (stage 0
// receives the next tile's first slab meanwhile): each wave owns EST_BYTES,
// 32 rows of its 64-column sub-tile with a row pitch of EPITCH elements (144 B:
// 16-byte aligned rows; the 8-byte writes of 32 consecutive rows hit each
// bank at most twice), waves 0-3 in P stage 1 and waves 4-7 in Q stage 1.
constexpr int SLAB_BYTES = 256 * BK * 2;   // 256 rows x 64 k, or 64 k x 256 columns, of bf16
__shared__ __attribute__((aligned(1024))) char lds_p0[SLAB_BYTES];
__shared__ __attribute__((aligned(1024))) char lds_p1[SLAB_BYTES];
__shared__ __attribute__((aligned(1024))) char lds_q0[SLAB_BYTES];
__shared__ __attribute__((aligned(1024))) char lds_q1[SLAB_BYTES];

__device__ __forceinline__ char *lds_p(int stage) { return stage ? lds_p1 : lds_p0; }
__device__ __forceinline__ char *lds_q(int stage) { return stage ? lds_q1 : lds_q0; }
constexpr int EPITCH = 72;
constexpr int EST_BYTES = 32 * EPITCH * 2;
static_assert(4 * EST_BYTES <= SLAB_BYTES, "epilogue staging fits the stage-1 variables");

// Operand layouts of a product, by K range.  A slab of an operand is read
// either row-major (its rows are the tile's 256 rows, K-contiguous: "R") or
// K-major (64 rows of k, each the tile's 256 columns: "K").  P is K-major for
// k < kP and Q for k < kQ, with kP <= kQ, so a K range is KK, RK or RR:
//   GM_RR      P, Q row-major everywhere            (A = X X^T, msr_gemm_nt)
//   GM_RK      Q K-major everywhere                  (msr_gemm_nn)
//   GM_TRI_P   Q K-major; P is a symmetric matrix stored as its upper
//              256-tiles only, so its row block ti is read K-major (as the
//              stored block (kb, ti)) for kb < ti         (X' = B' X)
//   GM_TRI_PQ  P and Q the same upper-stored symmetric matrix (B' = c A A + b A + a I)
//   GM_KK      P, Q K-major everywhere (the weight gradient dW = dY^T X of
//              row-major activations)
enum : int { GM_RR = 0, GM_RK = 1, GM_TRI_P = 2, GM_TRI_PQ = 3, GM_KK = 4 };

// Epilogues of the Newton-Schulz products.  The iteration keeps A, B' and X
// in bf16 between products; the diagonals of A and B' are the largest
// entries of those matrices (B' carries a = 3.4445 on it), so their bf16
// rounding is the largest rounding error of the iteration.  These epilogues
// carry the rounding residual of every diagonal element in fp32 to the next
// product:
//   EPI_A  A = alpha X X^T:  rho[m] = A_mm - bf16(A_mm)                 (resid)
//   EPI_B  B' = alpha (A A) + beta A + diag I with the diagonal corrected
//          for rho to first order, B'_mm += rho[m] (beta + 2 alpha A_mm)
//          (d/dA_mm of beta A_mm + alpha (A A)_mm with A_mm dominant):
//          r[m] = B'_mm - bf16(B'_mm)                                   (resid)
//   EPI_X  X' = alpha (B' X + bf16(r[m]) X), the second term as MFMAs of the diagonal
//          block (see mmdiag)
// EPI_NONE is the plain alpha P Q^T + beta C + diag I of the diagnostic GEMMs.
enum : int { EPI_NONE = 0, EPI_A = 1, EPI_B = 2, EPI_X = 3 };

// SRACC >= 0: D is a bf16 accumulator and the store adds to it with stochastic
// rounding (noise mode SRACC), as msr_sr_accum does with the RNE bf16 product.
// APPLY >= 0 (with OUT_D or OUT_DT): the store applies the Muon update to the
// parameters of a.ap with noise mode APPLY instead of writing D / DT.
// FULL: every tile of the launch is in range (Mv == M, Nv == N) with 16-byte
// rows of D / DT (or SRACC >= 0, whose stores are never bounded), so its
// stores are unconditional.
template <bool SYM, bool HAS_C, bool OUT_D, bool OUT_DT, int GM, int SRACC = -1, int EPI = EPI_NONE, int APPLY = -1,
          bool FULL = false>
__global__ __launch_bounds__(GEMM_THREADS) void gemm_nt_kernel(GemmArgs a) {
    using T_ = std::true_type;
    using F_ = std::false_type;
    constexpr bool HAS_KK = GM == GM_TRI_P || GM == GM_TRI_PQ || GM == GM_KK;
    constexpr bool HAS_RK = GM == GM_RK || GM == GM_TRI_P || GM == GM_TRI_PQ;
    constexpr bool HAS_RR = GM == GM_RR || GM == GM_TRI_PQ;
    // K ranges of the tile at (m0, n0): P is read K-major for k < kP, Q for k < kQ
    auto kp_of = [&](int tm0) { return GM == GM_KK ? a.K : HAS_KK ? tm0 : 0; };
    auto kq_of = [&](int tn0) { return GM == GM_RR ? 0 : GM == GM_TRI_PQ ? tn0 : a.K; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;   // 2 x 4 waves, 128 x 64 each
    const int r32 = lane & 31;
    const int khalf = lane >> 5;

    // Global -> LDS: buffer loads with the lds flag move 64 lanes x 16 B into
    // 1 KiB of consecutive LDS (lane l to byte 16 l, base in M0); load i
    // (0..3) of wave w fills LDS block 8 i + w of the operand's slab.
    //  * row-major slab (256 rows x 128 B): block 8 i + w = rows (8 i + w) 8 +
    //    l / 8, physical chunk l % 8, i.e. logical chunk (l % 8) ^ ((row >> 1)
    //    & 7) = (l % 8) ^ (4 (w & 1) + l / 16);
    //  * K-major slab (64 rows x 512 B): chunk c of row k is stored at c ^ 4
    //    (k & 3), so the four rows of one transposing read fall in different
    //    banks; block 8 i + w = rows 16 i + 2 w + l / 32, physical chunk l % 32.
    // Per-lane byte offsets are fixed per tile; the row block (i) and the K
    // slab go into the scalar offset.
    const int lrow = lane >> 3;
    const int lchunk = (lane & 7) ^ (4 * (wave & 1) + (lane >> 4));
    const int kr = 2 * wave + (lane >> 5);
    const int kc = (lane & 31) ^ (4 * (kr & 3));
    const uint32_t ldbP = (uint32_t)(a.ldp * 2), ldbQ = (uint32_t)(a.ldq * 2);
    // A tile's operands: its matrices and the lane's byte offsets in their
    // row-major (pr, qr) and K-major (pk, qk) slabs at k = 0.
    struct TileOps {
        const uint16_t *P, *Q;
        uint32_t pr, qr, pk, qk;
        bool qp;   // a diagonal tile of a symmetric product: its Q slabs are its P slabs
    };
    auto tile_ops = [&](int64_t tbz, int tm0, int tn0) {
        TileOps o;
        o.P = a.P + tbz * a.sP;
        o.Q = a.Q + tbz * a.sQ;
        o.pr = (uint32_t)(((int64_t)(tm0 + wave * 8 + lrow) * a.ldp + lchunk * 8) * 2);
        o.qr = (uint32_t)(((int64_t)(tn0 + wave * 8 + lrow) * a.ldq + lchunk * 8) * 2);
        o.pk = (uint32_t)(((int64_t)kr * a.ldp + tm0 + 8 * kc) * 2);
        o.qk = (uint32_t)(((int64_t)kr * a.ldq + tn0 + 8 * kc) * 2);
        o.qp = SYM && tm0 == tn0;
        return o;
    };
    // Load j (0..7) of the slab at k0 of tile o into `stage`: P block j/2 for
    // even j, Q block j/2 for odd j, each in the layout of the slab's K range
    // (pk, qk: wave-uniform).  QP: a diagonal tile of a symmetric product (P = Q,
    // m0 = n0, the same K ranges) loads P only and reads its Q fragments there.
    auto dma = [&](const TileOps &o, bool pk, bool qk, int stage, int k0, auto QP) {
        const __amdgpu_buffer_rsrc_t rP = __builtin_amdgcn_make_buffer_rsrc((void *)o.P, (short)0, 0x7fffffff, 0x00020000);
        const __amdgpu_buffer_rsrc_t rQ = __builtin_amdgcn_make_buffer_rsrc((void *)o.Q, (short)0, 0x7fffffff, 0x00020000);
        const uint32_t vp = pk ? o.pk : o.pr, vq = qk ? o.qk : o.qr;
        const uint32_t ip = pk ? 16 * ldbP : 64 * ldbP, iq = qk ? 16 * ldbQ : 64 * ldbQ;
        const uint32_t kp = pk ? k0 * ldbP : k0 * 2, kq = qk ? k0 * ldbQ : k0 * 2;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = j >> 1;
            const int dst = (8 * i + wave) * 1024;
            if (j & 1) {
                if constexpr (!decltype(QP)::value)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rQ, (lds_void_t *)(lds_q(stage) + dst), 16, vq, i * iq + kq, 0, 0);
            } else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rP, (lds_void_t *)(lds_p(stage) + dst), 16, vp, i * ip + kp, 0, 0);
        }
    };
    auto dma_first = [&](const TileOps &o, int tm0, int tn0) {   // a tile's first slab, into stage 0
        if (o.qp) dma(o, 0 < kp_of(tm0), 0 < kq_of(tn0), 0, 0, T_{});
        else dma(o, 0 < kp_of(tm0), 0 < kq_of(tn0), 0, 0, F_{});
    };
    // Row-major fragment reads: chunk (2 ks + khalf) ^ ((row >> 1) & 7) of row;
    // bits 1-3 of row come from r32 only, so one byte offset per (operand, ks)
    // serves all 32-row blocks through the instruction offset.
    const int sw = (r32 >> 1) & 7;
    uint32_t offP[4], offQ[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int ch = (2 * ks) ^ khalf ^ sw;
        offP[ks] = (uint32_t)((wm * 128 + r32) * 128 + ch * 16);
        offQ[ks] = (uint32_t)((wn * 64 + r32) * 128 + ch * 16);
    }
    // K-major fragment reads: the fragment of lane l (column l % 32, k = 8 (l /
    // 32) + 0..7 of the substep) is two transposing reads of 4 k each.  In a
    // read, lane i of a 16-lane group returns element i % 4 of the 8-byte rows
    // fetched by lanes i / 4 + 4 j (j = 0..3), so lane i fetches row k = i / 4
    // (+4 for the second read), columns 4 (i % 4) .. +3 of its group's 16.
    uint32_t offPK[4], offQK[2];
    {
        const int G = lane >> 4, i = lane & 15;
        const uint32_t rowb = (uint32_t)((8 * (G >> 1) + (i >> 2)) * 512 + (i & 1) * 8);
        const int c0 = 2 * (G & 1) + ((i >> 1) & 1);
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) offPK[mi] = rowb + (uint32_t)(((wm * 16 + mi * 4 + c0) ^ (4 * (i >> 2))) * 16);
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) offQK[ni] = rowb + (uint32_t)(((wn * 8 + ni * 4 + c0) ^ (4 * (i >> 2))) * 16);
    }
    auto trfrag = [](const char *p) {
        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(p));
        const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(p + 2048));
        return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    auto frags = [&](auto PK, auto QK, auto QP, int stage, int ks, bf16x8_t (&pa)[4], bf16x8_t (&qb)[2]) {
        const char *qs = decltype(QP)::value ? lds_p(stage) : lds_q(stage);   // Q from the P slabs (dma)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            if constexpr (decltype(PK)::value) pa[mi] = trfrag(lds_p(stage) + offPK[mi] + ks * 8192);
            else pa[mi] = *reinterpret_cast<const bf16x8_t *>(lds_p(stage) + offP[ks] + mi * 4096);
        }
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            if constexpr (decltype(QK)::value) qb[ni] = trfrag(qs + offQK[ni] + ks * 8192);
            else qb[ni] = *reinterpret_cast<const bf16x8_t *>(qs + offQ[ks] + ni * 4096);
        }
    };

    // Persistent work-groups: work-group g computes the tiles of virtual
    // work-groups g, g + G, g + 2 G, ... (G = gridDim.x, a multiple of 8 when
    // the grid is smaller than the launch, so each runs on the XCD that the
    // tile order assumes; launches of more than PERSIST_MAX tiles per CU get a
    // work-group per tile, which leaves the loop after its first).  The first
    // slab of a work-group's next tile streams into stage 0 while the epilogue
    // of its current tile runs.
    int v = blockIdx.x;
    int64_t bz;
    int m0, n0;
    locate_tile(a, v, bz, m0, n0);
    dma_first(tile_ops(bz, m0, n0), m0, n0);
    // EPI_X: the fp32 residuals r of the tile's rows 128 wm + 32 mi + r32, loaded
    // a tile ahead (with the tile's first slab) so that no load waits at its start
    float rf0 = 0.0f, rf1 = 0.0f, rf2 = 0.0f, rf3 = 0.0f;
    auto load_r = [&](int64_t tbz, int tm0) __attribute__((always_inline)) {
        if constexpr (EPI == EPI_X) {
            const float *rv = a.rvec + tbz * a.sv + tm0 + wm * 128 + r32;
            rf0 = rv[0];
            rf1 = rv[32];
            rf2 = rv[64];
            rf3 = rv[96];
        }
    };
    load_r(bz, m0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // Dynamic tile order (a.tile_ctr, launches of more tiles than work-groups; the
    // grid is then a multiple of 8): work-group g on XCD x = g % 8 takes slot g / 8 of
    // that XCD's tile list (the tiles of virtual work-groups x + 8 slot) first, as in
    // the static order, and each next slot from the XCD's counter, fetched while its
    // current tile runs.  The tiles in flight then stay a compact run of each XCD's
    // list however unevenly the work-groups progress.  The last work-group to finish
    // resets the counters for the next launch on the stream.
    const bool dyn = a.tile_ctr != nullptr;
    const int xcd = (int)(blockIdx.x % NXCD);
    __shared__ int s_next_slot;
    int my_slot = 0;
    for (;;) {
        if (dyn && tid == 0) my_slot = (int)(gridDim.x / NXCD) + atomicAdd(a.tile_ctr + xcd, 1);
        const TileOps ot = tile_ops(bz, m0, n0);
        const int kP = kp_of(m0), kQ = kq_of(n0);
        f32x16_t acc[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

        bf16x8_t fa[2][4], fb[2][2];
        auto mm = [&](int b) {
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[b][ni], fa[b][mi], acc[mi][ni], 0, 0, 0);
        };
        // EPI_X: the term r[m] X[m][n] of X' = B' X + r X enters the accumulators as the product
        // of X with the diagonal matrix bf16(r), over the K block k in [m0, m0 + 256) that holds
        // the tile's own rows of X (the first 4 slabs of the RK range).  Wave (wm, wn) owns rows
        // 128 wm .. 128 wm + 127 of the tile, which are slabs 2 wm and 2 wm + 1 of that block: in
        // slab 2 wm + st, substep ks, the diagonal crosses the 32-row block mi = 2 st + ks / 2,
        // and lane l's fragment (row r32, k = 8 khalf + e) holds it at e = r32 - 16 (ks & 1) -
        // 8 khalf.  That is 16 extra MFMAs per wave and no extra memory traffic.
        uint32_t rb16[4] = {0u, 0u, 0u, 0u};   // bf16(r) at rows 128 wm + 32 mi + r32
        if constexpr (EPI == EPI_X) {
            const uint32_t p01 = rne_bf16x2(rf0, rf1), p23 = rne_bf16x2(rf2, rf3);
            rb16[0] = p01 & 0xffffu;
            rb16[1] = p01 >> 16;
            rb16[2] = p23 & 0xffffu;
            rb16[3] = p23 >> 16;
        }
        auto mmdiag = [&](int b, auto ST, auto KS) {
            constexpr int ks = decltype(KS)::value;
            constexpr int mi = 2 * decltype(ST)::value + (ks >> 1);
            const int e = r32 - 16 * (ks & 1) - 8 * khalf;
            const uint32_t v = (unsigned)e < 8u ? rb16[mi] << (16 * (e & 1)) : 0u;
            const int w = e >> 1;
            const u32x4_t words = {w == 0 ? v : 0u, w == 1 ? v : 0u, w == 2 ? v : 0u, w == 3 ? v : 0u};
            const bf16x8_t rf = __builtin_bit_cast(bf16x8_t, words);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[b][ni], rf, acc[mi][ni], 0, 0, 0);
        };
        // dg: this wave's rows meet the slab pair of the diagonal block being computed
        auto diag = [&](auto DG, bool dg, int b, int stage, auto KS) {
            if constexpr (decltype(DG)::value) {
                if (dg) {
                    if (stage == 0) mmdiag(b, std::integral_constant<int, 0>{}, KS);
                    else mmdiag(b, std::integral_constant<int, 1>{}, KS);
                }
            }
        };
        // Each substep is one scheduling region: its 8 MFMAs interleaved with the
        // fragment reads of the next substep (6 row-major, 8 or 12 with K-major
        // operands: 4 reads per row-major P, 8 per K-major P, 2 or 4 for Q).
        auto pattern = [&](auto PK, auto QK) {
            constexpr int NDS = (decltype(PK)::value ? 8 : 4) + (decltype(QK)::value ? 4 : 2);
            if constexpr (NDS == 6) {
#pragma unroll
                for (int x = 0; x < 6; ++x) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    if (x == 0 || x == 2) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
            } else {
#pragma unroll
                for (int x = 0; x < 8; ++x) {
                    if (NDS == 12 && (x & 1) == 0) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
            }
        };
        // One K slab from `stage` (layouts PK, QK) while slab `knext` (layouts
        // pkn, qkn) streams into the other stage.  All 8 global->LDS loads of the
        // next slab are issued before the slab's first MFMA: the operands arrive
        // through L2 with a latency tail (misses to the Infinity Cache / HBM), and
        // the wait at the end of the slab then has the whole slab to cover it
        // (measured +3..19% over spreading the loads across the substeps).  The
        // last substep's MFMAs overlap the next slab's first fragment reads, in
        // this slab's layouts; after the last slab of a K range these are unused.
        using K0_ = std::integral_constant<int, 0>;
        using K1_ = std::integral_constant<int, 1>;
        using K2_ = std::integral_constant<int, 2>;
        using K3_ = std::integral_constant<int, 3>;
        auto slab = [&](auto PK, auto QK, auto QP, int stage, int knext, bool pkn, bool qkn, auto DG, bool dg, bool load) {
            if (load) dma(ot, pkn, qkn, stage ^ 1, knext, QP);   // wave-uniform: no load after the last slab of K
            __builtin_amdgcn_sched_barrier(0);
            frags(PK, QK, QP, stage, 1, fa[1], fb[1]);
            mm(0);
            diag(DG, dg, 0, stage, K0_{});
            pattern(PK, QK);
            __builtin_amdgcn_sched_barrier(0);
            frags(PK, QK, QP, stage, 2, fa[0], fb[0]);
            mm(1);
            diag(DG, dg, 1, stage, K1_{});
            pattern(PK, QK);
            __builtin_amdgcn_sched_barrier(0);
            frags(PK, QK, QP, stage, 3, fa[1], fb[1]);
            mm(0);
            diag(DG, dg, 0, stage, K2_{});
            pattern(PK, QK);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0);   // own loads of the next slab landed, own reads of this stage done
            __syncthreads();                 // everyone's
            frags(PK, QK, QP, stage ^ 1, 0, fa[0], fb[0]);
            mm(1);
            diag(DG, dg, 1, stage, K3_{});
            pattern(PK, QK);
            __builtin_amdgcn_sched_barrier(0);
        };
        // The K ranges [0, kP) (KK), [kP, kQ) (RK) and [kQ, K) (RR) run as
        // separate loops with uniform bodies, one after the other.  Each range
        // starts in stage 0 with its first slab landed (ranges are multiples of 4
        // slabs) and reads its own first fragments, so no fragment registers live
        // across ranges and the accumulators keep their registers.  The last slab
        // of a range loads the first slab of the next one (selected, not
        // branched); the last slab of K loads nothing (its first-fragment reads
        // of the other stage, in the loop's layouts, are then unused).
        const int KT = a.K / BK, ktP = kP / BK, ktQ = kQ / BK;
        // DG: the range is the diagonal block [m0, m0 + 256) of X' = B' X + r X (EPI_X), whose
        // slab pair (kt - kt0) / 2 holds the rows of waves with wm = (kt - kt0) / 2.
        auto range = [&](auto PK, auto QK, auto QP, int kt0, int kt1, auto DG) {
            const bool end = kt1 >= KT;
            const int kafter = end ? (kt1 - 1) * BK : kt1 * BK;
            const bool pka = end ? decltype(PK)::value : kt1 < ktP, qka = end ? decltype(QK)::value : kt1 < ktQ;
            frags(PK, QK, QP, 0, 0, fa[0], fb[0]);
#pragma clang loop unroll(disable)
            for (int kt = kt0; kt < kt1; kt += 2) {
                const bool more = kt + 2 < kt1;
                const bool dg = decltype(DG)::value && ((kt - kt0) >> 1) == wm;
                slab(PK, QK, QP, 0, (kt + 1) * BK, PK, QK, DG, dg, true);
                slab(PK, QK, QP, 1, more ? (kt + 2) * BK : kafter, more ? decltype(PK)::value : pka,
                     more ? decltype(QK)::value : qka, DG, dg, more || !end);
            }
        };
        auto kloop = [&](auto QP) {
            if constexpr (HAS_KK) {
                if (0 < ktP) range(T_{}, T_{}, QP, 0, ktP, F_{});
            }
            if constexpr (EPI == EPI_X) {   // GM_TRI_P: the RK range starts at k = m0 (ktP + 4 <= ktQ)
                range(F_{}, T_{}, QP, ktP, ktP + 4, T_{});
                if (ktP + 4 < ktQ) range(F_{}, T_{}, QP, ktP + 4, ktQ, F_{});
            } else if constexpr (HAS_RK) {
                if (ktP < ktQ) range(F_{}, T_{}, QP, ktP, ktQ, F_{});
            }
            if constexpr (HAS_RR) {
                if (ktQ < KT) range(F_{}, F_{}, QP, ktQ, KT, F_{});
            }
        };
        if constexpr (SYM) {   // diagonal tiles read Q from the P slabs (one K loop each)
            if (ot.qp) kloop(T_{});
            else kloop(F_{});
        } else {
            kloop(F_{});
        }

        // ---------------- epilogue ----------------
        // Each wave stages its own 128 x 64 sub-tile through its private LDS
        // region, one 32-row block mi at a time.  LDS accesses of one wave
        // execute in order, so the epilogue needs no work-group barrier.  Global
        // traffic is 16-byte chunks of whole 128-byte row segments: C is loaded
        // that way, D is stored that way, and the transposed copy (DT) is
        // gathered column-wise.  A symmetric product stores its upper tiles only.
        // Lane l holds D[m = l % 32][n = 8r + 4(l / 32) + q] of each 32x32 MFMA tile.
        __builtin_amdgcn_s_waitcnt(0);
        if (dyn && tid == 0) s_next_slot = my_slot;
        __syncthreads();   // every wave is done with the operand slabs
        const int vn = dyn ? xcd + NXCD * __builtin_amdgcn_readfirstlane(s_next_slot) : v + (int)gridDim.x;
        const bool next = vn < a.total;
        // The epilogue's lane indices, from an opaque copy of the thread index:
        // its addresses are then formed here instead of being hoisted out of
        // the tile loop, where they would stay live through the K loop.
        int e_tid = tid;
        asm volatile("" : "+v"(e_tid));
        const int e_lane = e_tid & 63;
        const int e_r32 = e_lane & 31, e_khalf = e_lane >> 5;
        const int crow = e_lane >> 3, cchk = e_lane & 7;     // chunk accesses: rows crow + 8 i, 16-byte chunk cchk
        const int wm0 = m0 + 128 * wm, wn0 = n0 + 64 * wn;   // the wave's sub-tile
        char *const wst = (wave < 4 ? lds_p1 : lds_q1) + (wave & 3) * EST_BYTES;
        auto est = [&](int row) __attribute__((always_inline)) { return reinterpret_cast<uint16_t *>(wst + row * (EPITCH * 2)); };
        // (alpha * acc (+ beta * C)) (+ diag where m == n), rounded to bf16 by the
        // hardware conversion; the multiply is skipped for alpha == 1 (x * 1 == x
        // for every non-NaN x) and the diagonal term outside diagonal tiles.
        // The Newton-Schulz epilogues (EPI_*) are described at their enum.
        const float alpha = a.alpha_b ? a.alpha_b[bz] : a.alpha;
        float rho0 = 0.0f, rho1 = 0.0f, rho2 = 0.0f, rho3 = 0.0f;   // EPI_B: rho at rows wm0 + 32 mi + e_r32
        if constexpr (EPI == EPI_B) {
            const float *rv = a.rvec + bz * a.sv + wm0 + e_r32;
            rho0 = rv[0];
            rho1 = rv[32];
            rho2 = rv[64];
            rho3 = rv[96];
        }
        // The next tile's first slab into stage 0
        int64_t nbz = bz;
        int nm0 = m0, nn0 = n0;
        if (next) {
            locate_tile(a, vn, nbz, nm0, nn0);
            dma_first(tile_ops(nbz, nm0, nn0), nm0, nn0);
            load_r(nbz, nm0);
        }
        // Diagonal tiles: the lane's diagonal element of each 32-row block mi (at most
        // one) and its fp32 rounding residual (selects in the unrolled loop, a store
        // after the block).
        const bool dtile = m0 == n0 && (a.diag != 0.0f || EPI == EPI_A || EPI == EPI_B);
        auto block = [&](auto MI, auto SC, auto DG, auto FL) __attribute__((always_inline)) {
            constexpr int mi = decltype(MI)::value;
            constexpr bool fl = decltype(FL)::value;
            if constexpr (HAS_C) {   // this block of C into the staging
                const uint16_t *Cb = a.C + bz * a.sC + (int64_t)(wm0 + 32 * mi + crow) * a.ldc + wn0 + 8 * cchk;
                const int64_t l8 = 8 * a.ldc;
                const uint4 c0 = *reinterpret_cast<const uint4 *>(Cb);
                const uint4 c1 = *reinterpret_cast<const uint4 *>(Cb + l8);
                const uint4 c2 = *reinterpret_cast<const uint4 *>(Cb + 2 * l8);
                const uint4 c3 = *reinterpret_cast<const uint4 *>(Cb + 3 * l8);
                *reinterpret_cast<uint4 *>(est(crow) + 8 * cchk) = c0;
                *reinterpret_cast<uint4 *>(est(crow + 8) + 8 * cchk) = c1;
                *reinterpret_cast<uint4 *>(est(crow + 16) + 8 * cchk) = c2;
                *reinterpret_cast<uint4 *>(est(crow + 24) + 8 * cchk) = c3;
            }
            const float rho = mi == 0 ? rho0 : mi == 1 ? rho1 : mi == 2 ? rho2 : rho3;
            float res_mi = 0.0f;
            bool has_mi = false;
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ml = wm * 128 + mi * 32 + e_r32;                  // tile row
                    const int nl = wn * 64 + ni * 32 + 8 * r + 4 * e_khalf;     // tile column
                    uint2 *sp = reinterpret_cast<uint2 *>(est(e_r32) + ni * 32 + 8 * r + 4 * e_khalf);
                    float v[4] = {acc[mi][ni][4 * r], acc[mi][ni][4 * r + 1], acc[mi][ni][4 * r + 2],
                                  acc[mi][ni][4 * r + 3]};
                    float cv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (decltype(SC)::value) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[q] = alpha * v[q];
                    }
                    if constexpr (HAS_C) {
                        const uint2 cw = *sp;
                        cv[0] = bf16_lo(cw.x);
                        cv[1] = bf16_hi(cw.x);
                        cv[2] = bf16_lo(cw.y);
                        cv[3] = bf16_hi(cw.y);
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[q] = v[q] + a.beta * cv[q];
                    }
                    if constexpr (decltype(DG)::value) {   // m0 == n0 here
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const bool on = ml == nl + q;
                            if constexpr (EPI == EPI_B)
                                v[q] = on ? v[q] + (a.diag + rho * (a.beta + 2.0f * alpha * cv[q])) : v[q];
                            else if constexpr (EPI != EPI_A)
                                v[q] = on ? v[q] + a.diag : v[q];
                        }
                    }
                    const uint2 w = make_uint2(rne_bf16x2(v[0], v[1]), rne_bf16x2(v[2], v[3]));
                    *sp = w;
                    if constexpr (decltype(DG)::value && (EPI == EPI_A || EPI == EPI_B)) {
                        const float rq[4] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const bool on = ml == nl + q;
                            res_mi = on ? v[q] - rq[q] : res_mi;
                            has_mi = has_mi || on;
                        }
                    }
                }
            }
            if constexpr (decltype(DG)::value && (EPI == EPI_A || EPI == EPI_B)) {
                if (has_mi) a.resid[bz * a.sv + wm0 + 32 * mi + e_r32] = res_mi;
            }
            // block mi of the output: rows wm0 + 32 mi + crow + 8 i, columns wn0 + 8 cchk
            const int bm0 = wm0 + 32 * mi;
            if constexpr (SRACC >= 0) {
                // acc <- SR(f32(acc) + f32(tile)), 8 elements (one noise8 group) per access
                uint16_t *Db = a.D + bz * a.sD;
                uint4 c[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t o0 = (int64_t)(bm0 + crow + 8 * i) * a.ldd + wn0 + 8 * cchk;
                    c[i] = a.zero_init ? make_uint4(0u, 0u, 0u, 0u) : *reinterpret_cast<const uint4 *>(Db + o0);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t o0 = (int64_t)(bm0 + crow + 8 * i) * a.ldd + wn0 + 8 * cchk;
                    const uint4 w = *reinterpret_cast<const uint4 *>(est(crow + 8 * i) + 8 * cchk);
                    const uint32_t gw[4] = {w.x, w.y, w.z, w.w}, cw[4] = {c[i].x, c[i].y, c[i].z, c[i].w};
                    uint32_t rn[8], o[4];
                    noise8<SRACC>(a.ns, o0, 8, rn);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        o[j] = pack2(sr_bf16(bf16_lo(cw[j]) + bf16_lo(gw[j]), rn[2 * j]),
                                     sr_bf16(bf16_hi(cw[j]) + bf16_hi(gw[j]), rn[2 * j + 1]));
                    *reinterpret_cast<uint4 *>(Db + o0) = make_uint4(o[0], o[1], o[2], o[3]);
                }
            } else if constexpr (OUT_D && APPLY >= 0) {
                uint16_t *Pp = a.ap.p[bz];
                Noise ns;
                ns.key = seed_key(a.ap.seed[bz], 0);
                ns.inject = a.ap.inject ? a.ap.inject + bz * a.ap.numel : nullptr;
                const int n = wn0 + 8 * cchk;
                const bool vec = fl || a.d_vec != 0;
                u32x4_t pw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = bm0 + crow + 8 * i;
                    const bool in = fl || (m < a.Mv && n < a.Nv);
                    pw[i] = in ? apply_load(Pp, (int64_t)m * a.ldd + n, fl ? 8 : min(8, a.Nv - n), vec)
                               : u32x4_t{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = bm0 + crow + 8 * i;
                    if (!fl && (m >= a.Mv || n >= a.Nv)) continue;
                    const uint4 w = *reinterpret_cast<const uint4 *>(est(crow + 8 * i) + 8 * cchk);
                    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
                    apply_chunk<APPLY>(a.ap, Pp, ns, (int64_t)m * a.ldd + n, fl ? 8 : min(8, a.Nv - n), vec, u, pw[i]);
                }
            } else if constexpr (OUT_D) {
                uint16_t *Db = a.D + bz * a.sD;
                const int n = wn0 + 8 * cchk;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = bm0 + crow + 8 * i;
                    const uint4 w = *reinterpret_cast<const uint4 *>(est(crow + 8 * i) + 8 * cchk);
                    uint16_t *dp = Db + (int64_t)m * a.ldd + n;
                    if (fl) {
                        st_nt4(dp, u32x4_t{w.x, w.y, w.z, w.w});   // streaming store: measured 0.4-1.6 % faster NS
                    } else if (m < a.Mv) {
                        if (a.d_vec && n + 8 <= a.Nv) {
                            st_nt4(dp, u32x4_t{w.x, w.y, w.z, w.w});
                        } else {
                            const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                            for (int j = 0; j < 8; ++j)
                                if (n + j < a.Nv) dp[j] = (uint16_t)(u[j >> 1] >> (16 * (j & 1)));
                        }
                    }
                }
            }
            // Transposed copy: T[n][m] = tile[m][n].  The block's 32 rows are 32
            // consecutive m of every output row n: lane l takes output rows
            // n = wn0 + l / 4 + 16 i (i = 0..3) and, in each, the 8 consecutive m
            // (16 bytes) from bm0 + 8 (l % 4), so four lanes write 64 contiguous
            // bytes of one output row (LDS: one 2-byte read per element, at most
            // two lanes per bank).
            const int tq = e_lane & 3, tn = e_lane >> 2;
            if constexpr (OUT_DT && APPLY >= 0) {
                uint16_t *Pp = a.ap.p[bz];
                Noise ns;
                ns.key = seed_key(a.ap.seed[bz], 0);
                ns.inject = a.ap.inject ? a.ap.inject + bz * a.ap.numel : nullptr;
                const int m = bm0 + 8 * tq;
                const bool vec = fl || a.dt_vec != 0;
                u32x4_t pw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int n = wn0 + tn + 16 * i;
                    const bool in = fl || (n < a.Nv && m < a.Mv);
                    pw[i] = in ? apply_load(Pp, (int64_t)n * a.lddt + m, fl ? 8 : min(8, a.Mv - m), vec)
                               : u32x4_t{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int nl = tn + 16 * i;
                    uint32_t u[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        u[j] = (uint32_t)est(8 * tq + 2 * j)[nl] | ((uint32_t)est(8 * tq + 2 * j + 1)[nl] << 16);
                    const int n = wn0 + nl;
                    if (!fl && (n >= a.Nv || m >= a.Mv)) continue;
                    apply_chunk<APPLY>(a.ap, Pp, ns, (int64_t)n * a.lddt + m, fl ? 8 : min(8, a.Mv - m), vec, u, pw[i]);
                }
            } else if constexpr (OUT_DT) {
                uint16_t *Tb = a.DT + bz * a.sDT;
                const int m = bm0 + 8 * tq;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int nl = tn + 16 * i;           // tile column = output row
                    uint32_t u[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        u[j] = (uint32_t)est(8 * tq + 2 * j)[nl] | ((uint32_t)est(8 * tq + 2 * j + 1)[nl] << 16);
                    const int n = wn0 + nl;
                    uint16_t *tp = Tb + (int64_t)n * a.lddt + m;
                    if (fl) {
                        *reinterpret_cast<uint4 *>(tp) = make_uint4(u[0], u[1], u[2], u[3]);
                    } else if (n < a.Nv) {
                        if (a.dt_vec && m + 8 <= a.Mv) {
                            *reinterpret_cast<uint4 *>(tp) = make_uint4(u[0], u[1], u[2], u[3]);
                        } else {
#pragma unroll
                            for (int j = 0; j < 8; ++j)
                                if (m + j < a.Mv) tp[j] = (uint16_t)(u[j >> 1] >> (16 * (j & 1)));
                        }
                    }
                }
            }
        };
        using I0_ = std::integral_constant<int, 0>;
        using I1_ = std::integral_constant<int, 1>;
        using I2_ = std::integral_constant<int, 2>;
        using I3_ = std::integral_constant<int, 3>;
        auto blocks = [&](auto SC, auto DG, auto FL) __attribute__((always_inline)) {
            block(I0_{}, SC, DG, FL);
            block(I1_{}, SC, DG, FL);
            block(I2_{}, SC, DG, FL);
            block(I3_{}, SC, DG, FL);
        };
        auto epilogue = [&](auto FL) __attribute__((always_inline)) {
            if (dtile) {
                if (alpha == 1.0f) blocks(F_{}, T_{}, FL);
                else blocks(T_{}, T_{}, FL);
            } else {
                if (alpha == 1.0f) blocks(F_{}, F_{}, FL);
                else blocks(T_{}, F_{}, FL);
            }
        };
        // The next tile's first slab was loaded before this tile's stores.  With
        // FL the epilogue issues 16 unconditional store instructions per lane
        // after those loads (with APPLY also 16 parameter loads, each block's before
        // its stores), and vector memory operations complete in order, so waiting
        // for all but the last 16 leaves stores in flight and the slab landed;
        // otherwise wait for everything.
        epilogue(std::integral_constant<bool, FULL>{});
        if constexpr (FULL) wait_vm<16>();
        else __builtin_amdgcn_s_waitcnt(0);
        if (!next) break;
        // Everyone's slab landed and every wave is done with its staging.  A
        // plain barrier: a fence here would also wait for this wave's stores.
        asm volatile("s_barrier" ::: "memory");
        v = vn;
        bz = nbz;
        m0 = nm0;
        n0 = nn0;
    }
    // every work-group has fetched its last slot when it gets here
    if (dyn && tid == 0 && atomicAdd(a.tile_ctr + NXCD, 1) == (int)gridDim.x - 1) {
#pragma unroll
        for (int i = 0; i <= NXCD; ++i) a.tile_ctr[i] = 0;
    }
}

// ---------------------------------------------------------------------------
// NS prologue: deterministic Frobenius norm and normalise + transpose
// ---------------------------------------------------------------------------

constexpr int NPART = 128;        // partial sums per matrix (fixed: deterministic order)
constexpr int NORM_THREADS = 256;

// partial[b][part] = sum of squares over a fixed interleaved slice of matrix b.
// VEC: 16-byte loads (numel % 8 == 0 and `in` 16-byte aligned), two loads in flight.
template <bool VEC>
__global__ __launch_bounds__(NORM_THREADS) void sumsq_kernel(const uint16_t *in, int64_t numel, float *partial) {
    const int64_t b = blockIdx.y;
    const uint16_t *x = in + b * numel;
    float s0 = 0.0f, s1 = 0.0f;
    const int64_t stride = (int64_t)NPART * NORM_THREADS;
    int64_t i = (int64_t)blockIdx.x * NORM_THREADS + threadIdx.x;
    if constexpr (VEC) {
        const uint4 *xv = reinterpret_cast<const uint4 *>(x);
        const int64_t nv = numel >> 3;
        auto acc8 = [](float s, uint4 w) {
            const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float lo = __uint_as_float(u[k] << 16), hi = __uint_as_float(u[k] & 0xffff0000u);
                s = s + lo * lo;
                s = s + hi * hi;
            }
            return s;
        };
        for (; i + stride < nv; i += 2 * stride) {
            const uint4 w0 = xv[i], w1 = xv[i + stride];
            s0 = acc8(s0, w0);
            s1 = acc8(s1, w1);
        }
        if (i < nv) s0 = acc8(s0, xv[i]);
    } else {
        for (; i < numel; i += stride) {
            const float v = bf16_to_f32(x[i]);
            s0 = s0 + v * v;
        }
    }
    __shared__ float red[NORM_THREADS];
    red[threadIdx.x] = s0 + s1;
    __syncthreads();
    for (int w = NORM_THREADS / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[b * NPART + blockIdx.x] = red[0];
}

__device__ __forceinline__ float sumsq_of(const float *partial, int64_t b) {
    float s = 0.0f;
    for (int i = 0; i < NPART; ++i) s = s + partial[b * NPART + i];
    return s;
}

// d = bf16(bf16(||u||_F) + 1e-7) from the partial sums of matrix b (fixed order):
// the reference's bf16 normalisation (muon_sr/muon_sr.py:93), used for steps = 0.
__device__ __forceinline__ float norm_divisor(const float *partial, int64_t b) {
    const float nrm = __uint_as_float(rne_bf16(sqrtf(sumsq_of(partial, b))) << 16);
    return __uint_as_float(rne_bf16(nrm + 1e-7f) << 16);
}

// Vector form of normalize_kernel (below) for cols % 8 == 0 with 16-byte aligned
// `in`, S and T rows: each thread moves 8 consecutive bf16 (16 bytes) per access.
// Rp and Cp are multiples of 8 here, so an 8-wide chunk is entirely inside or
// entirely outside every extent it is checked against.
__global__ __launch_bounds__(256) void normalize_vec_kernel(const uint16_t *in, int64_t rows, int64_t cols,
                                                            const float *partial, uint16_t *S, int64_t ldS,
                                                            int64_t sS, uint16_t *T, int64_t ldT, int64_t sT,
                                                            int64_t Rp, int64_t Cp) {
    __shared__ __align__(16) uint16_t tile[64][72];
    __shared__ float dsh;
    const int64_t b = blockIdx.z;
    if (threadIdx.x == 0) dsh = norm_divisor(partial, b);
    __syncthreads();
    const float d = dsh;
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const uint16_t *x = in + b * rows * cols;
    const int j = threadIdx.x & 7, i0 = threadIdx.x >> 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = i0 + 32 * h;
        const int64_t r = r0 + i, c = c0 + 8 * j;
        uint4 w = make_uint4(0u, 0u, 0u, 0u);
        if (r < rows && c < cols) {
            const uint4 v = *reinterpret_cast<const uint4 *>(x + r * cols + c);
            const uint32_t u[4] = {v.x, v.y, v.z, v.w};
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float lo = __uint_as_float(u[k] << 16), hi = __uint_as_float(u[k] & 0xffff0000u);
                o[k] = rne_bf16x2(lo / d, hi / d);
            }
            w = make_uint4(o[0], o[1], o[2], o[3]);
        }
        *reinterpret_cast<uint4 *>(&tile[i][8 * j]) = w;
        if (S && r < Rp && c < Cp) *reinterpret_cast<uint4 *>(S + b * sS + r * ldS + c) = w;
    }
    if (!T) return;
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int cc = i0 + 32 * h;            // T row (input column) within the tile
        const int64_t c = c0 + cc, r = r0 + 8 * j;
        if (c < Cp && r < Rp) {
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                o[k] = (uint32_t)tile[8 * j + 2 * k][cc] | ((uint32_t)tile[8 * j + 2 * k + 1][cc] << 16);
            *reinterpret_cast<uint4 *>(T + b * sT + c * ldT + r) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// Writes S = x0 in the input layout (Rp x Cp, ld ldS) and T = x0^T (Cp x Rp, ld ldT),
// x0 = bf16(u / d), d = bf16(bf16(||u||_F) + 1e-7) (the reference's bf16
// normalisation: the output of steps == 0); zeros outside rows x cols.  S or T
// may be null.  64 x 64 tiles, transposed through LDS.
__global__ __launch_bounds__(256) void normalize_kernel(const uint16_t *in, int64_t rows, int64_t cols,
                                                        const float *partial, uint16_t *S, int64_t ldS, int64_t sS,
                                                        uint16_t *T, int64_t ldT, int64_t sT, int64_t Rp,
                                                        int64_t Cp) {
    __shared__ uint16_t tile[64][66];
    __shared__ float dsh;
    const int64_t b = blockIdx.z;
    if (threadIdx.x == 0) dsh = norm_divisor(partial, b);
    __syncthreads();
    const float d = dsh;
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const uint16_t *x = in + b * rows * cols;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        uint16_t h = 0;
        if (r < rows && c < cols) {
            const float v = bf16_to_f32(x[r * cols + c]);
            h = (uint16_t)rne_bf16(v / d);
        }
        tile[i][tx] = h;
        if (S && r < Rp && c < Cp) S[b * sS + r * ldS + c] = h;
    }
    __syncthreads();
    if (T) {
        for (int i = ty; i < 64; i += 4) {
            const int64_t c = c0 + i, r = r0 + tx;  // T[c][r]
            if (c < Cp && r < Rp) T[b * sT + c * ldT + r] = tile[tx][i];
        }
    }
}

// ---------------------------------------------------------------------------
// The iteration's prologue (steps >= 1): the update u (bf16) goes into the
// workspace's first iterate X0 (transposed for tall matrices, zero padding),
// with the sum of squares of each 64 x 64 tile of u, in one pass.  u comes
// either from a bf16 input (SRC_COPY: msr_newton_schulz) or from the Muon
// momentum step itself (SRC_PREPARE: msr_muon_fused_step, the arithmetic and
// noise of muon_prepare_kernel, muon_sr/triton_muon_sr.py:18-50: the momentum
// is updated in place and u is never written to memory).
//
// Sum of squares, in a fixed order whatever the source: thread t of a tile
// handles rows t/8 and t/8 + 32 of the tile, columns 8 (t%8) .. 8 (t%8) + 7,
// adding u^2 in fp32 element by element; the tile's 256 sums are reduced by
// an LDS tree into tpart[b][tile] (tiles in row-major order over the padded
// extents; padding adds +0); ns_finalize_kernel sums a matrix's tiles (thread
// t: tiles t, t + 256, ...; then an LDS tree).
//
// Scaling: X0 = u / (||u||_F + 1e-7) is not rounded.  With e the exponent of
// ||u||_F, X0 is kept as x0 = u when |e| <= PRO_ELIM (the first products then
// multiply by s = 1 / (||u|| + 1e-7): A = s^2 x0 x0^T, X' = s (B' x0 + ...)),
// else as x0 = u 2^-e with s0 = 2^e s (ns_rescale_kernel; bounded values keep
// products in range).  Both are the same numbers: bf16 products are exact in
// fp32 and every fp32 rounding of the products commutes with the power-of-two
// scale while no partial result leaves the normal range.
// ---------------------------------------------------------------------------

constexpr int PRO_MAX = 96;       // matrices per prologue launch (kernel-argument table)
constexpr int PRO_ELIM = 16;
enum ProSrc : int { SRC_COPY = 0, SRC_PREPARE = 1 };

struct PrologueArgs {
    const uint16_t *in;              // SRC_COPY: u, [batch][rows][cols] (matrix 0 of this launch)
    const void *grad[PRO_MAX];       // SRC_PREPARE: gradients (bf16, or fp32 with G32)
    uint16_t *buf;                   // SRC_PREPARE: momentum of matrix 0 of this launch, [batch][rows][cols]
    int64_t noise0;                  // SRC_PREPARE: noise offset of matrix 0 of this launch
    float beta;
    Noise ns;
    int64_t rows, cols;
    uint16_t *S; int64_t ldS, sS;    // X0 in the input layout (wide), or null
    uint16_t *T; int64_t ldT, sT;    // X0 = u^T (tall), or null
    int64_t Rp, Cp;                  // padded extents of u's layout
    float *tpart;                    // [batch][ntiles] (matrix 0 of this launch)
    int64_t ntx, ntiles;
};

// Tiles in runs of MSR_PRO_XCD consecutive tiles per XCD (4 rows of 32 tiles of a
// 2048-column matrix, 512 KiB of u): config 4's prologue 17 % faster than tiles in dispatch
// order (1.27 -> 1.06 ms per step; runs of 8, 16, 32 and 64: 12-16 %), bit-exact.
#ifndef MSR_PRO_XCD
#define MSR_PRO_XCD 128
#endif
template <int SRC, int MODE, bool NEST, bool G32, bool VEC>
__global__ __launch_bounds__(256) void ns_prologue_kernel(PrologueArgs a) {
    __shared__ __align__(16) uint16_t tile[64][72];
    __shared__ float red[256];
    // tile (tx, ty) of matrix b: work-groups in runs of MSR_PRO_XCD consecutive tiles per XCD
    const int64_t gx = gridDim.x, gy = gridDim.y;
    const int64_t lin = xcd_place((int64_t)blockIdx.x + gx * ((int64_t)blockIdx.y + gy * (int64_t)blockIdx.z),
                                  gx * gy * (int64_t)gridDim.z, MSR_PRO_XCD);
    const int64_t tx = lin % gx, ty = (lin / gx) % gy, b = lin / (gx * gy);
    const int64_t r0 = ty * 64, c0 = tx * 64;
    const int64_t numel = a.rows * a.cols;
    const int j = threadIdx.x & 7, i0 = threadIdx.x >> 3;
    const float one_m_beta = 1.0f - a.beta;
    float s = 0.0f;
    // Both rows' loads are issued before any store: the momentum is updated in place, so
    // the compiler would not move row 1's loads above row 0's stores by itself.
    uint32_t ld0[2][4] = {}, ld1[2][4] = {};   // SRC_COPY: u; SRC_PREPARE: bf16 gradient, momentum
    float g32[2][8];                            // SRC_PREPARE with G32: the gradient
    int64_t offs[2];
    int valids[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t r = r0 + i0 + 32 * h, c = c0 + 8 * j;
        valids[h] = (r < a.rows && c < a.cols) ? (int)min<int64_t>(8, a.cols - c) : 0;
        offs[h] = r * a.cols + c;
        if (valids[h] > 0) {
            if constexpr (SRC == SRC_COPY) {
                load_bf16x8<VEC>(a.in + b * numel, offs[h], valids[h], ld0[h]);
            } else {
                if constexpr (G32)
                    load_f32x8<VEC>(static_cast<const float *>(a.grad[b]) + offs[h], 0, valids[h], g32[h]);
                else
                    load_bf16x8<VEC>(static_cast<const uint16_t *>(a.grad[b]) + offs[h], 0, valids[h], ld0[h]);
                load_bf16x8<VEC>(a.buf + b * numel + offs[h], 0, valids[h], ld1[h]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = i0 + 32 * h;
        const int64_t r = r0 + i, c = c0 + 8 * j;
        uint32_t w[4] = {0u, 0u, 0u, 0u};   // u as bf16 pairs
        if (valids[h] > 0) {
            const int64_t off = offs[h];
            const int valid = valids[h];
            if constexpr (SRC == SRC_COPY) {
#pragma unroll
                for (int k = 0; k < 4; ++k) w[k] = ld0[h][k];
            } else {
                float gf[8], bf[8];
                uint32_t wb[4];
                if constexpr (G32) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) gf[k] = g32[h][k];
                } else {
                    unpack8(ld0[h], gf);
                }
                uint16_t *bp = a.buf + b * numel + off;
                unpack8(ld1[h], bf);
                const int64_t o0 = a.noise0 + b * numel + off;
                uint32_t rn[8];
                if (VEC || MODE != NOISE_PHILOX8) {
                    noise8<MODE>(a.ns, o0, valid, rn);
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) rn[k] = (k < valid) ? noise1<MODE>(a.ns, o0 + k) : 0u;
                }
                float up[8];
                uint32_t ob[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    float nb;
                    muon_momentum<NEST>(gf[k], bf[k], a.beta, one_m_beta, nb, up[k]);   // :37-42
                    ob[k] = sr_bf16(nb, rn[k]);                                         // :44-49
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    wb[k] = pack2(ob[2 * k], ob[2 * k + 1]);
                    // :50 (RNE); lanes beyond `valid` hold u = 0
                    w[k] = rne_bf16x2(2 * k < valid ? up[2 * k] : 0.0f, 2 * k + 1 < valid ? up[2 * k + 1] : 0.0f);
                }
                store_bf16x8<VEC>(bp, 0, valid, wb);
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float lo = bf16_lo(w[k]), hi = bf16_hi(w[k]);
            s = s + lo * lo;
            s = s + hi * hi;
        }
        *reinterpret_cast<uint4 *>(&tile[i][8 * j]) = make_uint4(w[0], w[1], w[2], w[3]);
        if (a.S && r < a.Rp && c < a.Cp) {
            uint16_t *d = a.S + b * a.sS + r * a.ldS + c;
            if (VEC) {
                *reinterpret_cast<uint4 *>(d) = make_uint4(w[0], w[1], w[2], w[3]);
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) d[k] = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
            }
        }
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int wdt = 128; wdt > 0; wdt >>= 1) {
        if (threadIdx.x < wdt) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + wdt];
        __syncthreads();
    }
    if (threadIdx.x == 0) a.tpart[b * a.ntiles + ty * a.ntx + tx] = red[0];
    if (!a.T) return;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int cc = i0 + 32 * h;            // T row (u column) within the tile
        const int64_t c = c0 + cc, r = r0 + 8 * j;
        if (c < a.Cp && r < a.Rp) {
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                o[k] = (uint32_t)tile[8 * j + 2 * k][cc] | ((uint32_t)tile[8 * j + 2 * k + 1][cc] << 16);
            uint16_t *d = a.T + b * a.sT + c * a.ldT + r;
            if (VEC) {
                *reinterpret_cast<uint4 *>(d) = make_uint4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) d[k] = (uint16_t)(o[k >> 1] >> (16 * (k & 1)));
            }
        }
    }
}

// Per matrix b: ||u||_F from the tile sums, the first products' factors
// alphas[b] = s^2, alphas[batch + b] = s, and rexp[b]: 0 when x0 = u, else -e
// (ns_rescale_kernel scales x0 by 2^-e).  ||u|| >= 2^64 (inf) gives e = 127 and
// s = 0 (u / inf = 0, as the reference's normalisation); NaN propagates.
__global__ __launch_bounds__(256) void ns_finalize_kernel(const float *tpart, int64_t ntiles, int64_t batch,
                                                          float *alphas, int *rexp, int *tile_ctr) {
    __shared__ float red[256];
    const int64_t b = blockIdx.x;
    if (b == 0 && threadIdx.x <= NXCD) tile_ctr[threadIdx.x] = 0;   // the GEMMs' tile counters start at zero
    float s = 0.0f;
    for (int64_t t = threadIdx.x; t < ntiles; t += 256) s = s + tpart[b * ntiles + t];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x != 0) return;
    const float d = sqrtf(red[0]);
    int e = 0;
    float s0;
    if (d == __builtin_huge_valf()) {
        e = 127;
        s0 = 0.0f;
    } else {
        if (d == d) (void)frexpf(d, &e);
        s0 = ldexpf(1.0f / (d + 1e-7f), e);
    }
    const bool scaled = e > PRO_ELIM || e < -PRO_ELIM;
    const float f = scaled ? s0 : ldexpf(s0, -e);   // exact for |e| <= PRO_ELIM: 1 / (||u|| + 1e-7)
    alphas[b] = f * f;
    alphas[batch + b] = f;
    rexp[b] = scaled ? -e : 0;
}

// x0 <- x0 2^rexp[b] over matrix b's padded X0 (n8 16-byte chunks at X + b sX),
// for the matrices the finalisation marked; the others return at once.  `bpm`
// work-groups per matrix: work-group g serves matrix g / bpm.
__global__ __launch_bounds__(256) void ns_rescale_kernel(uint16_t *X, int64_t sX, int64_t n8, int64_t bpm,
                                                         const int *rexp) {
    const int64_t b = blockIdx.x / bpm, part = blockIdx.x % bpm;
    const int ne = rexp[b];
    if (ne == 0) return;
    uint4 *x = reinterpret_cast<uint4 *>(X + b * sX);
    for (int64_t i = part * 256 + threadIdx.x; i < n8; i += bpm * 256) {
        const uint4 v = x[i];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = rne_bf16x2(ldexpf(bf16_lo(u[k]), ne), ldexpf(bf16_hi(u[k]), ne));
        x[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

static inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

struct NSLayout {
    int64_t m, n, mp, np;
    bool transposed;
    size_t off_x[2], off_a, off_b, off_part, off_alpha, off_rho, off_r, off_tpart, off_rexp, off_ctr, total;
    int64_t ntiles;   // 64 x 64 tiles of the padded update (prologue sums of squares)
};

static NSLayout ns_layout(int64_t batch, int64_t rows, int64_t cols) {
    NSLayout L;
    L.transposed = rows > cols;
    L.m = L.transposed ? cols : rows;
    L.n = L.transposed ? rows : cols;
    L.mp = round_up(L.m, 256);
    L.np = round_up(L.n, 256);
    const size_t xs = (size_t)batch * L.mp * L.np * 2;
    const size_t as = (size_t)batch * L.mp * L.mp * 2;
    size_t o = 0;
    auto take = [&](size_t s) { size_t r = o; o += (s + 255) & ~(size_t)255; return r; };
    L.off_x[0] = take(xs);
    L.off_x[1] = take(xs);
    L.off_a = take(as);
    L.off_b = take(as);
    L.off_part = take((size_t)batch * NPART * 4);
    L.off_alpha = take((size_t)batch * 2 * 4);     // alphas of the first A and X' products
    L.off_rho = take((size_t)batch * L.mp * 4);    // residuals of A's diagonal
    L.off_r = take((size_t)batch * L.mp * 4);      // residuals of B''s diagonal
    L.ntiles = (L.mp / 64) * (L.np / 64);
    L.off_tpart = take((size_t)batch * L.ntiles * 4);   // tile sums of squares of the update
    L.off_rexp = take((size_t)batch * 4);               // prologue scale exponents
    L.off_ctr = take(16 * 4);                           // the GEMMs' dynamic tile counters
    L.total = o;
    return L;
}

// Compute units of the stream's device (cached per device).
static int cu_count(hipStream_t s, int *cus) {
    static std::atomic<int> cache[64];
    int dev = 0;
    hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) { set_error("gemm: device of the stream: %s", hipGetErrorString(e)); return (int)e; }
    if (dev >= 0 && dev < 64 && (*cus = cache[dev].load(std::memory_order_relaxed)) > 0) return MSR_OK;
    e = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || *cus <= 0) { set_error("gemm: compute unit count: %s", hipGetErrorString(e)); return e ? (int)e : MSR_ERR_ARG; }
    if (dev >= 0 && dev < 64) cache[dev].store(*cus, std::memory_order_relaxed);
    return MSR_OK;
}

static int launch_gemm(const GemmArgs &a0, int64_t batch, hipStream_t s) {
    GemmArgs a = a0;
    // an operand read from upper-stored symmetric tiles is square
    if ((a.gm == GM_TRI_P && a.M != a.K) || (a.gm == GM_TRI_PQ && (a.M != a.K || a.N != a.K || !a.symmetric)) ||
        (a.symmetric && a.gm != GM_RR && a.gm != GM_TRI_PQ)) {
        set_error("gemm: operand layout %d does not fit a %d x %d x %d product", a.gm, a.M, a.N, a.K);
        return MSR_ERR_ARG;
    }
    // operand loads address one matrix with 32-bit byte offsets
    const bool pk = a.gm == GM_TRI_P || a.gm == GM_TRI_PQ || a.gm == GM_KK, prow = a.gm != GM_KK;
    const bool qk = a.gm != GM_RR, qrow = a.gm == GM_RR || a.gm == GM_TRI_PQ;
    int64_t span = 0;
    if (prow) span = std::max(span, (int64_t)(a.M - 1) * a.ldp + a.K);
    if (pk) span = std::max(span, (int64_t)(a.K - 1) * a.ldp + a.M);
    if (qrow) span = std::max(span, (int64_t)(a.N - 1) * a.ldq + a.K);
    if (qk) span = std::max(span, (int64_t)(a.K - 1) * a.ldq + a.N);
    if (span * 2 >= (int64_t(1) << 31)) {
        set_error("gemm: an operand matrix spans 2 GiB or more");
        return MSR_ERR_ARG;
    }
    a.tiles_m = a.M / BM;
    a.tiles_n = a.N / BN;
    a.d_vec = a.D && aligned(a.D, 16) && (a.ldd % 8) == 0 && (a.sD % 8) == 0;
    a.dt_vec = a.DT && aligned(a.DT, 16) && (a.lddt % 8) == 0 && (a.sDT % 8) == 0;
    if (a.apply1) {   // the store goes to the parameters of the table, each its own allocation
        if (batch > APPLY_MAX) { set_error("gemm: more than %d matrices in an apply launch", APPLY_MAX); return MSR_ERR_ARG; }
        bool al = true;
        for (int64_t i = 0; i < batch; ++i) al = al && aligned(a.ap.p[i], 16);
        a.d_vec = a.D && al && (a.ldd % 8) == 0;
        a.dt_vec = a.DT && al && (a.lddt % 8) == 0;
    }
    const int64_t tiles = a.symmetric ? (int64_t)a.tiles_m * (a.tiles_m + 1) / 2 : (int64_t)a.tiles_m * a.tiles_n;
    a.tiles = (int)tiles;
    // At most one work-group per CU (the LDS of one fills a CU), persistent
    // over the tiles.  With tile counters (a.tile_ctr, the Newton-Schulz
    // products) and more tiles than work-groups, each XCD's work-groups draw
    // the XCD's tiles in order from its counter, so the tiles in flight stay
    // neighbours in L2 however long the run.  Without counters the order is
    // static (tile v + grid): persistent while each work-group takes at most
    // PERSIST_MAX tiles, one tile per work-group beyond that (over longer
    // static runs the work-groups drift apart and the tiles in flight stop
    // sharing operand rows: one tile per work-group measured faster on the
    // 4096 x 14336 products, 56 tiles per CU).  A grid smaller than the launch
    // is a multiple of 8.
    int cus = 0;
    {
        const int rc = cu_count(s, &cus);
        if (rc) return rc;
    }
    const int64_t gmax = std::max<int64_t>(NXCD, cus / NXCD * NXCD);
    auto launch = [&](const GemmArgs &ab_in, int64_t total) {
        const dim3 block(GEMM_THREADS);
        // the dynamic order needs more tiles than work-groups (and then a grid of gmax,
        // a multiple of 8); otherwise the static one
        const bool dyn = ab_in.tile_ctr != nullptr && total > gmax;
        GemmArgs ab = ab_in;
        if (!dyn) ab.tile_ctr = nullptr;
        const dim3 grid((unsigned)(dyn ? gmax : total <= PERSIST_MAX * gmax ? std::min<int64_t>(total, gmax) : total));
        const bool c = ab.C != nullptr, d = ab.D != nullptr, dt = ab.DT != nullptr;
        const int gm = ab.gm;
        // every tile in range with 16-byte output rows: unconditional stores
        const bool full = ab.Mv == ab.M && ab.Nv == ab.N && (d ? ab.d_vec : ab.dt_vec) != 0;
        if (ab.sracc > 0) {   // weight gradient accumulated into D with SR
            if (gm != GM_KK || ab.symmetric || c || !d || dt) { set_error("gemm: unsupported SR-accumulating product"); return (int)MSR_ERR_ARG; }
            MSR_DISPATCH_NOISE(ab.sracc - 1, M, hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_KK, M, EPI_NONE, -1, true>), grid, block, 0, s, ab));
        } else if (ab.symmetric) {   // A = X X^T (RR), B' = c A A + b A + a I (TRI_PQ)
            if (gm == GM_RR && !c && d && !dt && ab.resid) {
                if (full) hipLaunchKernelGGL((gemm_nt_kernel<true, false, true, false, GM_RR, -1, EPI_A, -1, true>), grid, block, 0, s, ab);
                else hipLaunchKernelGGL((gemm_nt_kernel<true, false, true, false, GM_RR, -1, EPI_A>), grid, block, 0, s, ab);
            } else if (gm == GM_TRI_PQ && c && d && !dt && ab.resid && ab.rvec) {
                if (full) hipLaunchKernelGGL((gemm_nt_kernel<true, true, true, false, GM_TRI_PQ, -1, EPI_B, -1, true>), grid, block, 0, s, ab);
                else hipLaunchKernelGGL((gemm_nt_kernel<true, true, true, false, GM_TRI_PQ, -1, EPI_B>), grid, block, 0, s, ab);
            }
            else { set_error("gemm: unsupported symmetric product"); return (int)MSR_ERR_ARG; }
        } else if (gm == GM_TRI_P) {   // X' = B' X + r X: D = X', or DT = X'^T for the tall output
            if (!ab.rvec) { set_error("gemm: X' = B' X needs the diagonal residuals"); return (int)MSR_ERR_ARG; }
            if (ab.apply1 > 0) {   // the last product of msr_muon_ns_apply: D / DT are the parameters
                if (c || d == dt) { set_error("gemm: unsupported apply epilogue"); return (int)MSR_ERR_ARG; }
                if (d && full) { MSR_DISPATCH_NOISE(ab.apply1 - 1, M, hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_TRI_P, -1, EPI_X, M, true>), grid, block, 0, s, ab)); }
                else if (d) { MSR_DISPATCH_NOISE(ab.apply1 - 1, M, hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_TRI_P, -1, EPI_X, M>), grid, block, 0, s, ab)); }
                else if (full) { MSR_DISPATCH_NOISE(ab.apply1 - 1, M, hipLaunchKernelGGL((gemm_nt_kernel<false, false, false, true, GM_TRI_P, -1, EPI_X, M, true>), grid, block, 0, s, ab)); }
                else { MSR_DISPATCH_NOISE(ab.apply1 - 1, M, hipLaunchKernelGGL((gemm_nt_kernel<false, false, false, true, GM_TRI_P, -1, EPI_X, M>), grid, block, 0, s, ab)); }
            } else if (!c && d && !dt) {
                if (full) hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_TRI_P, -1, EPI_X, -1, true>), grid, block, 0, s, ab);
                else hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_TRI_P, -1, EPI_X>), grid, block, 0, s, ab);
            } else if (!c && !d && dt) {
                if (full) hipLaunchKernelGGL((gemm_nt_kernel<false, false, false, true, GM_TRI_P, -1, EPI_X, -1, true>), grid, block, 0, s, ab);
                else hipLaunchKernelGGL((gemm_nt_kernel<false, false, false, true, GM_TRI_P, -1, EPI_X>), grid, block, 0, s, ab);
            }
            else { set_error("gemm: unsupported epilogue combination"); return (int)MSR_ERR_ARG; }
        } else if (gm == GM_RK) {   // msr_gemm_nn
            if (c && d && !dt) hipLaunchKernelGGL((gemm_nt_kernel<false, true, true, false, GM_RK>), grid, block, 0, s, ab);
            else if (!c && d && !dt && full) hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_RK, -1, EPI_NONE, -1, true>), grid, block, 0, s, ab);
            else if (!c && d && !dt) hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_RK>), grid, block, 0, s, ab);
            else { set_error("gemm: unsupported epilogue combination"); return (int)MSR_ERR_ARG; }
        } else if (gm == GM_RR) {   // msr_gemm_nt
            if (c && d && !dt) hipLaunchKernelGGL((gemm_nt_kernel<false, true, true, false, GM_RR>), grid, block, 0, s, ab);
            else if (!c && d && !dt && full) hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_RR, -1, EPI_NONE, -1, true>), grid, block, 0, s, ab);
            else if (!c && d && !dt) hipLaunchKernelGGL((gemm_nt_kernel<false, false, true, false, GM_RR>), grid, block, 0, s, ab);
            else { set_error("gemm: unsupported epilogue combination"); return (int)MSR_ERR_ARG; }
        } else {
            set_error("gemm: unknown operand layout %d", gm);
            return (int)MSR_ERR_ARG;
        }
        return check_launch("gemm_nt_kernel");
    };
    auto offset = [&](int64_t b0) {
        GemmArgs ab = a;
        ab.P += b0 * a.sP;
        ab.Q += b0 * a.sQ;
        if (ab.C) ab.C += b0 * a.sC;
        if (ab.D) ab.D += b0 * a.sD;
        if (ab.DT) ab.DT += b0 * a.sDT;
        if (ab.alpha_b) ab.alpha_b += b0;
        if (ab.resid) ab.resid += b0 * a.sv;
        if (ab.rvec) ab.rvec += b0 * a.sv;
        if (ab.apply1) {   // the launch's matrix 0 is matrix b0 of the table (batch <= APPLY_MAX)
            for (int64_t i = 0; i + b0 < APPLY_MAX; ++i) {
                ab.ap.p[i] = a.ap.p[i + b0];
                ab.ap.seed[i] = a.ap.seed[i + b0];
            }
            if (ab.ap.inject) ab.ap.inject += b0 * a.ap.numel;
        }
        return ab;
    };
    // whole matrices per XCD for the largest multiple of 8 matrices, the
    // remainder spread per matrix; launches of fewer than 2^30 tiles
    const int64_t per_launch = (int64_t(1) << 30) / tiles;
    if (per_launch < 1) { set_error("gemm: a matrix of 2^30 tiles or more"); return MSR_ERR_ARG; }
    int64_t b0 = 0;
    // X' = B' X (GM_TRI_P) keeps whole matrices per XCD up to 192 tiles: 1 % faster on
    // 48 x 2048 x 5632 (176 tiles per matrix), equal elsewhere; the symmetric products
    // measured slower that way at 136 tiles (4096 x 4096)
    const int64_t per_xcd_max = a.gm == GM_TRI_P ? 192 : PER_XCD_TILES;
    while (tiles <= per_xcd_max && per_launch >= NXCD && batch - b0 >= NXCD) {
        const int64_t nb = std::min((batch - b0) / NXCD * NXCD, per_launch / NXCD * NXCD);
        GemmArgs ab = offset(b0);
        ab.per_xcd = 1;
        ab.total = (int)(tiles * nb);
        const int rc = launch(ab, ab.total);
        if (rc) return rc;
        b0 += nb;
    }
    while (b0 < batch) {
        const int64_t nb = std::min(batch - b0, per_launch);
        GemmArgs ab = offset(b0);
        ab.per_xcd = 0;
        ab.total = (int)(tiles * nb);
        const int rc = launch(ab, ab.total);
        if (rc) return rc;
        b0 += nb;
    }
    return MSR_OK;
}

}  // namespace msr

using namespace msr;

static int gemm_entry(const char *name, int qk, const uint16_t *P, int64_t ldp, int64_t strideP, const uint16_t *Q,
                      int64_t ldq, int64_t strideQ, const uint16_t *C, int64_t ldc, int64_t strideC, uint16_t *D,
                      int64_t ldd, int64_t strideD, int64_t M, int64_t N, int64_t K, int64_t batch, float alpha,
                      float beta, float diag, msr_stream_t stream) {
    if (!P || !Q || !D || batch < 0 || M <= 0 || N <= 0 || K <= 0 || (M % BM) || (N % BN) || (K % (2 * BK))) {
        set_error("%s: need M, N multiples of 256 and K a multiple of 128 (got %lld, %lld, %lld)", name,
                  (long long)M, (long long)N, (long long)K);
        return MSR_ERR_ARG;
    }
    if (!aligned(P, 16) || !aligned(Q, 16) || (ldp % 8) || (ldq % 8) || (strideP % 8) || (strideQ % 8) ||
        (C && beta != 0.0f && (!aligned(C, 16) || (ldc % 8) || (strideC % 8)))) {
        set_error("%s: P, Q and C must be 16-byte aligned with row and batch strides a multiple of 8 elements", name);
        return MSR_ERR_ALIGN;
    }
    if (batch == 0) return MSR_OK;
    GemmArgs a = {};
    a.P = P; a.ldp = ldp; a.sP = strideP;
    a.Q = Q; a.ldq = ldq; a.sQ = strideQ;
    a.C = (beta != 0.0f) ? C : nullptr; a.ldc = ldc; a.sC = strideC;
    a.D = D; a.ldd = ldd; a.sD = strideD;
    a.DT = nullptr;
    a.M = (int)M; a.N = (int)N; a.K = (int)K; a.Mv = (int)M; a.Nv = (int)N;
    a.alpha = alpha; a.beta = beta; a.diag = diag; a.symmetric = 0; a.gm = qk ? GM_RK : GM_RR;
    return launch_gemm(a, batch, (hipStream_t)stream);
}

extern "C" {

int msr_gemm_nt(const uint16_t *P, int64_t ldp, int64_t strideP, const uint16_t *Q, int64_t ldq, int64_t strideQ,
                const uint16_t *C, int64_t ldc, int64_t strideC, uint16_t *D, int64_t ldd, int64_t strideD, int64_t M,
                int64_t N, int64_t K, int64_t batch, float alpha, float beta, float diag, msr_stream_t stream) {
    return gemm_entry("msr_gemm_nt", 0, P, ldp, strideP, Q, ldq, strideQ, C, ldc, strideC, D, ldd, strideD, M, N, K,
                      batch, alpha, beta, diag, stream);
}

int msr_gemm_nn(const uint16_t *P, int64_t ldp, int64_t strideP, const uint16_t *Q, int64_t ldq, int64_t strideQ,
                const uint16_t *C, int64_t ldc, int64_t strideC, uint16_t *D, int64_t ldd, int64_t strideD, int64_t M,
                int64_t N, int64_t K, int64_t batch, float alpha, float beta, float diag, msr_stream_t stream) {
    return gemm_entry("msr_gemm_nn", 1, P, ldp, strideP, Q, ldq, strideQ, C, ldc, strideC, D, ldd, strideD, M, N, K,
                      batch, alpha, beta, diag, stream);
}

int msr_linear_wgrad_sr_accum(uint16_t *acc, const uint16_t *x, int64_t ldx, const uint16_t *dy, int64_t ldy,
                              int64_t tokens, int64_t in_features, int64_t out_features, uint32_t seed,
                              int32_t zero_init, int32_t noise_mode, const uint16_t *inject, msr_stream_t stream) {
    if (!acc || !x || !dy || tokens <= 0 || in_features <= 0 || out_features <= 0 || (in_features % BN) ||
        (out_features % BM) || (tokens % (2 * BK)) || ldx < in_features || ldy < out_features ||
        in_features >= (1 << 30) || out_features >= (1 << 30) || tokens >= (1 << 30)) {
        set_error("msr_linear_wgrad_sr_accum: need in and out features multiples of 256 and tokens a multiple of 128 "
                  "(got %lld, %lld, %lld)", (long long)in_features, (long long)out_features, (long long)tokens);
        return MSR_ERR_ARG;
    }
    if (noise_mode < 0 || noise_mode > 2 || (noise_mode == NOISE_INJECT && !inject)) {
        set_error("msr_linear_wgrad_sr_accum: bad noise_mode %d", (int)noise_mode);
        return MSR_ERR_ARG;
    }
    if (!aligned(acc, 16) || !aligned(x, 16) || !aligned(dy, 16) || (ldx % 8) || (ldy % 8)) {
        set_error("msr_linear_wgrad_sr_accum: acc, x and dy must be 16-byte aligned with row strides a multiple of 8");
        return MSR_ERR_ALIGN;
    }
    const size_t ab = 2 * (size_t)in_features * (size_t)out_features;
    const size_t xb = 2 * ((size_t)(tokens - 1) * (size_t)ldx + (size_t)in_features);
    const size_t yb = 2 * ((size_t)(tokens - 1) * (size_t)ldy + (size_t)out_features);
    auto touch = [](const void *p, size_t np, const void *q, size_t nq) {
        const uintptr_t u = (uintptr_t)p, v = (uintptr_t)q;
        return u < v + nq && v < u + np;
    };
    if (touch(acc, ab, x, xb) || touch(acc, ab, dy, yb)) {
        set_error("msr_linear_wgrad_sr_accum: acc overlaps x or dy");
        return MSR_ERR_OVERLAP;
    }
    GemmArgs a = {};
    a.P = dy; a.ldp = ldy; a.sP = 0;   // P[o][t] = dy[t][o], K-major
    a.Q = x; a.ldq = ldx; a.sQ = 0;    // Q[i][t] = x[t][i], K-major
    a.C = nullptr;
    a.D = acc; a.ldd = in_features; a.sD = 0;
    a.DT = nullptr;
    a.M = (int)out_features; a.N = (int)in_features; a.K = (int)tokens; a.Mv = a.M; a.Nv = a.N;
    a.alpha = 1.0f; a.beta = 0.0f; a.diag = 0.0f; a.symmetric = 0; a.gm = GM_KK;
    a.sracc = 1 + noise_mode;
    a.zero_init = zero_init != 0;
    a.ns.key = seed_key(seed, 0);
    a.ns.inject = inject;
    return launch_gemm(a, 1, (hipStream_t)stream);
}

int msr_ns_workspace_bytes(int64_t batch, int64_t rows, int64_t cols, size_t *bytes) {
    if (!bytes || batch < 0 || rows <= 0 || cols <= 0) { set_error("msr_ns_workspace_bytes: bad arguments"); return MSR_ERR_ARG; }
    *bytes = ns_layout(batch, rows, cols).total;
    return MSR_OK;
}

}  // extern "C"

// The fused Muon apply of msr_muon_ns_apply (host tables of `batch` entries).
struct NSApply {
    uint16_t *const *params;
    const uint32_t *seeds;
    float lr, weight_decay, scale;
    int noise_mode;
    const uint16_t *inject;
};

// The Muon momentum step that produces the update inside the prologue
// (msr_muon_fused_step): gradients, the momentum of the call's matrix 0 and the
// index of that matrix in its momentum stack (the noise counter's base).
struct NSPrepare {
    const void *const *grads;
    bool g32;
    uint16_t *buf;
    int64_t first;
    float beta;
    bool nesterov;
    Noise ns;
    int noise_mode;
};

// Matrices [b0, b0 + batch) of a Newton-Schulz call, all of one shape group.
// Every part of a call has the same Newton-Schulz shape (m x n, m <= n); a
// part of rows > cols (tall) is iterated transposed.  The input is `in` (a
// [batch][rows][cols] stack), or the update made by the momentum step of `pp`;
// the last product writes `out` ([batch][rows][cols]), or, with `ap`, updates
// the parameters (then `out` only marks the layout and is never accessed).
struct NSPart {
    int64_t b0, batch, rows, cols;
    const uint16_t *in;
    uint16_t *out;
    const NSApply *ap;
    const NSPrepare *pp;
};

// The prologue of one part: its X0 (at X0 + b0 xs) and tile sums (see ns_prologue_kernel).
static int ns_prologue_part(const NSPart &pt, uint16_t *X0, float *tpart, const NSLayout &L, hipStream_t s) {
    const int64_t rows = pt.rows, cols = pt.cols, numel = rows * cols, xs = L.mp * L.np;
    const bool transposed = rows > cols;
    const int64_t Rp = transposed ? L.np : L.mp;
    const int64_t Cp = transposed ? L.mp : L.np;
    const NSPrepare *pp = pt.pp;
    bool vec = (cols % 8) == 0;
    if (pp) {
        vec = vec && aligned(pp->buf, 16);
        for (int64_t i = 0; i < pt.batch && vec; ++i) vec = aligned(pp->grads[i], 16);
    } else {
        vec = vec && aligned(pt.in, 16);
    }
    for (int64_t b0 = 0; b0 < pt.batch; b0 += PRO_MAX) {
        const int64_t nb = std::min<int64_t>(PRO_MAX, pt.batch - b0);
        uint16_t *x0 = X0 + (pt.b0 + b0) * xs;
        PrologueArgs a = {};
        a.rows = rows; a.cols = cols;
        a.S = transposed ? nullptr : x0; a.ldS = Cp; a.sS = xs;
        a.T = transposed ? x0 : nullptr; a.ldT = Rp; a.sT = xs;
        a.Rp = Rp; a.Cp = Cp;
        a.tpart = tpart + (pt.b0 + b0) * L.ntiles;
        a.ntx = Cp / 64; a.ntiles = L.ntiles;
        const dim3 grid((unsigned)(Cp / 64), (unsigned)(Rp / 64), (unsigned)nb);
        if (!pp) {
            a.in = pt.in + b0 * numel;
            if (vec) hipLaunchKernelGGL((ns_prologue_kernel<SRC_COPY, NOISE_TRITON, false, false, true>), grid, dim3(256), 0, s, a);
            else hipLaunchKernelGGL((ns_prologue_kernel<SRC_COPY, NOISE_TRITON, false, false, false>), grid, dim3(256), 0, s, a);
        } else {
            for (int64_t i = 0; i < nb; ++i) a.grad[i] = pp->grads[b0 + i];
            a.buf = pp->buf + b0 * numel;
            a.noise0 = (pp->first + b0) * numel;
            a.beta = pp->beta;
            a.ns = pp->ns;
#define PRO_LAUNCH(NEST, G, V) MSR_DISPATCH_NOISE(pp->noise_mode, M, hipLaunchKernelGGL((ns_prologue_kernel<SRC_PREPARE, M, NEST, G, V>), grid, dim3(256), 0, s, a))
            if (pp->g32) {
                if (pp->nesterov) { if (vec) { PRO_LAUNCH(true, true, true); } else { PRO_LAUNCH(true, true, false); } }
                else { if (vec) { PRO_LAUNCH(false, true, true); } else { PRO_LAUNCH(false, true, false); } }
            } else {
                if (pp->nesterov) { if (vec) { PRO_LAUNCH(true, false, true); } else { PRO_LAUNCH(true, false, false); } }
                else { if (vec) { PRO_LAUNCH(false, false, true); } else { PRO_LAUNCH(false, false, false); } }
            }
#undef PRO_LAUNCH
        }
        int rc = check_launch("ns_prologue_kernel");
        if (rc) return rc;
    }
    return MSR_OK;
}

// After the parts' prologues, over all `batch` matrices of the call: the first
// products' factors and the rescale of out-of-range matrices.
static int ns_prologue_finish(int64_t batch, uint16_t *X0, float *tpart, float *alphas, int *rexp, int *tile_ctr,
                              const NSLayout &L, hipStream_t s) {
    const int64_t xs = L.mp * L.np;
    hipLaunchKernelGGL(ns_finalize_kernel, dim3((unsigned)batch), dim3(256), 0, s, tpart, L.ntiles, batch, alphas, rexp,
                       tile_ctr);
    int rc = check_launch("ns_finalize_kernel");
    if (rc) return rc;
    const int64_t n8 = xs / 8, bpm = std::min<int64_t>((n8 + 255) / 256, 64);
    hipLaunchKernelGGL(ns_rescale_kernel, dim3((unsigned)(bpm * batch)), dim3(256), 0, s, X0, xs, n8, bpm, rexp);
    return check_launch("ns_rescale_kernel");
}

// Newton-Schulz (steps >= 1) of the `batch` matrices of `parts` (which cover
// [0, batch) in order): one prologue per part, the iterations over the whole
// batch, and the last product per part.  Arguments are validated by the callers.
static int ns_run_parts(const NSPart *parts, int n_parts, int64_t batch, int32_t steps, float a_coef, float b_coef,
                        float c_coef, void *workspace, const NSLayout &L, hipStream_t s) {
    char *ws = static_cast<char *>(workspace);
    uint16_t *X[2] = {(uint16_t *)(ws + L.off_x[0]), (uint16_t *)(ws + L.off_x[1])};
    uint16_t *A = (uint16_t *)(ws + L.off_a);
    uint16_t *B = (uint16_t *)(ws + L.off_b);
    float *alphas = (float *)(ws + L.off_alpha);   // [0, batch): s0^2, [batch, 2 batch): s0
    float *tpart = (float *)(ws + L.off_tpart);
    float *rho = (float *)(ws + L.off_rho);
    float *rr = (float *)(ws + L.off_r);
    int *tile_ctr = (int *)(ws + L.off_ctr);
    const int64_t xs = L.mp * L.np, as = L.mp * L.mp;
    int rc = MSR_OK;
    for (int i = 0; i < n_parts; ++i)
        if ((rc = ns_prologue_part(parts[i], X[0], tpart, L, s))) return rc;
    if ((rc = ns_prologue_finish(batch, X[0], tpart, alphas, (int *)(ws + L.off_rexp), tile_ctr, L, s))) return rc;

    const int mp = (int)L.mp, np = (int)L.np;
    int cur = 0;
    for (int it = 0; it < steps; ++it) {
        const bool last = it == steps - 1;
        GemmArgs g = {};
        // A = X X^T, upper tiles stored
        g.P = X[cur]; g.ldp = np; g.sP = xs;
        g.Q = X[cur]; g.ldq = np; g.sQ = xs;
        g.C = nullptr;
        g.D = A; g.ldd = mp; g.sD = as;
        g.DT = nullptr;
        g.M = mp; g.N = mp; g.K = np; g.Mv = mp; g.Nv = mp;
        g.alpha = 1.0f; g.beta = 0.0f; g.symmetric = 1; g.gm = GM_RR;
        g.alpha_b = it == 0 ? alphas : nullptr;   // s0^2 x0 x0^T
        g.resid = rho; g.sv = mp;
        g.tile_ctr = tile_ctr;
        if ((rc = launch_gemm(g, batch, s))) return rc;
        // B' = c (A A) + b A + a I (diagonal corrected for rho), reading A's lower tiles as the
        // transposed upper ones; upper tiles stored
        g = GemmArgs{};
        g.P = A; g.ldp = mp; g.sP = as;
        g.Q = A; g.ldq = mp; g.sQ = as;
        g.C = A; g.ldc = mp; g.sC = as;
        g.D = B; g.ldd = mp; g.sD = as;
        g.M = mp; g.N = mp; g.K = mp; g.Mv = mp; g.Nv = mp;
        g.alpha = c_coef; g.beta = b_coef; g.diag = a_coef; g.symmetric = 1; g.gm = GM_TRI_PQ;
        g.rvec = rho; g.resid = rr; g.sv = mp;
        g.tile_ctr = tile_ctr;
        if ((rc = launch_gemm(g, batch, s))) return rc;
        // X' = B' X + r X (= B X + a X), X read K-major, B' lower tiles as the transposed upper ones
        g = GemmArgs{};
        g.P = B; g.ldp = mp; g.sP = as;
        g.Q = X[cur]; g.ldq = np; g.sQ = xs;
        g.C = nullptr;
        g.M = mp; g.N = np; g.K = mp;
        g.alpha = 1.0f; g.beta = 0.0f; g.symmetric = 0; g.gm = GM_TRI_P;
        g.alpha_b = it == 0 ? alphas + batch : nullptr;   // s0 (B' x0 + r x0)
        g.rvec = rr; g.sv = mp;
        g.tile_ctr = tile_ctr;
        if (!last) {
            g.D = X[cur ^ 1]; g.ldd = np; g.sD = xs;
            g.DT = nullptr;
            g.Mv = mp; g.Nv = np;
            if ((rc = launch_gemm(g, batch, s))) return rc;
            cur ^= 1;
            continue;
        }
        for (int i = 0; i < n_parts; ++i) {   // the last product, per part: its output layout and update
            const NSPart &pt = parts[i];
            if (pt.batch == 0) continue;
            const int64_t numel = pt.rows * pt.cols;
            GemmArgs gp = g;
            gp.P += pt.b0 * g.sP;
            gp.Q += pt.b0 * g.sQ;
            gp.alpha_b = g.alpha_b ? g.alpha_b + pt.b0 : nullptr;
            gp.rvec += pt.b0 * g.sv;
            gp.Mv = (int)L.m; gp.Nv = (int)L.n;
            if (pt.rows <= pt.cols) {
                gp.D = pt.out; gp.ldd = pt.cols; gp.sD = numel;     // out[m][n], m = rows, n = cols
                gp.DT = nullptr;
            } else {
                gp.D = nullptr;
                gp.DT = pt.out; gp.lddt = pt.cols; gp.sDT = numel;  // out[n][m], n = rows, m = cols
            }
            const NSApply *ap = pt.ap;
            if (!ap) {
                if ((rc = launch_gemm(gp, pt.batch, s))) return rc;
                continue;
            }
            // the store updates params[b] (the layout of out) in launches of up to APPLY_MAX matrices
            gp.apply1 = 1 + ap->noise_mode;
            gp.ap.numel = numel;
            gp.ap.lr = ap->lr;
            gp.ap.decay = 1.0f - ap->lr * ap->weight_decay;          // :72
            gp.ap.scale = ap->scale;
            for (int64_t b0 = 0; b0 < pt.batch; b0 += APPLY_MAX) {
                const int64_t nb = std::min<int64_t>(APPLY_MAX, pt.batch - b0);
                GemmArgs ga = gp;
                ga.P += b0 * gp.sP;
                ga.Q += b0 * gp.sQ;
                ga.alpha_b = gp.alpha_b ? gp.alpha_b + b0 : nullptr;
                ga.rvec += b0 * gp.sv;
                for (int64_t j = 0; j < nb; ++j) {
                    ga.ap.p[j] = ap->params[b0 + j];
                    ga.ap.seed[j] = ap->seeds[b0 + j];
                }
                ga.ap.inject = ap->inject ? ap->inject + b0 * numel : nullptr;
                if ((rc = launch_gemm(ga, nb, s))) return rc;
            }
        }
    }
    return MSR_OK;
}

// Newton-Schulz of `batch` matrices of one shape; with `ap`, the last product
// updates the parameters instead of writing `out` (which is then unused); with
// `pp`, the update is made by the Muon momentum step in the prologue (`in` is
// unused).  Arguments are validated by the callers.
static int ns_run(const uint16_t *in, uint16_t *out, int64_t batch, int64_t rows, int64_t cols, int32_t steps,
                  float a_coef, float b_coef, float c_coef, void *workspace, const NSLayout &L, hipStream_t s,
                  const NSApply *ap, const NSPrepare *pp = nullptr) {
    if (steps >= 1) {
        const NSPart part{0, batch, rows, cols, in, out, ap, pp};
        return ns_run_parts(&part, 1, batch, steps, a_coef, b_coef, c_coef, workspace, L, s);
    }
    // steps == 0: the output is the reference's bf16 normalisation of the input
    char *ws = static_cast<char *>(workspace);
    float *part = (float *)(ws + L.off_part);
    const int64_t numel = rows * cols;
    // 16-byte accesses when every row of the input starts 16-byte aligned
    const bool vec = (cols % 8) == 0 && aligned(in, 16);
    if (vec)
        hipLaunchKernelGGL(sumsq_kernel<true>, dim3(NPART, (unsigned)batch), dim3(NORM_THREADS), 0, s, in, numel, part);
    else
        hipLaunchKernelGGL(sumsq_kernel<false>, dim3(NPART, (unsigned)batch), dim3(NORM_THREADS), 0, s, in, numel, part);
    int rc = check_launch("sumsq_kernel");
    if (rc) return rc;
    const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64), (unsigned)batch);
    const bool v = vec && aligned(out, 16) && cols % 8 == 0 && numel % 8 == 0 && rows % 8 == 0;
    if (v)
        hipLaunchKernelGGL(normalize_vec_kernel, grid, dim3(256), 0, s, in, rows, cols, part, out, cols, numel, nullptr,
                           0, 0, rows, cols);
    else
        hipLaunchKernelGGL(normalize_kernel, grid, dim3(256), 0, s, in, rows, cols, part, out, cols, numel, nullptr, 0,
                           0, rows, cols);
    return check_launch("normalize_kernel");
}

extern "C" {

int msr_newton_schulz(const uint16_t *in, uint16_t *out, int64_t batch, int64_t rows, int64_t cols, int32_t steps,
                      float a_coef, float b_coef, float c_coef, void *workspace, size_t workspace_bytes,
                      msr_stream_t stream) {
    if (!in || !out || batch < 0 || rows <= 0 || cols <= 0 || steps < 0) { set_error("msr_newton_schulz: bad arguments"); return MSR_ERR_ARG; }
    if (batch == 0) return MSR_OK;
    const NSLayout L = ns_layout(batch, rows, cols);
    if (!workspace || workspace_bytes < L.total) {
        set_error("msr_newton_schulz: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, L.total);
        return MSR_ERR_WORKSPACE;
    }
    if (L.mp > (1 << 30) || L.np > (1 << 30)) { set_error("msr_newton_schulz: matrix too large"); return MSR_ERR_ARG; }
    {
        // the input is consumed before the output is written, so in and out may
        // share memory; neither may share the workspace
        const uintptr_t w = (uintptr_t)workspace, i0 = (uintptr_t)in, o0 = (uintptr_t)out;
        const size_t io = 2 * (size_t)batch * (size_t)rows * (size_t)cols;
        if ((w < i0 + io && i0 < w + L.total) || (w < o0 + io && o0 < w + L.total)) {
            set_error("msr_newton_schulz: the workspace overlaps the input or the output");
            return MSR_ERR_OVERLAP;
        }
    }
    return ns_run(in, out, batch, rows, cols, steps, a_coef, b_coef, c_coef, workspace, L, (hipStream_t)stream, nullptr);
}

int msr_muon_ns_apply(const uint16_t *upd, uint16_t *const *params, const uint32_t *seeds, int64_t batch, int64_t rows,
                      int64_t cols, int32_t steps, float a_coef, float b_coef, float c_coef, float lr,
                      float weight_decay, float scale, int32_t noise_mode, const uint16_t *inject, void *workspace,
                      size_t workspace_bytes, msr_stream_t stream) {
    if (!upd || batch < 0 || rows <= 0 || cols <= 0 || steps < 1 || (batch > 0 && (!params || !seeds))) {
        set_error("msr_muon_ns_apply: bad arguments (steps must be >= 1)");
        return MSR_ERR_ARG;
    }
    if (noise_mode < 0 || noise_mode > 2 || (noise_mode == NOISE_INJECT && !inject)) {
        set_error("msr_muon_ns_apply: bad noise_mode %d", (int)noise_mode);
        return MSR_ERR_ARG;
    }
    if (batch == 0) return MSR_OK;
    const NSLayout L = ns_layout(batch, rows, cols);
    if (!workspace || workspace_bytes < L.total) {
        set_error("msr_muon_ns_apply: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, L.total);
        return MSR_ERR_WORKSPACE;
    }
    if (L.mp > (1 << 30) || L.np > (1 << 30)) { set_error("msr_muon_ns_apply: matrix too large"); return MSR_ERR_ARG; }
    {
        // the parameters are written while the update stack and the workspace are read: no
        // parameter may share memory with them or with another parameter
        const size_t pb = 2 * (size_t)rows * (size_t)cols, ub = pb * (size_t)batch;
        auto touch = [](const void *x, size_t nx, const void *y, size_t ny) {
            return (uintptr_t)x < (uintptr_t)y + ny && (uintptr_t)y < (uintptr_t)x + nx;
        };
        if (touch(upd, ub, workspace, L.total)) {
            set_error("msr_muon_ns_apply: the workspace overlaps the update stack");
            return MSR_ERR_OVERLAP;
        }
        for (int64_t i = 0; i < batch; ++i) {
            if (!params[i]) { set_error("msr_muon_ns_apply: null parameter pointer %lld", (long long)i); return MSR_ERR_ARG; }
            bool race = touch(params[i], pb, upd, ub) || touch(params[i], pb, workspace, L.total);
            for (int64_t j = 0; j < i && !race; ++j) race = touch(params[i], pb, params[j], pb);
            if (race) {
                set_error("msr_muon_ns_apply: parameter %lld overlaps another parameter, the update stack or the workspace",
                          (long long)i);
                return MSR_ERR_OVERLAP;
            }
        }
    }
    NSApply ap{params, seeds, lr, weight_decay, scale, (int)noise_mode, inject};
    // `out` only marks the output layout for the last product: the store writes params[b]
    return ns_run(upd, const_cast<uint16_t *>(upd), batch, rows, cols, steps, a_coef, b_coef, c_coef, workspace, L,
                  (hipStream_t)stream, &ap);
}

int msr_muon_fused_step(const void *const *grads, int32_t grads_f32, uint16_t *buf, int64_t first, int64_t batch,
                        int64_t rows, int64_t cols, float beta, int32_t nesterov, uint32_t prepare_seed, int32_t steps,
                        float a_coef, float b_coef, float c_coef, uint16_t *out, uint16_t *const *params,
                        const uint32_t *apply_seeds, float lr, float weight_decay, float scale, int32_t noise_mode,
                        const uint16_t *inject_prepare, const uint16_t *inject_apply, void *workspace,
                        size_t workspace_bytes, msr_stream_t stream) {
    if (!grads || !buf || first < 0 || batch < 0 || rows <= 0 || cols <= 0 || steps < 1 ||
        (batch > 0 && !params && !out) || (params && !apply_seeds)) {
        set_error("msr_muon_fused_step: bad arguments (steps must be >= 1; params with seeds, or out)");
        return MSR_ERR_ARG;
    }
    if (noise_mode < 0 || noise_mode > 2 ||
        (noise_mode == NOISE_INJECT && (!inject_prepare || (params && !inject_apply)))) {
        set_error("msr_muon_fused_step: bad noise_mode %d", (int)noise_mode);
        return MSR_ERR_ARG;
    }
    if (batch == 0) return MSR_OK;
    const NSLayout L = ns_layout(batch, rows, cols);
    if (!workspace || workspace_bytes < L.total) {
        set_error("msr_muon_fused_step: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, L.total);
        return MSR_ERR_WORKSPACE;
    }
    if (L.mp > (1 << 30) || L.np > (1 << 30)) { set_error("msr_muon_fused_step: matrix too large"); return MSR_ERR_ARG; }
    {
        // the momentum and the parameters (or the output) are written while the gradients,
        // the momentum and the workspace are read: none may share memory with another, except
        // that gradients may repeat
        const size_t gb = (grads_f32 ? 4 : 2) * (size_t)rows * (size_t)cols, pb = 2 * (size_t)rows * (size_t)cols;
        const size_t bb = pb * (size_t)batch;
        auto touch = [](const void *x, size_t nx, const void *y, size_t ny) {
            return (uintptr_t)x < (uintptr_t)y + ny && (uintptr_t)y < (uintptr_t)x + nx;
        };
        if (touch(buf, bb, workspace, L.total) || (out && (touch(out, bb, workspace, L.total) || touch(out, bb, buf, bb)))) {
            set_error("msr_muon_fused_step: the momentum, the output and the workspace must not overlap");
            return MSR_ERR_OVERLAP;
        }
        for (int64_t i = 0; i < batch; ++i) {
            if (!grads[i]) { set_error("msr_muon_fused_step: null gradient pointer %lld", (long long)i); return MSR_ERR_ARG; }
            if (touch(grads[i], gb, buf, bb) || touch(grads[i], gb, workspace, L.total) || (out && touch(grads[i], gb, out, bb))) {
                set_error("msr_muon_fused_step: gradient %lld overlaps the momentum, the output or the workspace", (long long)i);
                return MSR_ERR_OVERLAP;
            }
        }
        if (params) {
            for (int64_t i = 0; i < batch; ++i) {
                if (!params[i]) { set_error("msr_muon_fused_step: null parameter pointer %lld", (long long)i); return MSR_ERR_ARG; }
                bool race = touch(params[i], pb, buf, bb) || touch(params[i], pb, workspace, L.total);
                for (int64_t j = 0; j < batch && !race; ++j) race = touch(params[i], pb, grads[j], gb);
                for (int64_t j = 0; j < i && !race; ++j) race = touch(params[i], pb, params[j], pb);
                if (race) {
                    set_error("msr_muon_fused_step: parameter %lld overlaps another operand", (long long)i);
                    return MSR_ERR_OVERLAP;
                }
            }
        }
    }
    Noise pns;
    pns.key = seed_key(prepare_seed, 0);
    pns.inject = inject_prepare;   // indexed by the element offset in the momentum stack
    NSPrepare pp{grads, grads_f32 != 0, buf, first, beta, nesterov != 0, pns, (int)noise_mode};
    if (!params)
        return ns_run(nullptr, out, batch, rows, cols, steps, a_coef, b_coef, c_coef, workspace, L, (hipStream_t)stream,
                      nullptr, &pp);
    NSApply ap{params, apply_seeds, lr, weight_decay, scale, (int)noise_mode, inject_apply};
    // the last product's store writes params[b]: its `out` only marks the output layout (never accessed)
    return ns_run(nullptr, static_cast<uint16_t *>(workspace), batch, rows, cols, steps, a_coef, b_coef, c_coef,
                  workspace, L, (hipStream_t)stream, &ap, &pp);
}

int msr_muon_fused_steps(const msr_muon_group *groups, int32_t n_groups, float beta, int32_t nesterov, int32_t steps,
                         float a_coef, float b_coef, float c_coef, float lr, float weight_decay, int32_t noise_mode,
                         void *workspace, size_t workspace_bytes, msr_stream_t stream) {
    if (!groups || n_groups < 1 || steps < 1) {
        set_error("msr_muon_fused_steps: bad arguments (at least one group; steps must be >= 1)");
        return MSR_ERR_ARG;
    }
    if (noise_mode != NOISE_TRITON && noise_mode != NOISE_PHILOX8) {
        set_error("msr_muon_fused_steps: bad noise_mode %d (injected noise: msr_muon_fused_step)", (int)noise_mode);
        return MSR_ERR_ARG;
    }
    const int64_t m = std::min(groups[0].rows, groups[0].cols), n = std::max(groups[0].rows, groups[0].cols);
    int64_t total = 0;
    for (int32_t i = 0; i < n_groups; ++i) {
        const msr_muon_group &g = groups[i];
        if (!g.grads || !g.buf || !g.params || !g.apply_seeds || g.first < 0 || g.batch < 0 || g.rows <= 0 ||
            g.cols <= 0) {
            set_error("msr_muon_fused_steps: bad arguments in group %d", (int)i);
            return MSR_ERR_ARG;
        }
        if (std::min(g.rows, g.cols) != m || std::max(g.rows, g.cols) != n) {
            set_error("msr_muon_fused_steps: group %d is %lld x %lld, group 0 %lld x %lld: the groups of a call must "
                      "have the same shape up to transposition", (int)i, (long long)g.rows, (long long)g.cols,
                      (long long)groups[0].rows, (long long)groups[0].cols);
            return MSR_ERR_ARG;
        }
        total += g.batch;
    }
    if (total == 0) return MSR_OK;
    const NSLayout L = ns_layout(total, m, n);
    if (!workspace || workspace_bytes < L.total) {
        set_error("msr_muon_fused_steps: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                  L.total);
        return MSR_ERR_WORKSPACE;
    }
    if (L.mp > (1 << 30) || L.np > (1 << 30)) { set_error("msr_muon_fused_steps: matrix too large"); return MSR_ERR_ARG; }
    {
        // as msr_muon_fused_step, across the groups: the momenta and the parameters are
        // written while the gradients, the momenta and the workspace are read; none may
        // share memory with another, except that gradients may repeat
        const size_t pb = 2 * (size_t)m * (size_t)n;
        auto touch = [](const void *x, size_t nx, const void *y, size_t ny) {
            return (uintptr_t)x < (uintptr_t)y + ny && (uintptr_t)y < (uintptr_t)x + nx;
        };
        auto gbytes = [&](const msr_muon_group &g) { return (g.grads_f32 ? 4 : 2) * (size_t)m * (size_t)n; };
        auto bbytes = [&](const msr_muon_group &g) { return pb * (size_t)g.batch; };
        for (int32_t i = 0; i < n_groups; ++i) {
            const msr_muon_group &gi = groups[i];
            bool race = touch(gi.buf, bbytes(gi), workspace, L.total);
            for (int32_t j = 0; j < i && !race; ++j) race = touch(gi.buf, bbytes(gi), groups[j].buf, bbytes(groups[j]));
            if (race) {
                set_error("msr_muon_fused_steps: the momentum of group %d overlaps the workspace or another momentum",
                          (int)i);
                return MSR_ERR_OVERLAP;
            }
            for (int64_t k = 0; k < gi.batch; ++k) {
                if (!gi.grads[k] || !gi.params[k]) {
                    set_error("msr_muon_fused_steps: null pointer in group %d, matrix %lld", (int)i, (long long)k);
                    return MSR_ERR_ARG;
                }
                race = touch(gi.grads[k], gbytes(gi), workspace, L.total);
                for (int32_t j = 0; j < n_groups && !race; ++j)
                    race = touch(gi.grads[k], gbytes(gi), groups[j].buf, bbytes(groups[j]));
                if (race) {
                    set_error("msr_muon_fused_steps: gradient %lld of group %d overlaps a momentum or the workspace",
                              (long long)k, (int)i);
                    return MSR_ERR_OVERLAP;
                }
            }
        }
        for (int32_t i = 0; i < n_groups; ++i) {
            for (int64_t k = 0; k < groups[i].batch; ++k) {
                const void *p = groups[i].params[k];
                bool race = touch(p, pb, workspace, L.total);
                for (int32_t j = 0; j < n_groups && !race; ++j) {
                    const msr_muon_group &gj = groups[j];
                    race = touch(p, pb, gj.buf, bbytes(gj));
                    for (int64_t l = 0; l < gj.batch && !race; ++l) race = touch(p, pb, gj.grads[l], gbytes(gj));
                    for (int64_t l = 0; l < gj.batch && !race && (j < i || (j == i && l < k)); ++l)
                        race = touch(p, pb, gj.params[l], pb);
                }
                if (race) {
                    set_error("msr_muon_fused_steps: parameter %lld of group %d overlaps another operand", (long long)k,
                              (int)i);
                    return MSR_ERR_OVERLAP;
                }
            }
        }
    }
    std::vector<NSPrepare> pps((size_t)n_groups);
    std::vector<NSApply> aps((size_t)n_groups);
    std::vector<NSPart> parts((size_t)n_groups);
    int64_t b0 = 0;
    for (int32_t i = 0; i < n_groups; ++i) {
        const msr_muon_group &g = groups[i];
        Noise pns;
        pns.key = seed_key(g.prepare_seed, 0);
        pns.inject = nullptr;
        pps[i] = NSPrepare{g.grads, g.grads_f32 != 0, g.buf, g.first, beta, nesterov != 0, pns, (int)noise_mode};
        aps[i] = NSApply{g.params, g.apply_seeds, lr, weight_decay, g.scale, (int)noise_mode, nullptr};
        // the last product's store writes params[b]: `out` only marks the output layout (never accessed)
        parts[i] = NSPart{b0, g.batch, g.rows, g.cols, nullptr, static_cast<uint16_t *>(workspace), &aps[i], &pps[i]};
        b0 += g.batch;
    }
    return ns_run_parts(parts.data(), (int)n_groups, total, steps, a_coef, b_coef, c_coef, workspace, L,
                        (hipStream_t)stream);
}

}  // extern "C"
