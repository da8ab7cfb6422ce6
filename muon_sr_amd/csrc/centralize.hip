// Gradient centralization of TritonAdamW on the device (muon_sr/triton_adamw.py:179-187):
//     g' = bf16_rne( g - mean_over_all_but_dim0(g) * c )      (fp32 arithmetic)
// The reference runs this as five host-issued torch passes (fp32 copy, mean,
// scale, subtract, bf16 cast; about 24 bytes of traffic per element).  Here it
// is three launches over (row, chunk) work-groups reading the bf16 gradient
// twice and writing the bf16 result once (6 bytes per element):
//   1. row_partial_kernel   fp32 partial sums of CENT_CHUNK-element chunks
//   2. row_mean_kernel      per row: the partials summed in chunk order,
//                           m = (sum / cols) * c
//   3. centralize_kernel    g' = bf16_rne(g - m)
// Every sum has a fixed order (per-thread strides, then a fixed LDS tree), so
// results do not depend on the launch or on the other rows.
#include <mutex>

#include "common.hpp"
#include "vecio.hpp"
#include "../../include/muon_sr_amd.h"

namespace msr {

constexpr int CENT_THREADS = 256;
constexpr int64_t CENT_CHUNK = 16384;   // elements of one row per work-group

struct CentArgs {
    const uint16_t *g;
    uint16_t *out;
    int64_t rows, cols, chunks;
    float *partial;   // [rows * chunks]
    float *mean;      // [rows]
    float alpha;
    int vec;          // cols % 8 == 0 and g, out 16-byte aligned
};

__device__ __forceinline__ float block_sum(float s, float *red) {
    red[threadIdx.x] = s;
    __syncthreads();
#pragma unroll
    for (int w = CENT_THREADS / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    return red[0];
}

__global__ __launch_bounds__(CENT_THREADS) void row_partial_kernel(CentArgs a) {
    __shared__ float red[CENT_THREADS];
    const int64_t wg = blockIdx.x;
    const int64_t r = wg / a.chunks, c = wg - r * a.chunks;
    const int64_t c0 = c * CENT_CHUNK;
    const int64_t n = min(CENT_CHUNK, a.cols - c0);
    const uint16_t *x = a.g + r * a.cols + c0;
    float s = 0.0f;
    if (a.vec) {
        for (int64_t i = (int64_t)threadIdx.x * 8; i < n; i += CENT_THREADS * 8) {
            const uint4 w = *reinterpret_cast<const uint4 *>(x + i);
            const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                s = s + bf16_lo(u[k]);
                s = s + bf16_hi(u[k]);
            }
        }
    } else {
        for (int64_t i = threadIdx.x; i < n; i += CENT_THREADS) s = s + bf16_to_f32(x[i]);
    }
    const float t = block_sum(s, red);
    if (threadIdx.x == 0) a.partial[wg] = t;
}

__global__ __launch_bounds__(CENT_THREADS) void row_mean_kernel(CentArgs a) {
    const int64_t r = (int64_t)blockIdx.x * CENT_THREADS + threadIdx.x;
    if (r >= a.rows) return;
    float s = 0.0f;
    for (int64_t c = 0; c < a.chunks; ++c) s = s + a.partial[r * a.chunks + c];
    const float mean = s / (float)a.cols;
    a.mean[r] = mean * a.alpha;
}

__global__ __launch_bounds__(CENT_THREADS) void centralize_kernel(CentArgs a) {
    const int64_t wg = blockIdx.x;
    const int64_t r = wg / a.chunks, c = wg - r * a.chunks;
    const int64_t c0 = c * CENT_CHUNK;
    const int64_t n = min(CENT_CHUNK, a.cols - c0);
    const uint16_t *x = a.g + r * a.cols + c0;
    uint16_t *y = a.out + r * a.cols + c0;
    const float m = a.mean[r];
    if (a.vec) {
        for (int64_t i = (int64_t)threadIdx.x * 8; i < n; i += CENT_THREADS * 8) {
            const uint4 w = *reinterpret_cast<const uint4 *>(x + i);
            const uint32_t u[4] = {w.x, w.y, w.z, w.w};
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = rne_bf16x2(bf16_lo(u[k]) - m, bf16_hi(u[k]) - m);
            *reinterpret_cast<uint4 *>(y + i) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    } else {
        for (int64_t i = threadIdx.x; i < n; i += CENT_THREADS) y[i] = (uint16_t)rne_bf16(bf16_to_f32(x[i]) - m);
    }
}

static size_t cent_ws(int64_t rows, int64_t chunks) {
    return ((size_t)(rows * chunks) * 4 + 255) / 256 * 256 + (size_t)rows * 4;
}

// The three launches over a workspace of cent_ws(rows, chunks) bytes (validated by the caller).
static int centralize_launch(const uint16_t *g, uint16_t *out, int64_t rows, int64_t cols, int64_t chunks,
                             float alpha, char *workspace, hipStream_t s) {
    CentArgs a;
    a.g = g; a.out = out; a.rows = rows; a.cols = cols; a.chunks = chunks;
    a.partial = reinterpret_cast<float *>(workspace);
    a.mean = reinterpret_cast<float *>(workspace + ((size_t)(rows * chunks) * 4 + 255) / 256 * 256);
    a.alpha = alpha;
    a.vec = (cols % 8) == 0 && aligned(g, 16) && aligned(out, 16);
    const unsigned wgs = (unsigned)(rows * chunks);
    hipLaunchKernelGGL(row_partial_kernel, dim3(wgs), dim3(CENT_THREADS), 0, s, a);
    int rc = check_launch("row_partial_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(row_mean_kernel, dim3((unsigned)((rows + CENT_THREADS - 1) / CENT_THREADS)), dim3(CENT_THREADS), 0,
                       s, a);
    if ((rc = check_launch("row_mean_kernel"))) return rc;
    hipLaunchKernelGGL(centralize_kernel, dim3(wgs), dim3(CENT_THREADS), 0, s, a);
    return check_launch("centralize_kernel");
}

// ---------------------------------------------------------------------------
// Scratch of msr_centralize_bf16_noalloc: a file-scope device array, one copy
// per GPU for the life of the process.  Its device address is looked up once
// per device (hipGetSymbolAddress with that device current) and only that
// address is used by host code: the array's name is a host-side stand-in.
// Every word a call reads is written earlier in the same call (partials by
// row_partial_kernel, means by row_mean_kernel), so nothing is cleared.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[MSR_CENTRALIZE_NOALLOC_SCRATCH_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;
static std::mutex scratch_mu;
static void *scratch_ptr[SCRATCH_MAX_DEVICES];

// Device address of `scratch` on the device of `stream` (the current device for the
// null stream), looked up on the first call for that device.
static int scratch_for(hipStream_t stream, char **out) {
    int dev = 0;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) { set_error("scratch: no device for the stream (%s)", hipGetErrorString(e)); return (int)e; }
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) { set_error("scratch: device %d out of range", dev); return MSR_ERR_ARG; }
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        int cur = 0;
        if ((e = hipGetDevice(&cur)) != hipSuccess) { set_error("scratch: hipGetDevice: %s", hipGetErrorString(e)); return (int)e; }
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) {
            set_error("scratch: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
            return (int)e;
        }
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p) {
            set_error("scratch: hipGetSymbolAddress on device %d: %s", dev, hipGetErrorString(e));
            return e != hipSuccess ? (int)e : MSR_ERR_LAUNCH;
        }
        scratch_ptr[dev] = p;
    }
    *out = static_cast<char *>(scratch_ptr[dev]);
    return MSR_OK;
}

}  // namespace msr

using namespace msr;

extern "C" {

int msr_centralize_workspace_bytes(int64_t rows, int64_t cols, size_t *bytes) {
    if (!bytes || rows < 0 || cols < 0) { set_error("msr_centralize_workspace_bytes: bad arguments"); return MSR_ERR_ARG; }
    *bytes = cent_ws(rows, cols > 0 ? (cols + CENT_CHUNK - 1) / CENT_CHUNK : 0);
    return MSR_OK;
}

int msr_centralize_bf16(const uint16_t *g, uint16_t *out, int64_t rows, int64_t cols, float alpha, void *workspace,
                        size_t workspace_bytes, msr_stream_t stream) {
    if (rows < 0 || cols < 0 || (rows > 0 && cols > 0 && (!g || !out))) {
        set_error("msr_centralize_bf16: bad arguments");
        return MSR_ERR_ARG;
    }
    if (rows == 0 || cols == 0) return MSR_OK;
    const int64_t chunks = (cols + CENT_CHUNK - 1) / CENT_CHUNK;
    if (rows * chunks >= (int64_t(1) << 31)) { set_error("msr_centralize_bf16: too many rows"); return MSR_ERR_ARG; }
    const size_t need = cent_ws(rows, chunks);
    if (!workspace || workspace_bytes < need) {
        set_error("msr_centralize_bf16: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, need);
        return MSR_ERR_WORKSPACE;
    }
    const size_t gb = 2 * (size_t)rows * (size_t)cols;
    const bool ws_hit = [&] {
        const uintptr_t w = (uintptr_t)workspace, g0 = (uintptr_t)g, o0 = (uintptr_t)out;
        return (w < g0 + gb && g0 < w + need) || (w < o0 + gb && o0 < w + need);
    }();
    if (partial_overlap(g, gb, out, gb) || ws_hit) {
        set_error("msr_centralize_bf16: g, out and the workspace overlap (only out == g is allowed)");
        return MSR_ERR_OVERLAP;
    }
    return centralize_launch(g, out, rows, cols, chunks, alpha, static_cast<char *>(workspace), (hipStream_t)stream);
}

int msr_centralize_bf16_noalloc(const uint16_t *g, uint16_t *out, int64_t rows, int64_t cols, float alpha,
                                msr_stream_t stream) {
    if (rows < 0 || cols < 0 || (rows > 0 && cols > 0 && (!g || !out))) {
        set_error("msr_centralize_bf16_noalloc: bad arguments");
        return MSR_ERR_ARG;
    }
    if (rows == 0 || cols == 0) return MSR_OK;
    const int64_t chunks = (cols + CENT_CHUNK - 1) / CENT_CHUNK;
    if (rows > (int64_t(1) << 31) / chunks || cent_ws(rows, chunks) > MSR_CENTRALIZE_NOALLOC_SCRATCH_BYTES) {
        set_error("msr_centralize_bf16_noalloc: %lld rows x %lld chunks need more than the %d bytes of scratch "
                  "(use msr_centralize_bf16 with a workspace)", (long long)rows, (long long)chunks,
                  (int)MSR_CENTRALIZE_NOALLOC_SCRATCH_BYTES);
        return MSR_ERR_WORKSPACE;
    }
    const size_t gb = 2 * (size_t)rows * (size_t)cols;
    if (partial_overlap(g, gb, out, gb)) {
        set_error("msr_centralize_bf16_noalloc: g and out overlap (only out == g is allowed)");
        return MSR_ERR_OVERLAP;
    }
    hipStream_t s = (hipStream_t)stream;
    char *ws = nullptr;
    const int rc = scratch_for(s, &ws);
    if (rc) return rc;
    return centralize_launch(g, out, rows, cols, chunks, alpha, ws, s);
}

}  // extern "C"
