// elementwise.hip -- the reference's per-token vector ops on gfx950.
//
// Op-level equivalents of ops::rms_norm_inplace (ops.cpp:107-118),
// softmax_inplace (ops.cpp:242-259), silu_inplace (ops.cpp:218-222),
// add/mul/scale_inplace (ops.cpp:269-285) and dispatch_dot_f32
// (backend.cpp:109-127).  Reductions run in one workgroup (the vectors are
// hidden-size or context-length long) with a fixed tree order, so results
// are deterministic run to run; they differ from the reference's sequential
// fp32 sums only by summation order.
#include <algorithm>

#include "common.h"

namespace qraf_hip {

constexpr int EW = 1024;

// Block-wide sum; every thread gets the result.  `red` holds >= 16 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < nw; i++) t = fmaxf(t, red[i]);
    return t;
}

__global__ __launch_bounds__(EW) void rms_norm_kernel(float* __restrict__ x, const float* __restrict__ w, int n,
                                                     float eps) {
    __shared__ float red[16];
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += EW) ss = __builtin_fmaf(x[i], x[i], ss);
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += EW) x[i] = x[i] * r * w[i];
}

__global__ __launch_bounds__(EW) void softmax_kernel(float* __restrict__ x, int n) {
    __shared__ float red[16];
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += EW) m = fmaxf(m, x[i]);
    m = block_max(m, red);
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += EW) {
        float e = expf(x[i] - m);
        x[i] = e;
        s += e;
    }
    s = block_sum(s, red);
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < n; i += EW) x[i] *= inv;
}

__global__ __launch_bounds__(EW) void dot_kernel(const float* __restrict__ a, const float* __restrict__ b, int n,
                                                float* __restrict__ out) {
    __shared__ float red[16];
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += EW) s = __builtin_fmaf(a[i], b[i], s);
    s = block_sum(s, red);
    if (threadIdx.x == 0) *out = s;
}

// op: 0 silu, 1 add, 2 mul, 3 scale
__global__ void ew_kernel(int op, float* __restrict__ x, const float* __restrict__ y, float s, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = x[i];
    switch (op) {
        case 0: v = v / (1.0f + expf(-v)); break;
        case 1: v = v + y[i]; break;
        case 2: v = v * y[i]; break;
        default: v = v * s; break;
    }
    x[i] = v;
}

int launch_rms_norm(float* x, const float* w, int n, float eps, hipStream_t s) {
    QH_REQUIRE(x && w && n > 0, QRAF_HIP_ERR_INVALID, "bad rms_norm arguments");
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(EW), 0, s, x, w, n, eps);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_softmax(float* x, int n, hipStream_t s) {
    QH_REQUIRE(x && n > 0, QRAF_HIP_ERR_INVALID, "bad softmax arguments");
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(EW), 0, s, x, n);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_dot(const float* a, const float* b, int n, float* out, hipStream_t s) {
    QH_REQUIRE(a && b && out && n > 0, QRAF_HIP_ERR_INVALID, "bad dot arguments");
    hipLaunchKernelGGL(dot_kernel, dim3(1), dim3(EW), 0, s, a, b, n, out);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_ew(int op, float* x, const float* y, float sc, int n, hipStream_t s) {
    QH_REQUIRE(x && n > 0 && (op == 0 || op == 3 || y), QRAF_HIP_ERR_INVALID, "bad elementwise arguments");
    hipLaunchKernelGGL(ew_kernel, dim3((n + 255) / 256), dim3(256), 0, s, op, x, y, sc, n);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

// Streaming read of a buffer: the plain-read ceiling a memory-bound kernel of
// the same bytes is measured against.  Grid-stride over 16-byte
// nontemporal loads, 8 in flight per thread, 2048 workgroups of 256 threads
// (one pass for buffers up to 64 MB).  Of the read shapes
// swept on MI355X for one launch over 19-51 MB (grid-stride and contiguous
// chunk per workgroup, 4-16 loads in flight per thread, 256-1024 threads,
// 256 workgroups to one per chunk, plain and nontemporal loads) this one was
// the fastest or within 1% of it.  Each wave writes the sum of what it read,
// so no load is dead.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int RP_WGS = 2048, RP_WG = 256, RP_U = 8;
__global__ __launch_bounds__(RP_WG) void read_probe_kernel(const f32x4* __restrict__ p, size_t n4, float* out) {
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    const size_t step = (size_t)gridDim.x * RP_WG * RP_U;
    for (size_t base = (size_t)blockIdx.x * RP_WG * RP_U + threadIdx.x; base < n4; base += step) {
        f32x4 v[RP_U];
#pragma unroll
        for (int u = 0; u < RP_U; u++) v[u] = __builtin_nontemporal_load(p + std::min(base + (size_t)u * RP_WG, n4 - 1));
#pragma unroll
        for (int u = 0; u < RP_U; u++) a += base + (size_t)u * RP_WG < n4 ? v[u] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float v = (a[0] + a[1]) + (a[2] + a[3]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * (RP_WG / 64) + (threadIdx.x >> 6)] = v;
}

size_t read_probe_out_floats() { return (size_t)RP_WGS * (RP_WG / 64); }

// An empty kernel: the fixed cost of one launch of `wgs` 64-thread
// workgroups, the floor under every kernel of a latency-bound step.
__global__ __launch_bounds__(64) void empty_kernel() {}

int launch_empty(int wgs, hipStream_t s) {
    QH_REQUIRE(wgs > 0 && wgs <= 65536, QRAF_HIP_ERR_INVALID, "empty launch: %d workgroups", wgs);
    hipLaunchKernelGGL(empty_kernel, dim3(wgs), dim3(64), 0, s);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_read_probe(const void* p, size_t bytes, float* out, hipStream_t s) {
    QH_REQUIRE(p && out && bytes > 0 && bytes % 16 == 0 && ((uintptr_t)p & 15) == 0, QRAF_HIP_ERR_INVALID,
               "read probe: null or misaligned pointer, or bytes not a positive multiple of 16");
    // always RP_WGS workgroups, so that every output slot is written (those past the data write 0)
    hipLaunchKernelGGL(read_probe_kernel, dim3(RP_WGS), dim3(RP_WG), 0, s, (const f32x4*)p, bytes / 16, out);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip
