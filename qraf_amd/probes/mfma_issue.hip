// mfma_issue.hip -- issue rate of v_mfma_f32_16x16x32_f16 in the operand pattern of the three-product GEMM
// (gemm_three_product.hip), operands in registers, no memory traffic.
//
//     mfma_issue
//
// Per wave TM x TN accumulators, three dependent MFMAs per accumulator per step; ORDER 0 issues them in
// the GEMM's order (per batch tile: the three products of its TN accumulators), ORDER 1 plane-outer over
// all accumulators (dependent MFMAs TM*TN apart).  Prints PFLOP/s and the fraction of the 2.5 PFLOP/s
// dense fp16 peak for several waves per workgroup and grid sizes.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)

template <int TM, int TN, int ORDER, int WV>
__global__ __launch_bounds__(64 * WV) void mb_kernel(const f16x8* __restrict__ src, int iters, float* out) {
    const int lane = threadIdx.x & 63;
    f16x8 a[TM], al[TM], w[TN], wl[TN];
#pragma unroll
    for (int t = 0; t < TM; t++) { a[t] = src[(t * 64 + lane) & 1023]; al[t] = src[(t * 64 + lane + 7) & 1023]; }
#pragma unroll
    for (int u = 0; u < TN; u++) { w[u] = src[(u * 64 + lane + 3) & 1023]; wl[u] = src[(u * 64 + lane + 5) & 1023]; }
    f32x4 acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int u = 0; u < TN; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; it++) {
        if (ORDER == 0) {
#pragma unroll
            for (int t = 0; t < TM; t++) {
#pragma unroll
                for (int u = 0; u < TN; u++) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], w[u], acc[t][u], 0, 0, 0);
#pragma unroll
                for (int u = 0; u < TN; u++) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t], w[u], acc[t][u], 0, 0, 0);
#pragma unroll
                for (int u = 0; u < TN; u++) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], wl[u], acc[t][u], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int u = 0; u < TN; u++) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], w[u], acc[t][u], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int u = 0; u < TN; u++) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t], w[u], acc[t][u], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int u = 0; u < TN; u++) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], wl[u], acc[t][u], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int u = 0; u < TN; u++) s += acc[t][u][0] + acc[t][u][1] + acc[t][u][2] + acc[t][u][3];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <int TM, int TN, int ORDER, int waves_per_wg>
static void run( int wgs, const f16x8* src, float* out) {
    const int iters = 2000;
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    hipLaunchKernelGGL((mb_kernel<TM, TN, ORDER, waves_per_wg>), dim3(wgs), dim3(64 * waves_per_wg), 0, 0, src, 10, out);
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL((mb_kernel<TM, TN, ORDER, waves_per_wg>), dim3(wgs), dim3(64 * waves_per_wg), 0, 0, src, iters, out);
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    float ms; CK(hipEventElapsedTime(&ms, e0, e1));
    const double flops = 2.0 * 16 * 16 * 32 * 3.0 * TM * TN * iters * (double)waves_per_wg * wgs;
    const double pf = flops / (ms * 1e-3) / 1e15;
    printf("TM%d TN%d order %d, %2d waves/WG x %4d WGs: %.3f PFLOP/s (%.3f of 2.5)\n", TM, TN, ORDER, waves_per_wg, wgs, pf, pf / 2.5);
    fflush(stdout);
}

int main() {
    f16x8* src; float* out;
    CK(hipMalloc(&src, 1024 * sizeof(f16x8)));
    CK(hipMemset(src, 0, 1024 * sizeof(f16x8)));
    CK(hipMalloc(&out, 4096 * 1024 * 4));
    run<8, 2, 0, 8>(256, src, out);
    run<8, 2, 1, 8>(256, src, out);
    run<8, 2, 0, 4>(256, src, out);
    run<8, 2, 1, 4>(256, src, out);
    run<8, 2, 0, 16>(256, src, out);
    run<8, 2, 1, 16>(256, src, out);
    run<8, 4, 1, 4>(256, src, out);
    run<8, 4, 1, 8>(256, src, out);
    run<4, 2, 1, 16>(256, src, out);
    run<8, 1, 1, 16>(256, src, out);
    run<8, 2, 1, 8>(512, src, out);
    run<8, 2, 1, 8>(172, src, out);
    return 0;
}
