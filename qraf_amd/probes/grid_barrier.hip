// grid_barrier.hip -- cost of a grid-wide barrier inside one launch, against a launch boundary, and the
// read rate of the workgroups of one XCD.
//
//     grid_barrier
//
// Counter barrier: each workgroup adds 1 to one counter (agent-scope release) and polls it (acquire)
// until every workgroup of the round has arrived.  Flag barrier: workgroup w release-stores its own flag,
// thread t of every workgroup polls flag t.  Workgroups whose index is not a multiple of `stride` exit
// at once (workgroups are dealt to the 8 XCDs in turn, so stride 8 keeps one XCD's).  Every spin is
// bounded: a wave that polls more than LIMIT times sets the error flag and leaves, so no launch can hang
// (the printed timeout flag must be 0).  Then back-to-back empty launches, and 64 MB streamed by all CUs,
// by one XCD and by two.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)
constexpr unsigned LIMIT = 1u << 22;

// barrier among the workgroups with (blockIdx.x % stride == 0) (the others exit at once);
// gen-counting barrier: arrive with a release add, wait with acquire loads.
__global__ void bar_kernel(unsigned* cnt, int iters, int stride, unsigned nwg, int* err, float* sink) {
    if (blockIdx.x % stride) return;
    __shared__ int bad;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    float acc = 0.f;
    for (int it = 0; it < iters; it++) {
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned target = (unsigned)(it + 1) * nwg;
            __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            unsigned spins = 0;
            while (__hip_atomic_load(cnt, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
                if (++spins > LIMIT) { bad = 1; break; }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        if (bad) break;
        acc += (float)it;
    }
    if (threadIdx.x == 0 && bad) atomicOr(err, 1);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}


// flag-array barrier: workgroup w release-stores flag[w] = round; thread t (< nwg) of every workgroup
// polls flag[t] with acquire loads.  SLEEP 0: pure spin.
template <int SLEEP>
__global__ void flag_kernel(unsigned* flags, int iters, unsigned nwg, int* err, float* sink) {
    __shared__ int bad;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    float acc = 0.f;
    for (int it = 0; it < iters; it++) {
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_store(&flags[blockIdx.x], (unsigned)(it + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x < nwg) {
            unsigned spins = 0;
            while (__hip_atomic_load(&flags[threadIdx.x], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)(it + 1)) {
                if (++spins > LIMIT) { bad = 1; break; }
                if (SLEEP) __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        if (bad) break;
        acc += (float)it;
    }
    if (threadIdx.x == 0 && bad) atomicOr(err, 1);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

// streaming read by the workgroups with (blockIdx.x % stride == 0): nwg of them
__global__ __launch_bounds__(256) void read_kernel(const uint4* __restrict__ p, size_t n16, int stride, unsigned nwg, float* sink) {
    if (blockIdx.x % stride) return;
    const unsigned w = blockIdx.x / stride;
    uint32_t a = 0;
    for (size_t i = (size_t)w * 256 + threadIdx.x; i < n16; i += (size_t)nwg * 256 * 4) {
        uint4 v0 = p[i];
        uint4 v1 = (i + (size_t)nwg * 256 < n16) ? p[i + (size_t)nwg * 256] : uint4{0, 0, 0, 0};
        uint4 v2 = (i + 2 * (size_t)nwg * 256 < n16) ? p[i + 2 * (size_t)nwg * 256] : uint4{0, 0, 0, 0};
        uint4 v3 = (i + 3 * (size_t)nwg * 256 < n16) ? p[i + 3 * (size_t)nwg * 256] : uint4{0, 0, 0, 0};
        a ^= v0.x ^ v1.y ^ v2.z ^ v3.w;
    }
    if (a == 0x12345678u) sink[0] = 1.f;
}

int main() {
    unsigned* cnt; int* err; float* sink;
    CK(hipMalloc(&cnt, 4)); CK(hipMalloc(&err, 4)); CK(hipMalloc(&sink, 1 << 20));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    const int iters = 2000;
    struct { int wgs, stride; const char* what; } cfg[] = {
        {256, 1, "256 WGs, all XCDs"}, {128, 1, "128 WGs"}, {64, 1, "64 WGs"},
        {256, 8, "32 WGs on one XCD (stride 8 of 256)"}, {64, 8, "8 WGs on one XCD"}};
    for (auto& c : cfg) {
        const unsigned nwg = (c.wgs + c.stride - 1) / c.stride;
        CK(hipMemset(cnt, 0, 4)); CK(hipMemset(err, 0, 4));
        hipLaunchKernelGGL(bar_kernel, dim3(c.wgs), dim3(256), 0, 0, cnt, 10, c.stride, nwg, err, sink);
        CK(hipDeviceSynchronize());
        CK(hipMemset(cnt, 0, 4));
        CK(hipEventRecord(e0, 0));
        hipLaunchKernelGGL(bar_kernel, dim3(c.wgs), dim3(256), 0, 0, cnt, iters, c.stride, nwg, err, sink);
        CK(hipEventRecord(e1, 0));
        CK(hipEventSynchronize(e1));
        float ms; CK(hipEventElapsedTime(&ms, e0, e1));
        int h_err; CK(hipMemcpy(&h_err, err, 4, hipMemcpyDeviceToHost));
        printf("barrier %-40s: %.3f us per barrier (timeout flag %d)\n", c.what, ms * 1e3 / iters, h_err);
        fflush(stdout);
    }
    unsigned* flags; CK(hipMalloc(&flags, 4096));
    for (int nw : {256, 128, 64}) {
        for (int sl = 0; sl < 2; sl++) {
            CK(hipMemset(flags, 0, 4096)); CK(hipMemset(err, 0, 4));
            CK(hipEventRecord(e0, 0));
            if (sl) hipLaunchKernelGGL((flag_kernel<1>), dim3(nw), dim3(256), 0, 0, flags, iters, (unsigned)nw, err, sink);
            else hipLaunchKernelGGL((flag_kernel<0>), dim3(nw), dim3(256), 0, 0, flags, iters, (unsigned)nw, err, sink);
            CK(hipEventRecord(e1, 0));
            CK(hipEventSynchronize(e1));
            float ms; CK(hipEventElapsedTime(&ms, e0, e1));
            int h_err; CK(hipMemcpy(&h_err, err, 4, hipMemcpyDeviceToHost));
            printf("flag barrier %3d WGs, sleep %d: %.3f us per barrier (timeout flag %d)\n", nw, sl, ms * 1e3 / iters, h_err);
            fflush(stdout);
        }
    }
    // empty-kernel launch gap for comparison
    {
        CK(hipEventRecord(e0, 0));
        for (int i = 0; i < 1000; i++) hipLaunchKernelGGL(bar_kernel, dim3(256), dim3(256), 0, 0, cnt, 0, 1, 256u, err, sink);
        CK(hipEventRecord(e1, 0));
        CK(hipEventSynchronize(e1));
        float ms; CK(hipEventElapsedTime(&ms, e0, e1));
        printf("back-to-back empty 256-WG launches: %.3f us each\n", ms * 1e3 / 1000);
    }
    // bandwidth: 64 MB read by all CUs vs by one XCD
    const size_t bytes = 256u << 20;
    uint4* buf; CK(hipMalloc(&buf, bytes)); CK(hipMemset(buf, 1, bytes));
    struct { int wgs, stride; const char* what; } rc[] = {
        {2048, 1, "2048 WGs (all XCDs)"}, {256, 1, "256 WGs (all XCDs)"}, {256, 8, "32 WGs, one XCD"},
        {512, 8, "64 WGs, one XCD"}, {1024, 8, "128 WGs, one XCD"}, {1024, 4, "256 WGs, two XCDs"}};
    for (auto& c : rc) {
        const unsigned nwg = c.wgs / c.stride;
        const size_t n16 = (64u << 20) / 16;
        for (int rep = 0; rep < 2; rep++) {
            CK(hipEventRecord(e0, 0));
            for (int i = 0; i < 20; i++)
                hipLaunchKernelGGL(read_kernel, dim3(c.wgs), dim3(256), 0, 0, buf + (size_t)(i % 4) * n16, n16, c.stride, nwg, sink);
            CK(hipEventRecord(e1, 0));
            CK(hipEventSynchronize(e1));
            float ms; CK(hipEventElapsedTime(&ms, e0, e1));
            if (rep) printf("read 64 MB by %-24s: %.2f us, %.2f TB/s\n", c.what, ms * 1e3 / 20, (64u << 20) / (ms * 1e-3 / 20) / 1e12);
        }
        fflush(stdout);
    }
    return 0;
}
