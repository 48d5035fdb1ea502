// read_sweep.hip -- plain-read ceiling of one launch on this device.
//
//     read_sweep [bytes]     (default 50,785,280: the Q8_0 11008x4096 matvec's weights)
//
// Reads `bytes` from one of at least 8 copies in turn (together over 320 MB,
// more than the 256 MB last-level cache, so every launch streams from HBM),
// in two forms:
// grid-stride (workgroup w starts at chunk w, stride = grid x threads x U)
// and contiguous chunk (workgroup w reads bytes/grid consecutive bytes),
// with U 16-byte loads in flight per thread, 256-1024 threads per workgroup,
// plain or nontemporal loads, and grids from 256 workgroups to one chunk
// per workgroup.  For each shape it prints the time per launch back to back
// (200 launches between two events) and isolated (an event pair around
// each of 40 launches).  The library's qraf_hip_read_probe_dev uses the
// fastest shape.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1); } } while (0)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int U, int NT, int NTL>
__global__ __launch_bounds__(NT) void rd_stride(const u32x4* __restrict__ p, long n16, unsigned* out) {
    unsigned acc = 0;
    const long step = (long)gridDim.x * NT * U;
    for (long base = (long)blockIdx.x * NT * U + threadIdx.x; base < n16; base += step) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const long i = std::min(base + (long)u * NT, n16 - 1);
            if (NTL) v[u] = __builtin_nontemporal_load(p + i);
            else v[u] = p[i];
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

// each workgroup a contiguous chunk
template <int U, int NT, int NTL>
__global__ __launch_bounds__(NT) void rd_chunk(const u32x4* __restrict__ p, long n16, unsigned* out) {
    unsigned acc = 0;
    const long per = (n16 + gridDim.x - 1) / gridDim.x;
    const long b0 = (long)blockIdx.x * per, b1 = std::min(n16, b0 + per);
    for (long base = b0 + threadIdx.x; base < b1; base += (long)NT * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const long i = std::min(base + (long)u * NT, b1 - 1);
            if (NTL) v[u] = __builtin_nontemporal_load(p + i);
            else v[u] = p[i];
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

typedef void (*KFn)(const u32x4*, long, unsigned*);

int main(int argc, char** argv) {
    const long bytes = argc > 1 ? atol(argv[1]) : 50785280L;
    const int copies = std::max(8L, (320L * 1000 * 1000 + bytes - 1) / bytes);  // together > 320 MB
    const long n16 = bytes / 16;
    const size_t stride = ((size_t)bytes + 4095) / 4096 * 4096;
    char* pool;
    CK(hipMalloc(&pool, stride * copies));
    CK(hipMemset(pool, 1, stride * copies));
    unsigned* out;
    CK(hipMalloc(&out, 1 << 20));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    struct Cfg { const char* name; KFn f; int nt; int u; };
    std::vector<Cfg> cfgs = {
        {"stride U4 NT256", rd_stride<4, 256, 0>, 256, 4},
        {"stride U8 NT256", rd_stride<8, 256, 0>, 256, 8},
        {"stride U16 NT256", rd_stride<16, 256, 0>, 256, 16},
        {"stride U8 NT512", rd_stride<8, 512, 0>, 512, 8},
        {"stride U8 NT1024", rd_stride<8, 1024, 0>, 1024, 8},
        {"stride U8 NT256 nt", rd_stride<8, 256, 1>, 256, 8},
        {"stride U16 NT256 nt", rd_stride<16, 256, 1>, 256, 16},
        {"chunk U8 NT256", rd_chunk<8, 256, 0>, 256, 8},
        {"chunk U16 NT256", rd_chunk<16, 256, 0>, 256, 16},
        {"chunk U8 NT512", rd_chunk<8, 512, 0>, 512, 8},
        {"chunk U8 NT1024", rd_chunk<8, 1024, 0>, 1024, 8},
        {"chunk U16 NT256 nt", rd_chunk<16, 256, 1>, 256, 16},
    };
    printf("bytes %ld\n", bytes);
    for (auto& c : cfgs) {
        const long oneshot = (n16 + (long)c.nt * c.u - 1) / ((long)c.nt * c.u);
        std::vector<long> grids = {256, 512, 1024, 2048, oneshot};
        for (long g : grids) {
            if (g > 65535 * 16) continue;
            const int reps = 200;
            for (int w = 0; w < 16; w++)
                hipLaunchKernelGGL(c.f, dim3(g), dim3(c.nt), 0, 0, (const u32x4*)(pool + stride * (w % copies)), n16, out);
            CK(hipDeviceSynchronize());
            // back-to-back launches
            CK(hipEventRecord(e0, 0));
            for (int r = 0; r < reps; r++)
                hipLaunchKernelGGL(c.f, dim3(g), dim3(c.nt), 0, 0, (const u32x4*)(pool + stride * (r % copies)), n16, out);
            CK(hipEventRecord(e1, 0));
            CK(hipEventSynchronize(e1));
            float ms;
            CK(hipEventElapsedTime(&ms, e0, e1));
            const double us = ms * 1000.0 / reps;
            // isolated launches (event pair around each)
            double iso = 0;
            const int ireps = 40;
            for (int r = 0; r < ireps; r++) {
                CK(hipEventRecord(e0, 0));
                hipLaunchKernelGGL(c.f, dim3(g), dim3(c.nt), 0, 0, (const u32x4*)(pool + stride * (r % copies)), n16, out);
                CK(hipEventRecord(e1, 0));
                CK(hipEventSynchronize(e1));
                float m2;
                CK(hipEventElapsedTime(&m2, e0, e1));
                iso += m2 * 1000.0;
            }
            iso /= ireps;
            printf("%-22s grid %6ld  b2b %7.2f us %7.1f GB/s (%.3f)   isolated %7.2f us %7.1f GB/s\n", c.name, g, us,
                   bytes / us / 1e3, bytes / us / 1e3 / 8000.0, iso, bytes / iso / 1e3);
            fflush(stdout);
        }
    }
    return 0;
}
