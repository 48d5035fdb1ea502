// qmatvec.hip -- Q8_0 / Q4_0 block-dequant matvec for gfx950 (batch 1).
//
// Replaces the row loop of dispatch_matvec_q (reference backend.cpp:131-199)
// and the per-row dot products dot_q8_0_f32 / dot_q4_0_f32
// (reference quantize.cpp:187-239).  Weights are read in the reference's own
// block layout, straight from HBM:
//   Q8_0 block (36 B) = [f32 scale][32 x int8]
//   Q4_0 block (18 B) = [f16 scale][16 B: byte j = elem 2j (low nibble),
//                                          elem 2j+1 (high nibble)], value = nibble - 8
// The fast kernel works on 36-byte "units": one Q8_0 block or a pair of Q4_0
// blocks.  Lane l of a wave owns units l, l+64, ... of every row it visits
// and loads each unit with one dword + two dwordx4 loads (4-byte aligned),
// so a wave reads 2304 contiguous bytes per row step.  The activation vector
// is staged once per workgroup in LDS, padded to 36 floats per 32-element
// block (16-byte aligned, free of bank conflicts for ds_read_b128), and for
// Q4 permuted inside each 8-element group to match the even/odd nibble split.
// Dequantisation happens in registers: v_cvt_f32_i32 with an SDWA byte select
// for Q8, v_cvt_f32_ubyteN of a 0x0F0F0F0F-masked dword for Q4 (the -8 offset
// is applied once per block through the staged block sum).  Accumulation is
// fp32; each wave reduces its R rows with a transposing butterfly.
#include "common.h"

namespace qraf_hip {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int XS8 = 36;  // staged floats per Q8 block  (32 + pad)
constexpr int XS4 = 76;  // staged floats per Q4 block pair (2 x (32 + sum + pad) + pad)
constexpr int WG = 256;  // 4 waves

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// Q4 staging position of element e (0..31) of a block: inside each group of 8,
// even elements first, then odd ones.
__device__ __forceinline__ int q4_slot(int e) {
    int g = e >> 3, o = e & 7;
    return g * 8 + ((o & 1) ? 4 + (o >> 1) : (o >> 1));
}

// Sum over the 64 lanes for each of R accumulators.  On return lanes with
// (lane & (64/R - 1)) == 0 hold the total of row `*row` in acc[0].
template <int R>
__device__ __forceinline__ float wave_reduce_rows(float (&acc)[R], int lane, int* row) {
    int r = 0;
    int m = 32;
#pragma unroll
    for (int c = R; c > 1; c >>= 1, m >>= 1) {
        const bool up = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < c / 2; i++) {
            float send = up ? acc[i] : acc[i + c / 2];
            float keep = up ? acc[i + c / 2] : acc[i];
            acc[i] = keep + __shfl_xor(send, m);
        }
        r = r * 2 + (up ? 1 : 0);
    }
    float v = acc[0];
#pragma unroll
    for (; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    *row = r;
    return v;
}

// ----------------------------------------------------------------------------
// Fast path: block_size 32, 4-byte aligned rows, staged x fits in LDS.
// ----------------------------------------------------------------------------
template <int R>
__global__ __launch_bounds__(WG) void qmv_q8_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes,
                                                   int N, int K, int nb, const float* __restrict__ x,
                                                   float* __restrict__ y) {
    extern __shared__ __align__(16) float sx[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * R;

    for (int i = threadIdx.x; i < nb * 32; i += WG) sx[(i >> 5) * XS8 + (i & 31)] = (i < K) ? x[i] : 0.f;
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

    const uint8_t* rowp[R];
#pragma unroll
    for (int r = 0; r < R; r++) rowp[r] = W + (size_t)min(row0 + r, N - 1) * row_bytes;

    for (int u = lane; u < nb; u += 64) {
        uint32_t s[R];
        u32x4a4 a[R], b[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t* p = rowp[r] + (size_t)u * 36;
            s[r] = *(const uint32_t*)p;
            a[r] = *(const u32x4a4*)(p + 4);
            b[r] = *(const u32x4a4*)(p + 20);
        }
        const f32x4* xv = (const f32x4*)(sx + u * XS8);
        f32x4 xr[8];
#pragma unroll
        for (int j = 0; j < 8; j++) xr[j] = xv[j];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float bs = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint32_t d = j < 4 ? a[r][j] : b[r][j - 4];
#pragma unroll
                for (int k = 0; k < 4; k++) bs = __builtin_fmaf((float)(int8_t)(d >> (8 * k)), xr[j][k], bs);
            }
            acc[r] = __builtin_fmaf(bs, __builtin_bit_cast(float, s[r]), acc[r]);
        }
    }
    int rr;
    float v = wave_reduce_rows<R>(acc, lane, &rr);
    if ((lane & (64 / R - 1)) == 0 && row0 + rr < N) y[row0 + rr] = v;
}

template <int R>
__global__ __launch_bounds__(WG) void qmv_q4_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes,
                                                   int N, int K, int nb, const float* __restrict__ x,
                                                   float* __restrict__ y) {
    extern __shared__ __align__(16) float sx[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    const int U = nb >> 1;
    // The reference drops the last element of an odd-length final block
    // (quantize.cpp:227 iterates this_block/2 pairs): stage it as zero.
    const int Keff = K & ~1;

    for (int i = threadIdx.x; i < nb * 32; i += WG) {
        int blk = i >> 5;
        sx[(blk >> 1) * XS4 + (blk & 1) * 36 + q4_slot(i & 31)] = (i < Keff) ? x[i] : 0.f;
    }
    __syncthreads();
    for (int blk = threadIdx.x; blk < nb; blk += WG) {
        const float* p = sx + (blk >> 1) * XS4 + (blk & 1) * 36;
        float t = 0.f;
        for (int e = 0; e < 32; e++) t += p[e];
        sx[(blk >> 1) * XS4 + (blk & 1) * 36 + 32] = t;
    }
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    const uint8_t* rowp[R];
#pragma unroll
    for (int r = 0; r < R; r++) rowp[r] = W + (size_t)min(row0 + r, N - 1) * row_bytes;

    for (int u = lane; u < U; u += 64) {
        uint32_t d0[R];
        u32x4a4 a[R], b[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t* p = rowp[r] + (size_t)u * 36;
            d0[r] = *(const uint32_t*)p;
            a[r] = *(const u32x4a4*)(p + 4);
            b[r] = *(const u32x4a4*)(p + 20);
        }
        const float* xu = sx + u * XS4;
        f32x4 xe[8], xo[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            xe[j] = ((const f32x4*)xu)[j];
            xo[j] = ((const f32x4*)(xu + 36))[j];
        }
        const float se8 = 8.f * xu[32], so8 = 8.f * xu[36 + 32];
#pragma unroll
        for (int r = 0; r < R; r++) {
            // a = dwords 1..4, b = dwords 5..8 of the unit
            uint32_t dw[9] = {d0[r], a[r][0], a[r][1], a[r][2], a[r][3], b[r][0], b[r][1], b[r][2], b[r][3]};
            float be = 0.f, bo = 0.f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint32_t ne = __builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2);  // even block bytes 4k..4k+3
                uint32_t no = dw[5 + k];                                         // odd block bytes 4k..4k+3
                uint32_t elo = ne & 0x0F0F0F0Fu, ehi = (ne >> 4) & 0x0F0F0F0Fu;
                uint32_t olo = no & 0x0F0F0F0Fu, ohi = (no >> 4) & 0x0F0F0F0Fu;
                asm volatile("" : "+v"(elo), "+v"(ehi), "+v"(olo), "+v"(ohi));
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    be = __builtin_fmaf((float)((elo >> (8 * q)) & 0xFFu), xe[2 * k][q], be);
                    be = __builtin_fmaf((float)((ehi >> (8 * q)) & 0xFFu), xe[2 * k + 1][q], be);
                    bo = __builtin_fmaf((float)((olo >> (8 * q)) & 0xFFu), xo[2 * k][q], bo);
                    bo = __builtin_fmaf((float)((ohi >> (8 * q)) & 0xFFu), xo[2 * k + 1][q], bo);
                }
            }
            float se = half_bits_to_float(dw[0]), so = half_bits_to_float(dw[4] >> 16);
            acc[r] = __builtin_fmaf(be - se8, se, acc[r]);
            acc[r] = __builtin_fmaf(bo - so8, so, acc[r]);
        }
    }
    int rr;
    float v = wave_reduce_rows<R>(acc, lane, &rr);
    if ((lane & (64 / R - 1)) == 0 && row0 + rr < N) y[row0 + rr] = v;
}

// ----------------------------------------------------------------------------
// General path: any block size, any alignment (byte loads).  One wave per row;
// lane l takes blocks l, l+64, ...  Follows the reference's block geometry
// exactly, including the Q4 odd-tail rule (this_block/2 pairs).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(WG) void qmv_generic_kernel(const uint8_t* __restrict__ W, uint32_t dtype,
                                                        int bs, size_t row_bytes, int N, int K,
                                                        const float* __restrict__ x, float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nb = (K + bs - 1) / bs;
    const size_t bb = q_block_bytes(dtype, bs);
    const uint8_t* rp = W + (size_t)row * row_bytes;
    float part = 0.f;
    for (int b = lane; b < nb; b += 64) {
        const uint8_t* p = rp + (size_t)b * bb;
        const int off = b * bs, tb = min(bs, K - off);
        float bsum = 0.f, scale;
        if (dtype == DT_Q8_0) {
            uint32_t sb = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
            scale = __builtin_bit_cast(float, sb);
            for (int i = 0; i < tb; i++) bsum = __builtin_fmaf((float)(int8_t)p[4 + i], x[off + i], bsum);
        } else {
            scale = half_bits_to_float((uint32_t)p[0] | ((uint32_t)p[1] << 8));
            for (int i = 0; i < tb / 2; i++) {
                uint8_t v = p[2 + i];
                bsum = __builtin_fmaf((float)((v & 0x0F) - 8), x[off + 2 * i], bsum);
                bsum = __builtin_fmaf((float)(((v >> 4) & 0x0F) - 8), x[off + 2 * i + 1], bsum);
            }
        }
        part = __builtin_fmaf(bsum, scale, part);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m);
    if (lane == 0) y[row] = part;
}

// f32 weights (reference dispatch_matvec_opt, backend.cpp:62-105; used for F32
// projection weights and the tied f32 lm_head).  One wave per row, float4 loads.
__global__ __launch_bounds__(WG) void mv_f32_kernel(const float* __restrict__ W, const float* __restrict__ x,
                                                   float* __restrict__ y, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const float* rp = W + (size_t)row * K;
    float part = 0.f;
    if ((K & 3) == 0 && (((uintptr_t)W) & 15) == 0) {
        for (int i = lane * 4; i < K; i += 256) {
            f32x4 w = *(const f32x4*)(rp + i);
            f32x4 v = *(const f32x4*)(x + i);
            part = __builtin_fmaf(w[0], v[0], part);
            part = __builtin_fmaf(w[1], v[1], part);
            part = __builtin_fmaf(w[2], v[2], part);
            part = __builtin_fmaf(w[3], v[3], part);
        }
    } else {
        for (int i = lane; i < K; i += 64) part = __builtin_fmaf(rp[i], x[i], part);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m);
    if (lane == 0) y[row] = part;
}

// ----------------------------------------------------------------------------
// Launchers
// ----------------------------------------------------------------------------
static int g_rows_per_wave = 4;  // tunable: 1, 2, 4 or 8

int set_matvec_rows_per_wave(int r) {
    QH_REQUIRE(r == 1 || r == 2 || r == 4 || r == 8, QRAF_HIP_ERR_INVALID, "rows per wave must be 1, 2, 4 or 8");
    g_rows_per_wave = r;
    return QRAF_HIP_OK;
}

template <int R>
static int launch_fast(uint32_t dtype, const uint8_t* W, size_t rb, int N, int K, int nb, const float* x, float* y,
                       size_t lds, hipStream_t s) {
    dim3 grid((N + 4 * R - 1) / (4 * R));
    if (dtype == DT_Q8_0) {
        if (lds > 65536) QH_CHECK_HIP(hipFuncSetAttribute((const void*)qmv_q8_kernel<R>,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(qmv_q8_kernel<R>, grid, dim3(WG), lds, s, W, (uint32_t)rb, N, K, nb, x, y);
    } else {
        if (lds > 65536) QH_CHECK_HIP(hipFuncSetAttribute((const void*)qmv_q4_kernel<R>,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(qmv_q4_kernel<R>, grid, dim3(WG), lds, s, W, (uint32_t)rb, N, K, nb, x, y);
    }
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_matvec_q(const void* Wv, uint32_t dtype, int bs, uint32_t N, uint32_t K, const float* x, float* y,
                    hipStream_t s) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "unsupported weight dtype %u", dtype);
    QH_REQUIRE(bs > 0 && bs <= 4096, QRAF_HIP_ERR_INVALID, "bad block size %d", bs);
    QH_REQUIRE(K > 0 && N > 0, QRAF_HIP_ERR_INVALID, "empty matvec (%u x %u)", N, K);
    QH_REQUIRE(Wv && x && y, QRAF_HIP_ERR_INVALID, "null pointer");
    const uint8_t* W = (const uint8_t*)Wv;
    const size_t rb = q_row_bytes(dtype, bs, K);
    const int nb = (int)((K + bs - 1) / bs);
    const size_t lds = dtype == DT_Q8_0 ? (size_t)nb * XS8 * 4 : (size_t)(nb / 2) * XS4 * 4;
    const bool fast = bs == 32 && (((uintptr_t)W) & 3) == 0 && (dtype == DT_Q8_0 || (nb % 2) == 0) &&
                      lds <= 160 * 1024 && rb <= 0xFFFFFFFFu;
    if (fast) {
        switch (g_rows_per_wave) {
            case 1: return launch_fast<1>(dtype, W, rb, (int)N, (int)K, nb, x, y, lds, s);
            case 2: return launch_fast<2>(dtype, W, rb, (int)N, (int)K, nb, x, y, lds, s);
            case 8: return launch_fast<8>(dtype, W, rb, (int)N, (int)K, nb, x, y, lds, s);
            default: return launch_fast<4>(dtype, W, rb, (int)N, (int)K, nb, x, y, lds, s);
        }
    }
    hipLaunchKernelGGL(qmv_generic_kernel, dim3((N + 3) / 4), dim3(WG), 0, s, W, dtype, bs, rb, (int)N, (int)K, x, y);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_matvec_f32(const float* W, const float* x, float* y, uint32_t N, uint32_t K, hipStream_t s) {
    QH_REQUIRE(W && x && y && N > 0 && K > 0, QRAF_HIP_ERR_INVALID, "bad f32 matvec arguments");
    hipLaunchKernelGGL(mv_f32_kernel, dim3((N + 3) / 4), dim3(WG), 0, s, W, x, y, (int)N, (int)K);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip
