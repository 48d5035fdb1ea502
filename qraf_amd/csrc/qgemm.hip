// qgemm.hip -- batched Q8_0 / Q4_0 GEMM on gfx950 matrix cores.
//
// Y[m][n] = sum_k X[m][k] * W[n][k]  (+ add[m][n])  for a continuous-batch
// decode step: the B rows of X are B sequences' activations, W is a weight
// matrix in the reference's Q8_0/Q4_0 block layout (quantize.h:11-30).  The
// reference has no batched product: this is dispatch_matvec_q
// (backend.cpp:131-199) applied to B vectors at once.
//
// Exactness: each quant block is one K=32 step of v_mfma_f32_16x16x32_bf16.
// Weights enter as bf16 copies of the block integers (exact: |q| <= 127), X
// as two bf16 planes hi + lo with x = hi + lo + r, |r| <= 2^-17 |x| (split
// once per activation by split_bf16_kernel).  The two MFMAs of a block
// accumulate sum_k q (x_hi + x_lo) in fp32 (products exact), then the block
// is scaled by its fp32 (Q8) or fp16 (Q4) scale with one FMA per output:
//     |y - y_exact| <= (2^-17 + (K + 2) 2^-24) sum_k |w_k x_k|.
//
// Tiling: a workgroup of 4 waves owns 64 weight rows (16 per wave) and all
// B <= 128 batch rows (8 row tiles of 16).  Per K step the workgroup stages
// X[0:B, 32 k] hi/lo in LDS (rows padded to 80 B: conflict-free ds_read_b128)
// with a double buffer; every wave reads each weight block once, converts it
// to bf16 in registers and reuses it for all batch row tiles.
// MFMA operand layout (16x16x32): lane l supplies row l%16, k = 8*(l/16)..+7
// of A (= X) and of B^T (= W); it receives D[4*(l/16) + r][l%16], r = 0..3,
// i.e. four batch rows of one weight row, so one block scale per lane.
#include "common.h"

namespace qraf_hip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

constexpr int GW = 256;       // threads per workgroup
constexpr int GN = 64;        // weight rows per workgroup
constexpr int GMAX = 128;     // max batch rows
constexpr int XROW = 40;      // LDS row stride in bf16 (80 B)

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// X fp32 [M][K] -> hi, lo bf16 planes [M][K] (hi = rne(x), lo = rne(x - hi)).
// op 0: x as given; op 1: x = silu(g) * u from an interleaved gate/up row
// [M][2K] (g = even columns, u = odd columns), ops.cpp:218-222 then :275-279.
__global__ void split_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                  int M, int K, int op, float* __restrict__ xout) {
    const size_t n = (size_t)M * K;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v;
        if (op == 1) {
            const size_t m = i / K, k = i % K;
            const float g = x[m * 2 * K + 2 * k], u = x[m * 2 * K + 2 * k + 1];
            v = __fmul_rn(g / (1.0f + expf(-g)), u);
            if (xout) xout[i] = v;
        } else {
            v = x[i];
        }
        const uint32_t h = f32_to_bf16_rne(v);
        const float r = v - __builtin_bit_cast(float, h << 16);
        hi[i] = (uint16_t)h;
        lo[i] = (uint16_t)f32_to_bf16_rne(r);
    }
}

// 8 weights of row `rp`, block b, k = 8*seg..+7 as bf16x8, and the block scale
template <int FMT>
__device__ __forceinline__ void load_wblock(const uint8_t* rp, int b, int seg, bf16x8& w, float& scale) {
    if (FMT == 8) {
        const uint8_t* p = rp + (size_t)b * 36;
        scale = __builtin_bit_cast(float, *(const uint32_t*)p);
        const u32x2a4 q = *(const u32x2a4*)(p + 4 + 8 * seg);
        uint32_t f[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t d = j < 4 ? q[0] : q[1];
            f[j] = __builtin_bit_cast(uint32_t, (float)(int8_t)(d >> (8 * (j & 3))));
        }
        u32x4 packed;
#pragma unroll
        for (int j = 0; j < 4; j++) packed[j] = __builtin_amdgcn_perm(f[2 * j + 1], f[2 * j], 0x07060302u);
        w = __builtin_bit_cast(bf16x8, packed);
    } else {
        // Q4 rows are 4-byte aligned but blocks are 18 B, so block fields are
        // only 2-byte aligned: read them with 16-bit loads, never past the block.
        const uint16_t* p = (const uint16_t*)(rp + (size_t)b * 18);
        scale = (float)__builtin_bit_cast(_Float16, p[0]);
        const uint32_t d = (uint32_t)p[1 + 2 * seg] | ((uint32_t)p[2 + 2 * seg] << 16);  // nibble bytes 4seg..4seg+3
        uint32_t f[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t byte = (d >> (8 * j)) & 0xFFu;
            f[2 * j] = __builtin_bit_cast(uint32_t, (float)(int)(byte & 15u) - 8.0f);
            f[2 * j + 1] = __builtin_bit_cast(uint32_t, (float)(int)(byte >> 4) - 8.0f);
        }
        u32x4 packed;
#pragma unroll
        for (int j = 0; j < 4; j++) packed[j] = __builtin_amdgcn_perm(f[2 * j + 1], f[2 * j], 0x07060302u);
        w = __builtin_bit_cast(bf16x8, packed);
    }
}

// MT: number of 16-row batch tiles (1..8)
template <int FMT, int MT>
__global__ __launch_bounds__(GW) void qgemm_kernel(const uint8_t* __restrict__ W, size_t row_bytes, int N, int K,
                                                  const uint16_t* __restrict__ xh, const uint16_t* __restrict__ xl,
                                                  int M, float* __restrict__ Y, const float* __restrict__ add) {
    __shared__ __align__(16) uint16_t sx[2][2][GMAX * XROW];  // [buffer][hi/lo][row * XROW + k]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * GN + wave * 16;
    const int wr = min(n0 + (lane & 15), N - 1);  // weight row of this lane (clamped)
    const int seg = lane >> 4;
    const uint8_t* rp = W + (size_t)wr * row_bytes;
    const int nb = K / 32;
    const int Mp = MT * 16;

    // stage X[:, 32b..32b+31] (hi and lo) into buffer `buf`: 2*Mp rows of 64 B
    auto stage = [&](int buf, int b) {
        for (int i = tid; i < Mp * 2 * 4; i += GW) {  // 16-byte pieces: row, plane, quarter
            const int q = i & 3, plane = (i >> 2) & 1, m = i >> 3;
            u32x4 v = {0, 0, 0, 0};
            if (m < M) {
                const uint16_t* src = (plane ? xl : xh) + (size_t)m * K + 32 * b + 8 * q;
                v = *(const u32x4*)src;
            }
            *(u32x4*)&sx[buf][plane][m * XROW + 8 * q] = v;
        }
    };

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    bf16x8 wcur;
    float scur;
    load_wblock<FMT>(rp, 0, seg, wcur, scur);
    stage(0, 0);
    __syncthreads();
    for (int b = 0; b < nb; b++) {
        const int buf = b & 1;
        bf16x8 wnext;
        float snext;
        if (b + 1 < nb) {
            load_wblock<FMT>(rp, b + 1, seg, wnext, snext);
            stage(buf ^ 1, b + 1);
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int row = t * 16 + (lane & 15);
            const bf16x8 ah = *(const bf16x8*)&sx[buf][0][row * XROW + 8 * seg];
            const bf16x8 al = *(const bf16x8*)&sx[buf][1][row * XROW + 8 * seg];
            f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wcur, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, wcur, c, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[t][r] = __builtin_fmaf(c[r], scur, acc[t][r]);
        }
        __syncthreads();
        if (b + 1 < nb) {
            wcur = wnext;
            scur = snext;
        }
    }

    const int n = n0 + (lane & 15);
    if (n < N) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = t * 16 + 4 * seg + r;
                if (m < M) {
                    float v = acc[t][r];
                    if (add) v += add[(size_t)m * N + n];
                    Y[(size_t)m * N + n] = v;
                }
            }
        }
    }
}

int launch_split_bf16(const float* x, uint16_t* hi, uint16_t* lo, int M, int K, int op, float* xout, hipStream_t s) {
    QH_REQUIRE(x && hi && lo && M > 0 && K > 0, QRAF_HIP_ERR_INVALID, "split: bad arguments");
    const size_t n = (size_t)M * K;
    const int grid = (int)min((n + 255) / 256, (size_t)4096);
    hipLaunchKernelGGL(split_bf16_kernel, dim3(grid), dim3(256), 0, s, x, hi, lo, M, K, op, xout);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_qgemm(const void* W, uint32_t dtype, int bs, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                 float* Y, const float* add, hipStream_t s) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "qgemm: unsupported dtype %u", dtype);
    QH_REQUIRE(bs == 32, QRAF_HIP_ERR_DTYPE, "qgemm: block size %d (32 required)", bs);
    QH_REQUIRE(K % 32 == 0 && K > 0 && N > 0, QRAF_HIP_ERR_INVALID, "qgemm: K=%d must be a positive multiple of 32", K);
    QH_REQUIRE(M > 0 && M <= GMAX, QRAF_HIP_ERR_INVALID, "qgemm: batch %d outside 1..%d", M, GMAX);
    QH_REQUIRE(W && xh && xl && Y, QRAF_HIP_ERR_INVALID, "qgemm: null pointer");
    // Q8 blocks are read with 4-byte loads (36-byte blocks keep rows 4-aligned),
    // Q4 blocks with 2-byte loads (18-byte blocks)
    QH_REQUIRE((((uintptr_t)W) & (dtype == DT_Q8_0 ? 3 : 1)) == 0 && (((uintptr_t)xh) & 15) == 0 &&
                   (((uintptr_t)xl) & 15) == 0,
               QRAF_HIP_ERR_INVALID, "qgemm: misaligned operands");
    const size_t rb = q_row_bytes(dtype, bs, K);
    const int MT = (M + 15) / 16;
    dim3 grid((N + GN - 1) / GN);
#define QH_G(F, T)                                                                                          \
    case T:                                                                                                 \
        hipLaunchKernelGGL((qgemm_kernel<F, T>), grid, dim3(GW), 0, s, (const uint8_t*)W, rb, N, K, xh, xl, M, \
                           Y, add);                                                                         \
        break;
    if (dtype == DT_Q8_0) {
        switch (MT) { QH_G(8, 1) QH_G(8, 2) QH_G(8, 3) QH_G(8, 4) QH_G(8, 5) QH_G(8, 6) QH_G(8, 7) QH_G(8, 8) }
    } else {
        switch (MT) { QH_G(4, 1) QH_G(4, 2) QH_G(4, 3) QH_G(4, 4) QH_G(4, 5) QH_G(4, 6) QH_G(4, 7) QH_G(4, 8) }
    }
#undef QH_G
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip

extern "C" {

int qraf_hip_split_bf16_dev(const float* x, uint16_t* x_hi, uint16_t* x_lo, int32_t rows, int32_t cols, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_split_bf16(x, x_hi, x_lo, rows, cols, 0, nullptr, qraf_hip::as_stream(stream));
}

int qraf_hip_qgemm_dev(const void* w, uint32_t dtype, uint32_t block_size, uint32_t out_dim, uint32_t in_dim,
                       const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, float* y, const float* add,
                       void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_qgemm(w, dtype, block_size ? (int)block_size : 32, (int)out_dim, (int)in_dim, x_hi, x_lo,
                                  batch, y, add, qraf_hip::as_stream(stream));
}

}  // extern "C"
