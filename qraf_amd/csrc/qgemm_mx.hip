// qgemm_mx.hip -- batched Q8_0 / Q4_0 GEMM for large batches (the 128-row
// continuous-batch step and prefill chunks) on an MFMA-ready weight copy.
//
// Y[m][n] = sum_k X[m][k] W[n][k] for M activation rows, the reference's
// dispatch_matvec_q (backend.cpp:131-199) applied to M vectors at once, with
// the arithmetic of qgemm.hip: per quant block two matrix-core products,
// v_mfma_f32_16x16x32_bf16 on the hi plane of X and _f16 on the lo plane,
// against the block's exact integer weights, then one FMA per output with the
// block scale (error bound in include/qraf_hip.h, qraf_hip_qgemm_dev).
//
// At 128 rows this product is bound by the matrix cores, not by HBM: the two
// MFMAs per block cost 2 x 2 M N K flops against N K / 2 bytes of Q4 weights.
// So the weights are repacked once into a form that costs the fewest VALU
// operations per MFMA ("mx" form), even though it has twice the bytes of Q4:
//   per quant block b and 16-row tile t, 576 bytes at (b * tiles + t) * 576
//   (block-major: the tiles a workgroup reads for one block are one run):
//     [0, 64)    the 16 rows' block scales as fp32 (Q4's fp16 scale widened, exact)
//     [64, 576)  the 16 rows' 32 values, 8 bytes per (k segment s, row r) at
//                64 + (16 s + r) * 8, byte v = element k = 8 s + v:
//                Q8: the int8 quant; Q4: fp8 e4m3 of (nibble - 8) (integers
//                -8..7 are exact in fp8), written by the hardware encoder.
// Lane l of an MFMA reads its B operand (row l % 16, k = 8 (l / 16) .. +7) as
// one 8-byte load; Q4 values become bf16 and fp16 by v_cvt_scalef32_pk_*_fp8
// (4 instructions each for 8 values), Q8 values fp16 by the exponent-bias
// trick and bf16 through fp32.
//
// Workgroup: WMG x 4 waves, 4 side by side along N (TN 16-row weight tiles
// each) and WMG along M (64 batch rows each): MW = 64 WMG batch rows x
// NW = 64 TN weight rows.  X (both planes) is staged one quant block at a
// time in a double-buffered LDS stage, [plane][row][4 pieces of 16 bytes],
// the pieces of row r stored in slot piece ^ f(r), f(r) = ((r >> 1) ^ (r >> 3))
// & 3, so that the MFMA operand reads of 16 rows hit distinct banks.  The
// weights do not pass through LDS: no two waves share a weight tile, so each
// lane loads its own fragments (8 values and the row's scale per tile and
// block) into registers.  All loads are ordinary 16/8/4-byte global loads
// issued three blocks ahead (the direct-to-LDS load path moves only about 8
// bytes per cycle per CU on this part, a third of what the matrix cores
// consume here, and weight fragments through LDS would leave the X reads
// short of LDS bandwidth).
// Split-K over blockIdx.y writes fp32 partial slices [S][M][N] that the
// consumer sums in slice order (deterministic); with one split the epilogue
// writes Y (+ residual), or, for the interleaved gate/up projection,
// silu(gate) * up straight into the down projection's hi/lo planes.
#include <type_traits>

#include "common.h"

namespace qraf_hip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

constexpr int MX_TB = 576;  // bytes per (16-row tile, quant block)

// four values -> four fp8 bytes (element i in byte i), by the hardware encoder
__device__ __forceinline__ uint32_t fp8x4(float a, float b, float c, float d) {
    s16x2 w = {0, 0};
    w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, a, b, 1.0f, false);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, c, d, 1.0f, true);
    return __builtin_bit_cast(uint32_t, w);
}

// reference row-major blocks -> mx form; thread per (tile, block, row); rows past N are zero
template <int FMT>
__global__ void repack_mx_kernel(const uint8_t* __restrict__ src, int N, int nb, uint8_t* __restrict__ dst) {
    constexpr int BB = FMT == 8 ? 36 : 18;
    const size_t rb = (size_t)nb * BB;
    const size_t nt = (size_t)(N + 15) / 16;
    const size_t total = nt * nb * 16;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i & 15);
        const size_t bt = i >> 4;  // block * tiles + tile
        const size_t b = bt / nt, t = bt % nt;
        const size_t row = t * 16 + r;
        uint8_t* d = dst + bt * MX_TB;
        float scale = 0.f;
        uint32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = 0;
        if (row < (size_t)N) {
            const uint8_t* sp = src + row * rb + b * BB;
            if (FMT == 8) {  // 36-byte blocks of 4-byte-aligned rows
                scale = __builtin_bit_cast(float, *(const uint32_t*)sp);
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = *(const uint32_t*)(sp + 4 + 4 * j);
            } else {  // 18-byte blocks: 16-bit fields
                scale = (float)__builtin_bit_cast(_Float16, *(const uint16_t*)sp);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t q = *(const uint16_t*)(sp + 2 + 2 * j);  // elements 4j .. 4j+3
                    v[j] = fp8x4((float)((int)(q & 15) - 8), (float)((int)((q >> 4) & 15) - 8),
                                 (float)((int)((q >> 8) & 15) - 8), (float)((int)((q >> 12) & 15) - 8));
                }
            }
        }
        ((float*)d)[r] = scale;
#pragma unroll
        for (int s = 0; s < 4; s++) *(uint2*)(d + 64 + (16 * s + r) * 8) = make_uint2(v[2 * s], v[2 * s + 1]);
    }
}

// One lane's B operands (bf16 for the hi plane, fp16 for the lo plane) from
// its 8 stored values.
template <int FMT>
__device__ __forceinline__ void mx_convert(uint2 q, bf16x8& wb, f16x8& wh);
template <>
__device__ __forceinline__ void mx_convert<4>(uint2 q, bf16x8& wb, f16x8& wh) {
    const f16x2 h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q.x, 1.0f, false);
    const f16x2 h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q.x, 1.0f, true);
    const f16x2 h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q.y, 1.0f, false);
    const f16x2 h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q.y, 1.0f, true);
    const bf16x2 b0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.x, 1.0f, false);
    const bf16x2 b1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.x, 1.0f, true);
    const bf16x2 b2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.y, 1.0f, false);
    const bf16x2 b3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q.y, 1.0f, true);
    wh = __builtin_bit_cast(f16x8, u32x4{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                                         __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3)});
    wb = __builtin_bit_cast(bf16x8, u32x4{__builtin_bit_cast(uint32_t, b0), __builtin_bit_cast(uint32_t, b1),
                                          __builtin_bit_cast(uint32_t, b2), __builtin_bit_cast(uint32_t, b3)});
}
// 4 int8 (byte i = element i) -> 4 fp16, exactly: the biased byte u = q + 128
// goes under the exponent of 1024 (fp16 0x6400 | u = 1024 + u), then 1152 is
// subtracted
__device__ __forceinline__ void i8x4_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const f16x2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(uint32_t,
                            __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - off);
    hi = __builtin_bit_cast(uint32_t,
                            __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - off);
}
// bf16 pair of two exact small integers held as fp16 (the high halves of their fp32 values)
__device__ __forceinline__ uint32_t bf16_pair_of_f16(uint32_t h2) {
    const f16x2 h = __builtin_bit_cast(f16x2, h2);
    const float a = (float)h[0], b = (float)h[1];
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, a), 0x07060302u);
}
template <>
__device__ __forceinline__ void mx_convert<8>(uint2 q, bf16x8& wb, f16x8& wh) {
    uint32_t h[4];
    i8x4_f16(q.x, h[0], h[1]);
    i8x4_f16(q.y, h[2], h[3]);
    wh = __builtin_bit_cast(f16x8, u32x4{h[0], h[1], h[2], h[3]});
    wb = __builtin_bit_cast(bf16x8, u32x4{bf16_pair_of_f16(h[0]), bf16_pair_of_f16(h[1]), bf16_pair_of_f16(h[2]),
                                          bf16_pair_of_f16(h[3])});
}

template <int WMG, int TN>
struct MxGeom {
    static constexpr int TMW = 4;                       // 16-row batch tiles per wave
    static constexpr int NWAVE = 4 * WMG, NTHR = 64 * NWAVE;
    static constexpr int MW = 16 * TMW * WMG;           // batch rows per workgroup
    static constexpr int NT = 4 * TN;                   // weight tiles per workgroup
    static constexpr int NW = 16 * NT;                  // weight rows per workgroup
    static constexpr int XB = MW * 128;                 // X bytes per block: 2 planes x MW rows x 4 pieces of 16 B
    static constexpr int D = 3;                         // blocks in flight in registers
    static_assert(2 * XB <= 64 * 1024, "stage shape");
    static_assert(MW * 4 == NTHR, "one X piece per plane and thread");
};

// EPI 0: Y (+ add) or partial slices; EPI 1: silu(gate) * up of interleaved
// gate/up rows into hi/lo planes oh/ol [M][N/2] (one split)
template <int FMT, int WMG, int TN, int EPI>
__global__ __launch_bounds__(256 * WMG, 2 / WMG) void qgemm_mx_kernel(const uint8_t* __restrict__ Wmx, int N, int nb,
                                                                     const uint16_t* __restrict__ xh,
                                                                     const uint16_t* __restrict__ xl, int K, int M,
                                                                     float* Y, const float* add, int bps,
                                                                     float* __restrict__ part, uint16_t* __restrict__ oh,
                                                                     uint16_t* __restrict__ ol) {
    using G = MxGeom<WMG, TN>;
    constexpr int TMW = G::TMW, D = G::D;
    __shared__ __align__(16) uint8_t mx_lds[2 * G::XB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 3, wm = wave >> 2;
    const int seg = lane >> 4, l16 = lane & 15;
    const int m0 = blockIdx.z * G::MW;
    const int ntile16 = (N + 15) / 16;
    const int tile0 = blockIdx.x * G::NT + wn * TN;  // first 16-row weight tile of this wave
    const int b_begin = blockIdx.y * bps;
    const int b_end = min(nb, b_begin + bps);
    const int nst = b_end - b_begin;  // blocks of this split, uniform

    // ---- X staging: thread tid holds the X piece of plane 0 and plane 1 at
    // LDS row tid / 4, slot tid % 4 (piece slot ^ f(row) of the row's block).
    // ---- W: each wave loads its own TN tiles' fragments (lane: the 8 values
    // of row l16, k = 8 seg .. + 7, and that row's scale) straight into
    // registers; nothing shares them.  Every load is issued unconditionally,
    // its block clamped into the split and its tile into the matrix: with no
    // branch around them the compiler's waits count exactly the loads a use
    // needs, and blocks D ahead stay in flight.
    const int xrow = tid >> 2, xslot = tid & 3;
    const int xpiece = xslot ^ (((xrow >> 1) ^ (xrow >> 3)) & 3);
    const size_t xoff = ((size_t)min(m0 + xrow, M - 1) * K + xpiece * 8) * 2;
    const uint8_t* xsrc0 = (const uint8_t*)xh + xoff;
    const uint8_t* xsrc1 = (const uint8_t*)xl + xoff;
    const uint8_t* wv[TN];  // this lane's value bytes in block 0 of tile u
    const uint8_t* ws[TN];  // its scale
#pragma unroll
    for (int u = 0; u < TN; u++) {
        const size_t t = (size_t)min(tile0 + u, ntile16 - 1);
        wv[u] = Wmx + t * MX_TB + 64 + 8 * lane;
        ws[u] = Wmx + t * MX_TB + 4 * l16;
    }
    const size_t wstride = (size_t)ntile16 * MX_TB;  // bytes from one block's tiles to the next
    u32x4 rx[D][2];
    uint2 rwv[D][TN];
    float rws[D][TN];
    auto load = [&](int c, auto slot) {  // block c of the split (clamped) into register slot
        constexpr int sl = decltype(slot)::value;
        const size_t cb = (size_t)min(b_begin + c, b_end - 1);
        rx[sl][0] = *(const u32x4*)(xsrc0 + cb * 64);
        rx[sl][1] = *(const u32x4*)(xsrc1 + cb * 64);
#pragma unroll
        for (int u = 0; u < TN; u++) {
            rwv[sl][u] = *(const uint2*)(wv[u] + cb * wstride);
            rws[sl][u] = *(const float*)(ws[u] + cb * wstride);
        }
    };
    auto store_x = [&](auto slot, int buf) {  // X pieces of register slot into LDS buffer buf
        constexpr int sl = decltype(slot)::value;
        uint8_t* base = mx_lds + buf * G::XB;
        *(u32x4*)(base + tid * 16) = rx[sl][0];
        *(u32x4*)(base + G::MW * 64 + tid * 16) = rx[sl][1];
    };

    f32x4 acc[TMW][TN];
#pragma unroll
    for (int t = 0; t < TMW; t++)
#pragma unroll
        for (int u = 0; u < TN; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

    // One block: the wave's weight fragments are converted from registers and
    // its X fragments read from LDS; per batch tile the TN bf16 (hi plane)
    // products are issued, then the TN fp16 (lo plane) products accumulating
    // on them, then the scale FMAs of the previous batch tile, whose products
    // are complete by then: the matrix pipe does not wait on its own results
    // and the VALU work runs under it.
    auto compute = [&](const uint8_t* xb, const bf16x8 (&wb)[TN], const f16x8 (&wh)[TN], const float (&sc)[TN]) {
        bf16x8 ah[TMW];
        f16x8 al[TMW];
#pragma unroll
        for (int t = 0; t < TMW; t++) {
            const int row = (wm * TMW + t) * 16 + l16;
            const int slot = seg ^ (((row >> 1) ^ (row >> 3)) & 3);
            ah[t] = *(const bf16x8*)(xb + row * 64 + slot * 16);
            al[t] = *(const f16x8*)(xb + G::MW * 64 + row * 64 + slot * 16);
        }
        f32x4 P[2][TN];
#pragma unroll
        for (int t = 0; t <= TMW; t++) {
            if (t < TMW) {
#pragma unroll
                for (int u = 0; u < TN; u++)
                    P[t & 1][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[t], wb[u], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                                          0);
#pragma unroll
                for (int u = 0; u < TN; u++)
                    P[t & 1][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t], wh[u], P[t & 1][u], 0, 0, 0);
            }
            if (t >= 1) {
#pragma unroll
                for (int u = 0; u < TN; u++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[t - 1][u][r] = __builtin_fmaf(P[(t - 1) & 1][u][r], sc[u], acc[t - 1][u][r]);
            }
        }
    };

    // Pipeline: blocks c+1 .. c+D-1 sit in registers while block c is
    // computed; each step converts block c's weights out of their registers,
    // issues block c+D's loads into them, computes block c from LDS, stores
    // block c+1's X into the other LDS buffer (its loads were issued D-1 steps
    // earlier) and meets the other waves.  Steps past the split compute nothing.
    load(0, std::integral_constant<int, 0>{});
    load(1, std::integral_constant<int, 1>{});
    load(2, std::integral_constant<int, 2>{});
    store_x(std::integral_constant<int, 0>{}, 0);
    __syncthreads();
    auto step = [&](int c, auto slot) {
        constexpr int sl = decltype(slot)::value;
        bf16x8 wb[TN];
        f16x8 wh[TN];
        float sc[TN];
#pragma unroll
        for (int u = 0; u < TN; u++) {
            mx_convert<FMT>(rwv[sl][u], wb[u], wh[u]);
            sc[u] = rws[sl][u];
        }
        load(c + D, slot);  // slot sl held block c, whose X is in LDS and weights converted
        if (c < nst) compute(mx_lds + (c & 1) * G::XB, wb, wh, sc);
        store_x(std::integral_constant<int, (sl + 1) % D>{}, (c + 1) & 1);
        __syncthreads();
    };
    for (int c = 0; c < nst; c += D) {
        step(c, std::integral_constant<int, 0>{});
        step(c + 1, std::integral_constant<int, 1>{});
        step(c + 2, std::integral_constant<int, 2>{});
    }

    // ---- epilogue.  Lane (l16, seg) holds rows m = m0 + 16 (wm TMW + t) + 4 seg + r of weight row
    // n = 16 (tile0 + u) + l16.
    if (EPI == 1) {
        const int F = N / 2;
#pragma unroll
        for (int t = 0; t < TMW; t++)
#pragma unroll
            for (int u = 0; u < TN; u++) {
                const int n = (tile0 + u) * 16 + l16;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float v = acc[t][u][r];
                    const float up = __shfl_xor(v, 1);  // the odd partner row (up) of an even (gate) row
                    const int m = m0 + (wm * TMW + t) * 16 + seg * 4 + r;
                    if ((l16 & 1) == 0 && m < M && n < N) {
                        const size_t e = (size_t)m * F + (n >> 1);
                        split_bf16(silu_gate(v, up), &oh[e], &ol[e]);
                    }
                }
            }
        return;
    }
    float* dst = part ? part + (size_t)blockIdx.y * M * N : Y;
#pragma unroll
    for (int t = 0; t < TMW; t++)
#pragma unroll
        for (int u = 0; u < TN; u++) {
            const int n = (tile0 + u) * 16 + l16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + (wm * TMW + t) * 16 + seg * 4 + r;
                if (m < M && n < N) {
                    float v = acc[t][u][r];
                    if (!part && add) v += add[(size_t)m * N + n];
                    dst[(size_t)m * N + n] = v;
                }
            }
        }
}

// ---------------------------------------------------------------- host side


size_t mx_weight_bytes(uint32_t dtype, int N, int K) {
    if ((dtype != DT_Q8_0 && dtype != DT_Q4_0) || N <= 0 || K <= 0 || K % 32) return 0;
    return (size_t)((N + 15) / 16) * (K / 32) * MX_TB;
}

int launch_repack_mx(const void* W, uint32_t dtype, int N, int K, void* dst, hipStream_t s) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "repack mx: unsupported dtype %u", dtype);
    QH_REQUIRE(K % 32 == 0 && K > 0 && N > 0, QRAF_HIP_ERR_INVALID, "repack mx: K=%d must be a positive multiple of 32",
               K);
    QH_REQUIRE(W && dst && (((uintptr_t)W) & (dtype == DT_Q8_0 ? 3 : 1)) == 0 && (((uintptr_t)dst) & 15) == 0,
               QRAF_HIP_ERR_INVALID, "repack mx: null or misaligned pointer");
    const size_t total = (size_t)((N + 15) / 16) * (K / 32) * 16;
    const int grid = (int)std::min<size_t>((total + 255) / 256, 8192);
    if (dtype == DT_Q8_0)
        hipLaunchKernelGGL(repack_mx_kernel<8>, dim3(grid), dim3(256), 0, s, (const uint8_t*)W, N, K / 32,
                           (uint8_t*)dst);
    else
        hipLaunchKernelGGL(repack_mx_kernel<4>, dim3(grid), dim3(256), 0, s, (const uint8_t*)W, N, K / 32,
                           (uint8_t*)dst);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

// Workgroup shapes: (WMG, TN): WMG x 64 batch rows x 64 TN weight rows
enum MxShape { MX_128x256 = 0, MX_64x256 = 1, MX_128x192 = 2, MX_64x192 = 3, MX_SHAPES = 4 };
static const int kMxShape[MX_SHAPES][2] = {{2, 4}, {1, 4}, {2, 3}, {1, 3}};

static int g_mx_shape = -1;  // tuning: forced shape (-1 automatic)
static int g_mx_splits = 0;  // tuning: forced splits (0 automatic)

struct MxPlan {
    int shape, MW, NW, ntiles, mchunks, S, bps;
};

// Shape and split count: about one round of workgroups over the 256 CUs (one
// resident per CU), fewer splits when a split would hold under 8 blocks.
static MxPlan mx_plan(int N, int K, int M) {
    MxPlan p{};
    const int nb = K / 32;
    int best = -1;
    double best_cost = 0;
    for (int sh = 0; sh < MX_SHAPES; sh++) {
        if (g_mx_shape >= 0 && sh != g_mx_shape) continue;
        const int MW = 64 * kMxShape[sh][0], NW = 64 * kMxShape[sh][1];
        const int ntiles = (N + NW - 1) / NW, mch = (M + MW - 1) / MW;
        int S = 1;
        if (g_mx_splits > 0) S = g_mx_splits;
        else
            while (S < 64 && (long)ntiles * mch * (S * 2) <= 256 && nb / (S * 2) >= 8) S *= 2;
        const int bps = (nb + S - 1) / S;
        const long wgs = (long)ntiles * mch * ((nb + bps - 1) / bps);
        // cost: rounds of one workgroup per CU x work per workgroup (MW x NW x blocks), plus partial traffic
        const double rounds = (double)((wgs + 255) / 256);
        const double work = rounds * (double)MW * NW * bps;
        const double partial = S > 1 ? (double)S * M * N * 4.0 * 8.0 / 256 : 0;  // bytes per CU, weighted
        const double cost = work / 1024.0 + partial / 64.0;
        if (best < 0 || cost < best_cost) {
            best = sh;
            best_cost = cost;
            p.S = S;
        }
    }
    p.shape = best;
    p.MW = 64 * kMxShape[best][0];
    p.NW = 64 * kMxShape[best][1];
    p.ntiles = (N + p.NW - 1) / p.NW;
    p.mchunks = (M + p.MW - 1) / p.MW;
    p.bps = (nb + p.S - 1) / p.S;
    p.S = (nb + p.bps - 1) / p.bps;
    return p;
}

int set_mx_tuning(int shape, int splits) {
    QH_REQUIRE(shape >= -1 && shape < MX_SHAPES && splits >= 0 && splits <= 256, QRAF_HIP_ERR_INVALID,
               "mx tuning: shape %d, splits %d", shape, splits);
    g_mx_shape = shape;
    g_mx_splits = splits;
    bump_tuning_generation();
    return QRAF_HIP_OK;
}

size_t qgemm_mx_partials_bytes(uint32_t dtype, int N, int K, int M) {
    if ((dtype != DT_Q8_0 && dtype != DT_Q4_0) || N <= 0 || K <= 0 || K % 32 || M <= 0) return 0;
    const MxPlan p = mx_plan(N, K, M);
    return p.S > 1 ? (size_t)p.S * M * N * 4 : 0;
}

template <int FMT, int EPI>
static void launch_mx_shape(int shape, dim3 grid, hipStream_t s, const uint8_t* W, int N, int nb, const uint16_t* xh,
                            const uint16_t* xl, int K, int M, float* Y, const float* add, int bps, float* part,
                            uint16_t* oh, uint16_t* ol) {
#define QH_MX(WMG_, TN_)                                                                                       \
    hipLaunchKernelGGL((qgemm_mx_kernel<FMT, WMG_, TN_, EPI>), grid, dim3(256 * WMG_), 0, s, W, N, nb, xh, xl, K, M, Y, \
                       add, bps, part, oh, ol)
    switch (shape) {
        case MX_128x256: QH_MX(2, 4); break;
        case MX_64x256: QH_MX(1, 4); break;
        case MX_128x192: QH_MX(2, 3); break;
        default: QH_MX(1, 3); break;
    }
#undef QH_MX
}

// W: mx form.  slices != null: partials mode (S slices [S][M][N] into ws for
// the caller's consumer, *slices = S; S may be 1, then ws holds Y).  silu_hi /
// silu_lo != null: the interleaved gate/up epilogue (one split; N even).
int launch_qgemm_mx(const void* W, uint32_t dtype, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                    float* Y, const float* add, void* ws, size_t ws_bytes, hipStream_t s, int* slices,
                    uint16_t* silu_hi, uint16_t* silu_lo) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "qgemm mx: unsupported dtype %u", dtype);
    QH_REQUIRE(K % 32 == 0 && K > 0 && N > 0 && M > 0, QRAF_HIP_ERR_INVALID, "qgemm mx: shape %d x %d, batch %d", N, K,
               M);
    QH_REQUIRE(W && xh && xl && (((uintptr_t)W) & 15) == 0 && (((uintptr_t)xh) & 15) == 0 &&
                   (((uintptr_t)xl) & 15) == 0,
               QRAF_HIP_ERR_INVALID, "qgemm mx: null or misaligned operands");
    QH_REQUIRE((size_t)M * K * 2 <= 0xFFFFFFFFu && (size_t)((N + 15) / 16) * (K / 32) * MX_TB <= 0xFFFFFFFFu,
               QRAF_HIP_ERR_INVALID, "qgemm mx: operands beyond 4 GiB");
    const int nb = K / 32;
    MxPlan p = mx_plan(N, K, M);
    const bool silu = silu_hi != nullptr;
    float* part = nullptr;
    if (silu) {
        QH_REQUIRE(silu_lo && N % 2 == 0 && !add, QRAF_HIP_ERR_INVALID, "qgemm mx: SiLU-gate epilogue arguments");
        p.S = 1;
        p.bps = nb;
    } else if (slices) {
        QH_REQUIRE(ws && ws_bytes >= (size_t)p.S * M * N * 4 && (((uintptr_t)ws) & 15) == 0 && !add,
                   QRAF_HIP_ERR_INVALID, "qgemm mx: partials need a workspace of %zu bytes and no residual",
                   (size_t)p.S * M * N * 4);
        part = (float*)ws;
        *slices = p.S;
    } else {
        QH_REQUIRE(Y, QRAF_HIP_ERR_INVALID, "qgemm mx: null output");
        if (p.S > 1) {
            if (ws && ws_bytes >= (size_t)p.S * M * N * 4 && (((uintptr_t)ws) & 15) == 0) {
                part = (float*)ws;
            } else {
                p.S = 1;
                p.bps = nb;
            }
        }
    }
    QH_REQUIRE(p.mchunks <= 65535 && p.S <= 65535, QRAF_HIP_ERR_INVALID, "qgemm mx: batch %d too large", M);
    const dim3 grid(p.ntiles, p.S, p.mchunks);
    const uint8_t* w = (const uint8_t*)W;
    if (dtype == DT_Q8_0) {
        if (silu) launch_mx_shape<8, 1>(p.shape, grid, s, w, N, nb, xh, xl, K, M, Y, add, p.bps, part, silu_hi, silu_lo);
        else launch_mx_shape<8, 0>(p.shape, grid, s, w, N, nb, xh, xl, K, M, Y, add, p.bps, part, nullptr, nullptr);
    } else {
        if (silu) launch_mx_shape<4, 1>(p.shape, grid, s, w, N, nb, xh, xl, K, M, Y, add, p.bps, part, silu_hi, silu_lo);
        else launch_mx_shape<4, 0>(p.shape, grid, s, w, N, nb, xh, xl, K, M, Y, add, p.bps, part, nullptr, nullptr);
    }
    QH_CHECK_HIP(hipGetLastError());
    if (part && !slices) {
        const size_t MN = (size_t)M * N;
        QH_TRY(launch_reduce_slices(part, p.S, MN, Y, add, s));
    }
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip

extern "C" {

uint64_t qraf_hip_mx_weight_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim) {
    return qraf_hip::mx_weight_bytes(dtype, (int)out_dim, (int)in_dim);
}

int qraf_hip_repack_mx_dev(const void* w, uint32_t dtype, uint32_t out_dim, uint32_t in_dim, void* dst, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_repack_mx(w, dtype, (int)out_dim, (int)in_dim, dst, qraf_hip::as_stream(stream));
}

uint64_t qraf_hip_qgemm_mx_workspace_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim, int32_t batch) {
    return qraf_hip::qgemm_mx_partials_bytes(dtype, (int)out_dim, (int)in_dim, batch);
}

int qraf_hip_qgemm_mx_dev(const void* w_mx, uint32_t dtype, uint32_t out_dim, uint32_t in_dim, const uint16_t* x_hi,
                          const uint16_t* x_lo, int32_t batch, float* y, const float* add, void* workspace,
                          uint64_t workspace_bytes, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_qgemm_mx(w_mx, dtype, (int)out_dim, (int)in_dim, x_hi, x_lo, batch, y, add, workspace,
                                     workspace_bytes, qraf_hip::as_stream(stream), nullptr, nullptr, nullptr);
}

int qraf_hip_qgemm_mx_silu_dev(const void* w_mx, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                               const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, uint16_t* out_hi,
                               uint16_t* out_lo, void* stream) {
    qraf_hip::clear_error();
    if (!out_hi || !out_lo)
        return qraf_hip::set_error(QRAF_HIP_ERR_INVALID, "qgemm mx silu: null output planes");
    return qraf_hip::launch_qgemm_mx(w_mx, dtype, (int)out_dim, (int)in_dim, x_hi, x_lo, batch, nullptr, nullptr,
                                     nullptr, 0, qraf_hip::as_stream(stream), nullptr, out_hi, out_lo);
}

int qraf_hip_set_mx_tuning(int32_t shape, int32_t splits) {
    qraf_hip::clear_error();
    return qraf_hip::set_mx_tuning(shape, splits);
}

}  // extern "C"
