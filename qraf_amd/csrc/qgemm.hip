// qgemm.hip -- batched Q8_0 / Q4_0 GEMM on gfx950 matrix cores.
//
// Y[m][n] = sum_k X[m][k] * W[n][k]  (+ add[m][n])  for a continuous-batch
// decode step: the M rows of X are M sequences' activations, W is a weight
// matrix in the reference's Q8_0/Q4_0 block layout (quantize.h:11-30).  The
// reference has no batched product: this is dispatch_matvec_q
// (backend.cpp:131-199) applied to M vectors at once.
//
// Exactness: each quant block is one K=32 step of two matrix-core products,
// v_mfma_f32_16x16x32_bf16 then _f16.  Weights enter as bf16 and fp16 copies
// of the block integers (exact: |q| <= 127), X as two planes: hi = the bf16 of
// x, lo = the fp16 of the rest, x = hi + lo + r with |r| <= 2^-20 |x| + 2^-25
// for |x| < 2^24 (split once per activation by split_bf16_kernel).  The two
// MFMAs of a block accumulate sum_k q (x_hi + x_lo) in fp32 (products exact),
// then the block is scaled by its fp32 (Q8) or fp16 (Q4) scale with one FMA
// per output:
//     |y - y_exact| <= sum_k |w_k| (2^-20 |x_k| + 2^-25) + (K + 2) 2^-24 sum_k |w_k x_k|.
//
// Tiling.  A workgroup (4 waves) owns a tile of MW batch rows x 128 weight
// rows over a range of quant blocks.  For MW > 32 the waves form a 2 x 2
// grid, each wave 64 weight rows (four 16-row MFMA tiles) x MW/2 batch rows;
// otherwise the four waves split the 128 weight rows.  X is staged in LDS KC
// quant blocks at a time (both planes; KC = 2, 4 or 8 as the batch tile
// shrinks, so every stage moves enough bytes; rows padded so ds_read_b128 of
// an MFMA operand is conflict-free), double-buffered with one barrier per
// stage; each X fragment read from LDS feeds TN weight tiles.  Weights are
// read straight into registers through a buffer resource, two stages ahead.
// MFMA operand layout (16x16x32): lane l supplies row l%16, k = 8*(l/16)..+7
// of A (= X) and of B^T (= W); it receives D[4*(l/16) + r][l%16], r = 0..3,
// i.e. four batch rows of one weight row, so one block scale per lane.
//
// Split-K.  When the weight matrix has too few 128-row tiles to fill the
// chip, the block range is split S ways; each split writes an fp32 partial
// tile to a workspace and qgemm_reduce_kernel adds the S partials in split
// order (deterministic), plus the residual.
#include <type_traits>

#include "common.h"

namespace qraf_hip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32a2 __attribute__((aligned(2)));

constexpr int QG_MCHUNK = 128;         // batch rows per workgroup at most

// X fp32 [M][K] -> hi (bf16), lo (fp16) planes [M][K] (hi = rne(x), lo = rne(x - hi)).
// op 0: x as given; op 1: x = silu(g) * u from an interleaved gate/up row
// [M][2K] (g = even columns, u = odd columns), ops.cpp:218-222 then :275-279.
// x may be S slices (GEMM split-K partials) of `slice` floats, summed in order.
__global__ void split_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                  int M, int K, int op, float* __restrict__ xout, int S, size_t slice) {
    const size_t n = (size_t)M * K;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v;
        if (op == 1) {
            const size_t m = i / K, k = i % K;
            const size_t e = m * 2 * K + 2 * k;
            const float g = sum_slices(x, S, slice, e), u = sum_slices(x, S, slice, e + 1);
            v = silu_gate(g, u);
            if (xout) xout[i] = v;
        } else {
            v = sum_slices(x, S, slice, i);
        }
        split_bf16(v, &hi[i], &lo[i]);
    }
}

// op 1 with four outputs per thread: outputs k..k+3 of row m read the 8
// interleaved gate/up floats 2k..2k+7 of each slice as two 16-byte loads (all
// slices' loads issued before the first add, sums in slice order as in
// split_bf16_kernel, so the planes are the same bit for bit) and write 8-byte
// hi and lo stores.  K % 4 == 0, 16-byte aligned x and slice, 8-byte aligned
// planes, M * K < 2^31.
template <int S>
__global__ __launch_bounds__(256) void silu_split4_kernel(const float* __restrict__ x, uint16_t* __restrict__ hi,
                                                          uint16_t* __restrict__ lo, int M, int K, size_t slice) {
    const int n4 = M * (K >> 2);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const int m = i / (K >> 2), k = (i - m * (K >> 2)) << 2;
        const float* p = x + (size_t)m * 2 * K + 2 * k;
        f32x4 a[S], b[S];
#pragma unroll
        for (int u = 0; u < S; u++) {
            a[u] = *(const f32x4*)(p + (size_t)u * slice);
            b[u] = *(const f32x4*)(p + (size_t)u * slice + 4);
        }
        f32x4 ga = a[0], gb = b[0];
#pragma unroll
        for (int u = 1; u < S; u++) {
            ga += a[u];
            gb += b[u];
        }
        const float v0 = silu_gate(ga[0], ga[1]), v1 = silu_gate(ga[2], ga[3]);
        const float v2 = silu_gate(gb[0], gb[1]), v3 = silu_gate(gb[2], gb[3]);
        uint16_t h[4], l[4];
        split_bf16(v0, &h[0], &l[0]);
        split_bf16(v1, &h[1], &l[1]);
        split_bf16(v2, &h[2], &l[2]);
        split_bf16(v3, &h[3], &l[3]);
        const size_t e = (size_t)m * K + k;
        *(uint2*)(hi + e) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
        *(uint2*)(lo + e) = make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    }
}

// Raw weight fragment of one lane for one (16-row tile, block): the block
// scale and the 8 quants k = 8*seg..8*seg+7 of the lane's row.
template <int FMT>
struct WRaw;
template <>
struct WRaw<8> {
    uint32_t scale;  // fp32 bits
    uint32_t q0, q1;  // int8 x 8
};
template <>
struct WRaw<4> {
    uint32_t scale;  // fp16 bits
    uint32_t q;       // 8 nibbles: byte j = elements 2j (low), 2j+1 (high)
};

// Raw buffer resource over [p, p + bytes): a load whose VGPR offset is at or
// past `bytes` returns zeros (gfx9 raw buffer: 32-bit data format, no swizzle).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr uint32_t OOB = 0x80000000u;  // VGPR offset that is always out of range

// sc: byte offset of the lane's row, qo: of its 8 quants within a block,
// boff: the (uniform) byte offset of the block within a row
template <int FMT>
__device__ __forceinline__ void load_raw(rsrc_t w, uint32_t sc, uint32_t qo, uint32_t boff, WRaw<FMT>& r);
template <>
__device__ __forceinline__ void load_raw<8>(rsrc_t w, uint32_t sc, uint32_t qo, uint32_t boff, WRaw<8>& r) {
    r.scale = __builtin_amdgcn_raw_buffer_load_b32(w, sc, boff, 0);
    const auto q = __builtin_amdgcn_raw_buffer_load_b64(w, qo, boff, 0);  // 36-byte blocks: 4-byte aligned
    r.q0 = q[0];
    r.q1 = q[1];
}
template <>
__device__ __forceinline__ void load_raw<4>(rsrc_t w, uint32_t sc, uint32_t qo, uint32_t boff, WRaw<4>& r) {
    // 18-byte blocks: every field is read with aligned 16-bit loads
    r.scale = __builtin_amdgcn_raw_buffer_load_b16(w, sc, boff, 0);
    const uint32_t a = __builtin_amdgcn_raw_buffer_load_b16(w, qo, boff, 0);
    const uint32_t b = __builtin_amdgcn_raw_buffer_load_b16(w, qo + 2, boff, 0);
    r.q = a | (b << 16);
}

// Tile-major weights (repack_tiles_kernel): for every 16-row tile and quant
// block, the 16 scales then the 16 rows' quants, so one load instruction of a
// wave reads contiguous memory.  sc / qo: byte offsets of the lane's scale and
// 8 quants within the first tile-block, boff: the (uniform) offset of the block.
template <int FMT>
__device__ __forceinline__ void load_tiled(rsrc_t w, uint32_t sc, uint32_t qo, uint32_t boff, WRaw<FMT>& r);
template <>
__device__ __forceinline__ void load_tiled<8>(rsrc_t w, uint32_t sc, uint32_t qo, uint32_t boff, WRaw<8>& r) {
    r.scale = __builtin_amdgcn_raw_buffer_load_b32(w, sc, boff, 0);
    const auto q = __builtin_amdgcn_raw_buffer_load_b64(w, qo, boff, 0);
    r.q0 = q[0];
    r.q1 = q[1];
}
template <>
__device__ __forceinline__ void load_tiled<4>(rsrc_t w, uint32_t sc, uint32_t qo, uint32_t boff, WRaw<4>& r) {
    r.scale = __builtin_amdgcn_raw_buffer_load_b16(w, sc, boff, 0);
    r.q = __builtin_amdgcn_raw_buffer_load_b32(w, qo, boff, 0);
}

// bytes of one tile-block: 16 scales + 16 rows of 32 quants
__host__ __device__ constexpr int tile_block_bytes(int fmt) { return fmt == 8 ? 16 * 36 : 16 * 18; }

// Reference row-major blocks -> tile-major: thread per (tile, block, row).
// Rows past N are zero (scale 0, quants 0).
template <int FMT>
__global__ void repack_tiles_kernel(const uint8_t* __restrict__ src, int N, int nb, uint8_t* __restrict__ dst) {
    constexpr int BB = FMT == 8 ? 36 : 18, SB = FMT == 8 ? 4 : 2, QB = BB - SB, TB = tile_block_bytes(FMT);
    const size_t rb = (size_t)nb * BB;
    const size_t total = (size_t)((N + 15) / 16) * nb * 16;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i & 15);
        const size_t tb = i >> 4;  // tile * nb + block
        const size_t t = tb / nb, b = tb % nb;
        const size_t row = t * 16 + r;
        uint8_t* d = dst + tb * TB;
        uint16_t* ds = (uint16_t*)(d + SB * r);
        uint16_t* dq = (uint16_t*)(d + 16 * SB + QB * r);
        if (row < (size_t)N) {
            const uint16_t* sp = (const uint16_t*)(src + row * rb + b * BB);  // 2-byte aligned fields
#pragma unroll
            for (int h = 0; h < SB / 2; h++) ds[h] = sp[h];
#pragma unroll
            for (int h = 0; h < QB / 2; h++) dq[h] = sp[SB / 2 + h];
        } else {
#pragma unroll
            for (int h = 0; h < SB / 2; h++) ds[h] = 0;
#pragma unroll
            for (int h = 0; h < QB / 2; h++) dq[h] = 0;
        }
    }
}

__device__ __forceinline__ uint32_t bf16_pair(float even, float odd) {
    // exact small integers: the bf16 value is the high half of the fp32 bits
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, odd), __builtin_bit_cast(uint32_t, even), 0x07060302u);
}

__device__ __forceinline__ uint32_t f16_pair(float even, float odd) {
    // exact small integers: round-toward-zero packing loses nothing
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(even, odd));
}

// One lane's 8 quants of a block as the bf16 operand (for the hi plane) and
// the fp16 operand (for the lo plane) of the block's two MFMAs, and its scale.
template <int FMT>
__device__ __forceinline__ void convert(const WRaw<FMT>& r, bf16x8& w, f16x8& wh, float& scale);
template <>
__device__ __forceinline__ void convert<8>(const WRaw<8>& r, bf16x8& w, f16x8& wh, float& scale) {
    scale = __builtin_bit_cast(float, r.scale);
    u32x4 p, ph;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t d = j ? r.q1 : r.q0;
        const float f0 = (float)(int8_t)(d), f1 = (float)(int8_t)(d >> 8);
        const float f2 = (float)(int8_t)(d >> 16), f3 = (float)(int8_t)(d >> 24);
        p[2 * j] = bf16_pair(f0, f1);
        p[2 * j + 1] = bf16_pair(f2, f3);
        ph[2 * j] = f16_pair(f0, f1);
        ph[2 * j + 1] = f16_pair(f2, f3);
    }
    w = __builtin_bit_cast(bf16x8, p);
    wh = __builtin_bit_cast(f16x8, ph);
}
template <>
__device__ __forceinline__ void convert<4>(const WRaw<4>& r, bf16x8& w, f16x8& wh, float& scale) {
    scale = (float)__builtin_bit_cast(_Float16, (uint16_t)r.scale);
    // nibble u -> signed byte u - 8: (u + 0x78) ^ 0x80, no carry between bytes
    const uint32_t lo = ((r.q & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    const uint32_t hi = (((r.q >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    u32x4 p, ph;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float f0 = (float)(int8_t)(lo >> (8 * j)), f1 = (float)(int8_t)(hi >> (8 * j));
        p[j] = bf16_pair(f0, f1);
        ph[j] = f16_pair(f0, f1);
    }
    w = __builtin_bit_cast(bf16x8, p);
    wh = __builtin_bit_cast(f16x8, ph);
}

// A wave's TM x TN tiles of 16 x 16 MFMA results (lane: weight row nb + 16u +
// l16, batch rows mb + 16t + 4seg + r) stored to dst[m][n] (+ add[m][n]).  A
// wave whose tiles lie wholly inside M x N (the uniform case) stores without
// per-element bounds checks and issues all its residual loads before the first
// store; the other waves check every element.
template <int TM, int TN>
__device__ __forceinline__ void store_tiles(const f32x4 (&acc)[TM][TN], float* dst, const float* add, int M, int N,
                                            int mb, int nb, int seg, int l16) {
    if (mb + 16 * TM <= M && nb + 16 * TN <= N) {
        const size_t o = (size_t)(mb + 4 * seg) * N + nb + l16;
        float* d = dst + o;
        if (add) {
            const float* a = add + o;
            float av[TM][TN][4];
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int u = 0; u < TN; u++)
#pragma unroll
                    for (int r = 0; r < 4; r++) av[t][u][r] = a[(size_t)(16 * t + r) * N + 16 * u];
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int u = 0; u < TN; u++)
#pragma unroll
                    for (int r = 0; r < 4; r++) d[(size_t)(16 * t + r) * N + 16 * u] = acc[t][u][r] + av[t][u][r];
        } else {
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int u = 0; u < TN; u++)
#pragma unroll
                    for (int r = 0; r < 4; r++) d[(size_t)(16 * t + r) * N + 16 * u] = acc[t][u][r];
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < TM; t++) {
#pragma unroll
        for (int u = 0; u < TN; u++) {
            const int n = nb + u * 16 + l16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mb + t * 16 + seg * 4 + r;
                if (m < M && n < N) {
                    float v = acc[t][u][r];
                    if (add) v += add[(size_t)m * N + n];
                    dst[(size_t)m * N + n] = v;
                }
            }
        }
    }
}

// WM x WN waves (batch x weight rows); TM: 16-row batch tiles per wave; TN:
// 16-row weight tiles per wave; KC: quant blocks per stage.  A workgroup
// owns WM*TM*16 batch rows x WN*TN*16 weight rows.
//
// Pipeline (two stages per loop trip, no register copies): while stage c
// computes from LDS buffer c&1 and weight registers set c&1, X of stage c+1
// sits in registers (stored to LDS after the compute, one barrier per
// stage) and the weights of stage c+1 are in flight into the other set; the
// weights of stage c+2 are requested as soon as stage c has consumed its set.
template <int FMT, int WM, int WNW, int TM, int TN, int KC, bool TILED>
__global__ __launch_bounds__(64 * WM * WNW, 512 / (64 * WM * WNW)) void qgemm_kernel(
    const uint8_t* __restrict__ W, size_t row_bytes, int N, int nb, const uint16_t* __restrict__ xh,
    const uint16_t* __restrict__ xl, int K, int M, float* Y, const float* add, int bps, float* __restrict__ part) {
    constexpr int QG_THREADS = 64 * WM * WNW;
    constexpr int QG_NW = WNW * TN * 16;
    static_assert(QG_THREADS % (KC * 4) == 0, "stage shape");
    constexpr int MW = WM * TM * 16;
    constexpr int XS = KC * 32 + 8;  // LDS row stride in bf16: (4 KC + 1) 16-byte units, odd -> conflict-free
    constexpr int PLANE = MW * XS;
    constexpr int PIECES = 2 * MW * KC * 4;  // 16-byte pieces of X per stage
    constexpr int PP = PIECES / QG_THREADS;
    static_assert(PIECES % QG_THREADS == 0, "staging shape");
    __shared__ __align__(16) uint16_t sx[2 * 2 * PLANE];  // [buffer][plane][MW][XS]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WNW, wn = wave % WNW;
    const int seg = lane >> 4, l16 = lane & 15;
    const int m0 = blockIdx.z * MW;
    const int nbase = blockIdx.x * QG_NW + wn * TN * 16;
    const int b_begin = blockIdx.y * bps;  // bps: a positive multiple of 2 KC
    const int b_end = min(nb, b_begin + bps);
    const int nchunks = bps / KC;  // even; blocks past b_end are read clamped and weighted 0

    // block stride of the weight stream: a row's next block (reference
    // layout) or the tile's next tile-block (tile-major layout)
    constexpr int BB = TILED ? tile_block_bytes(FMT) : (FMT == 8 ? 36 : 18);
    const int ntile16 = (N + 15) / 16;
    const size_t wbytes = TILED ? (size_t)ntile16 * nb * BB : (size_t)N * row_bytes;
    const rsrc_t wrs = make_rsrc(W, (uint32_t)min(wbytes, (size_t)0xFFFFFFFFu));
    uint32_t wsc[TN], wq[TN];  // per weight tile: scale offset, quant offset
#pragma unroll
    for (int u = 0; u < TN; u++) {
        if (TILED) {
            const uint32_t tb = (uint32_t)((size_t)min((nbase >> 4) + u, ntile16 - 1) * nb * BB);
            wsc[u] = tb + (FMT == 8 ? 4 * l16 : 2 * l16);
            wq[u] = tb + (FMT == 8 ? 64 + 32 * l16 + 8 * seg : 32 + 16 * l16 + 4 * seg);
        } else {
            wsc[u] = (uint32_t)((size_t)min(nbase + u * 16 + l16, N - 1) * row_bytes);
            wq[u] = wsc[u] + (FMT == 8 ? 4 + 8 * seg : 2 + 4 * seg);
        }
    }

    // X staging: piece p of this thread is (row r, plane, 16-byte quarter q of
    // block j of the stage); q and j are the same for every p.
    // Rows past M read row M-1 (finite data whose outputs are never stored);
    // blocks past the end are clamped to the last block (never used).
    const int xq = tid % (KC * 4), xj = xq >> 2;
    const uint16_t* xptr[PP];
    int xlds[PP];
#pragma unroll
    for (int p = 0; p < PP; p++) {
        const int rest = (tid + p * QG_THREADS) / (KC * 4);
        const int plane = rest & 1, r = rest >> 1, m = m0 + r;
        xptr[p] = (plane ? xl : xh) + (size_t)min(m, M - 1) * K + (xq & 3) * 8;
        xlds[p] = plane * PLANE + r * XS + xq * 8;
    }
    u32x4 xr[PP];
    auto load_x = [&](int c) {
        const int boff = min(b_begin + c * KC + xj, nb - 1) * 32;
#pragma unroll
        for (int p = 0; p < PP; p++) xr[p] = *(const u32x4*)(xptr[p] + boff);
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PP; p++) *(u32x4*)&sx[buf * 2 * PLANE + xlds[p]] = xr[p];
    };
    auto load_w = [&](WRaw<FMT>(&dst)[KC][TN], int c) {
        const int cb = b_begin + c * KC;
#pragma unroll
        for (int j = 0; j < KC; j++) {
            const uint32_t boff = (uint32_t)max(min(cb + j, b_end - 1), 0) * BB;
#pragma unroll
            for (int u = 0; u < TN; u++) {
                if (TILED) load_tiled<FMT>(wrs, wsc[u], wq[u], boff, dst[j][u]);
                else load_raw<FMT>(wrs, wsc[u], wq[u], boff, dst[j][u]);
            }
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int u = 0; u < TN; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int c, const WRaw<FMT>(&wc)[KC][TN]) {
        const int buf = c & 1, cb = b_begin + c * KC;
#pragma unroll
        for (int j = 0; j < KC; j++) {
            const bool valid = cb + j < b_end;  // uniform; an invalid block's scale is 0 (its data is finite)
            bf16x8 wf[TN];
            f16x8 wh[TN];
            float sc[TN];
#pragma unroll
            for (int u = 0; u < TN; u++) {
                WRaw<FMT> r = wc[j][u];
                r.scale = valid ? r.scale : 0u;
                convert<FMT>(r, wf[u], wh[u], sc[u]);
            }
#pragma unroll
            for (int t = 0; t < TM; t++) {
                const int row = (wm * TM + t) * 16 + l16;
                const bf16x8 ah = *(const bf16x8*)&sx[(buf * 2 + 0) * PLANE + row * XS + j * 32 + seg * 8];
                const f16x8 al = *(const f16x8*)&sx[(buf * 2 + 1) * PLANE + row * XS + j * 32 + seg * 8];
#pragma unroll
                for (int u = 0; u < TN; u++) {
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wf[u], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, wh[u], d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[t][u][r] = __builtin_fmaf(d[r], sc[u], acc[t][u][r]);
                }
            }
        }
    };
    // one stage: compute c, publish X of c+1, request X and weights of c+2
    // (past the end these are clamped loads that are never read)
    // (past the end these are clamped loads that are never read).  X loads are
    // issued before weight loads so that waiting for X never waits for weights.
    auto step = [&](int c, WRaw<FMT>(&wc)[KC][TN]) {
        compute(c, wc);
        __builtin_amdgcn_sched_barrier(0);
        store_x((c & 1) ^ 1);
        __builtin_amdgcn_sched_barrier(0);
        load_x(c + 2);
        __builtin_amdgcn_sched_barrier(0);
        load_w(wc, c + 2);
        __syncthreads();
    };

    WRaw<FMT> wa[KC][TN], wb[KC][TN];
    load_w(wa, 0);
    load_x(0);
    store_x(0);
    load_x(1);
    __builtin_amdgcn_sched_barrier(0);
    load_w(wb, 1);
    __syncthreads();
    for (int c = 0; c < nchunks; c += 2) {
        step(c, wa);
        step(c + 1, wb);
    }

    // epilogue: direct (+ residual) or this split's partial tile
    float* dst = part ? part + (size_t)blockIdx.y * M * N : Y;
    store_tiles<TM, TN>(acc, dst, part ? nullptr : add, M, N, m0 + wm * TM * 16, nbase, seg, l16);
}

// ---------------------------------------------------------------------------
// Pipelined GEMM for tile-major weights and batches over 32 rows.
//
// Workgroup tile: MW = 32*TM batch rows x NW = 32*TN weight rows, 4 waves in
// a 2 x 2 grid, each wave TM x TN MFMA tiles of 16 x 16.  Three LDS stage
// buffers, each holding KC quant blocks of X (both planes) and of W, are
// filled by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds): while
// stage c computes, stages c+1 and c+2 are in flight.  One raw s_barrier per
// stage, after the wave's own loads of stage c have landed (explicit vmcnt
// wait with one stage still outstanding) and its LDS reads are done.
// X rows in LDS are XOR-swizzled by 16-byte piece (slot = piece ^ (row & 7))
// so the MFMA operand reads of 16 rows are bank-conflict-free; the swizzle
// is applied through the per-lane global source addresses of the DMA.
// Blocks past the split's range (stage padding) are read from wherever the
// clamped or out-of-range address points and not computed.
// ---------------------------------------------------------------------------
// The three stage buffers are file-scope LDS objects reached through
// compile-time accessors: the compiler then sees that a DMA into one buffer
// does not alias reads of another and inserts no waits of its own.
// Kernels whose stages fit QG_STAGE_SMALL use the small set (72 KB in all),
// so two workgroups fit in a CU's LDS.
constexpr int QG_STAGE_MAX = 53248;
constexpr int QG_STAGE_SMALL = 24576;
__shared__ __align__(16) uint8_t qg_sb0[QG_STAGE_MAX];
__shared__ __align__(16) uint8_t qg_sb1[QG_STAGE_MAX];
__shared__ __align__(16) uint8_t qg_sb2[QG_STAGE_MAX];
__shared__ __align__(16) uint8_t qg_ss0[QG_STAGE_SMALL];
__shared__ __align__(16) uint8_t qg_ss1[QG_STAGE_SMALL];
__shared__ __align__(16) uint8_t qg_ss2[QG_STAGE_SMALL];
template <int B, bool SMALL>
__device__ __forceinline__ uint8_t* qg_stage() {
    if (SMALL) return B == 0 ? qg_ss0 : B == 1 ? qg_ss1 : qg_ss2;
    return B == 0 ? qg_sb0 : B == 1 ? qg_sb1 : qg_sb2;
}

// WN: waves along the weight rows (2 x WN waves); wave tile 16*TM x 16*TN.
template <int FMT, int TM, int TN, int KC, int WN, int WMN>
struct PipeGeom {
    static constexpr int NWV = WMN * WN;              // waves per workgroup
    static constexpr int MW = 16 * TM * WMN, NW = 16 * TN * WN;
    static constexpr int TB = tile_block_bytes(FMT);
    static constexpr int XROW = KC * 64;              // bytes of one X row (one plane) per stage
    static constexpr int XPL = MW * XROW;             // bytes of one plane per stage
    static constexpr int XT = 2 * XPL / 1024;         // X DMA instructions per stage (1 KB each)
    static constexpr int XI = XT / NWV;               // ... per wave
    static constexpr int WBYTES = (NW / 16) * KC * TB;
    static constexpr int WT = (WBYTES + 1023) / 1024;  // W DMA instructions per stage
    static constexpr int WIL = WT / NWV, WEXTRA = WT % NWV;  // waves < WEXTRA issue WIL + 1
    static constexpr int WIH = WIL + (WEXTRA ? 1 : 0);
    static constexpr int STAGE = 2 * XPL + WT * 1024;  // bytes per stage buffer
    static_assert(XT % NWV == 0, "X stage must split evenly over the waves");
    static_assert((XPL / 16) % 64 == 0, "an X DMA instruction must stay in one plane");
    static_assert(KC * 4 >= 8, "swizzle needs 8 pieces per row");
    static_assert(STAGE <= QG_STAGE_MAX, "stage buffer too small");
    static constexpr bool SMALL = STAGE <= QG_STAGE_SMALL;  // two workgroups per CU
    static constexpr int MINB = SMALL ? 2 : 1;
};

// Sampler::argmax's order (sampler.cpp:25-35: the first of the largest
// values) as one unsigned 64-bit key: the value's bits made monotonic in the
// high word (-0 counted as +0, as the reference's > comparison counts them
// equal), 0xFFFFFFFF - index in the low word, so a larger key is a larger
// value or, for equal values, a smaller index.  A NaN's high word is 0, below
// every number's: a NaN is chosen only in a row of NaNs (then the first, as
// the reference); the reference would also keep a NaN at position 0.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    const uint32_t b = __float_as_uint(v + 0.0f);
    const uint32_t o = v != v ? 0u : (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (0xFFFFFFFFu - idx);
}

// One step of a prefix max over the 16 lanes of each DPP row, for every key
// of a lane: key = max(key, the key of the lane CTRL's row_shr names), lanes
// shifted in from outside the row reading 0 (the keys' identity).
template <int CTRL>
__device__ __forceinline__ void key_row_max(uint64_t (&k)[4]) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        lo[r] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)k[r], CTRL, 0xF, 0xF, false);
        hi[r] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(k[r] >> 32), CTRL, 0xF, 0xF, false);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint64_t o = ((uint64_t)hi[r] << 32) | lo[r];
        k[r] = o > k[r] ? o : k[r];
    }
}

// Stream-K schedule: workgroup w of G owns blocks [w T / G, (w+1) T / G) of the T = units x nb
// (tile, quant block) pairs, units in tile-major order; the workgroup that owns pair x:
__host__ __device__ inline int sk_owner(long long x, long long T, int G) {
    int w = (int)(x * G / T);
    while (w + 1 < G && (long long)(w + 1) * T / G <= x) w++;
    return w;
}

// SK: the stream-K schedule (skG workgroups), else the uniform split grid.  Two
// instantiations, since one kernel holding both loops spills ~100-200 SGPRs
// into VGPR lanes (a readlane per descriptor word at every DMA issue).
// AMAX: the greedy head's argmax epilogue (amax), an instantiation of its own
// so that its registers do not raise the other forms' allocation.
template <int FMT, int TM, int TN, int KC, int WN, int WMN, bool SK, bool AMAX = false>
__global__ __launch_bounds__(64 * WMN * WN, (PipeGeom<FMT, TM, TN, KC, WN, WMN>::MINB)) void qgemm_pipe_kernel(const uint8_t* __restrict__ Wt, int N, int nb,
                                                                 const uint16_t* __restrict__ xh,
                                                                 const uint16_t* __restrict__ xl, int K, int M,
                                                                 float* Y, const float* add, int bps,
                                                                 float* __restrict__ part, int skG, int sk_ntiles,
                                                                 int skS, uint16_t* __restrict__ act_hi,
                                                                 uint16_t* __restrict__ act_lo,
                                                                 uint64_t* __restrict__ amax) {
    using G = PipeGeom<FMT, TM, TN, KC, WN, WMN>;
    constexpr int MW = G::MW, NW = G::NW, TB = G::TB, NWV = G::NWV;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: selects descriptors and M0
    const int wm = wave / WN, wn = wave % WN;
    const bool wextra = wave < G::WEXTRA;  // this wave issues one more W instruction per stage
    const int seg = lane >> 4, l16 = lane & 15;
    const uint32_t xbytes = (uint32_t)((size_t)M * K * 2);
    const v4i xrs[2] = {make_rsrc_words(xh, xbytes), make_rsrc_words(xl, xbytes)};
    const int ntile16 = (N + 15) / 16;
    const v4i wrs = make_rsrc_words(Wt, (uint32_t)min((size_t)ntile16 * nb * TB, (size_t)0xFFFFFFFFu));

    // One segment: weight rows [n0, n0 + NW) x batch rows [m0, m0 + MW) over
    // quant blocks [b_begin, b_end), written to dst (+ add when given).
    auto segment = [&](const int n0, const int m0, const int b_begin, const int b_end, float* dst, const float* addp) {
    const int nstages = ((b_end - b_begin + KC - 1) / KC + 2) / 3 * 3;  // whole trips of the 3-stage loop

    // ---- DMA source offsets (bytes), fixed per lane and instruction; the
    // stage's first block adds cb*64 (X) or cb*TB (W)
    uint32_t xo[G::XI], wo[G::WIH];
#pragma unroll
    for (int q = 0; q < G::XI; q++) {
        const int f = (q * NWV + wave) * 64 + lane;  // 16-byte slot in the stage's X area
        const int plane = f / (G::XPL / 16);
        const int rem = f % (G::XPL / 16);
        const int row = rem / (KC * 4), slot = rem % (KC * 4);
        const int piece = slot ^ (row & 7);
        (void)plane;
        xo[q] = (uint32_t)((size_t)min(m0 + row, M - 1) * K * 2) + 16u * piece;
    }
#pragma unroll
    for (int q = 0; q < G::WIH; q++) {
        const int f = (q * NWV + wave) * 64 + lane;  // 16-byte slot in the stage's W area
        const int u = min((16 * f) / (KC * TB), NW / 16 - 1);  // slots past WBYTES re-read the last tile
        const int off = (16 * f) % (KC * TB);
        const int T = min(n0 / 16 + u, ntile16 - 1);
        wo[q] = (uint32_t)((size_t)T * nb * TB) + off;
    }
    auto issue = [&](auto bsel, int c) {
        uint8_t* buf = qg_stage<decltype(bsel)::value, G::SMALL>();
        const int cb = min(b_begin + c * KC, b_end - 1);  // stages past the range re-read valid blocks
#pragma unroll
        for (int q = 0; q < G::XI; q++) {
            const int plane = ((q * NWV + wave) * 64) / (G::XPL / 16);  // wave-uniform
            dma16(xrs[plane], xo[q] + (uint32_t)cb * 64u, buf + (size_t)(q * NWV + wave) * 1024);
        }
#pragma unroll
        for (int q = 0; q < G::WIL; q++)
            dma16(wrs, wo[q] + (uint32_t)cb * TB, buf + 2 * G::XPL + (size_t)(q * NWV + wave) * 1024);
        if (G::WEXTRA && wextra)
            dma16(wrs, wo[G::WIH - 1] + (uint32_t)cb * TB, buf + 2 * G::XPL + (size_t)(G::WIL * NWV + wave) * 1024);
    };
    // this wave's loads of the oldest stage in flight have landed (one stage may
    // remain outstanding) and its LDS reads are done
    auto wait_stage = [&]() {
        if (wextra) wait_vm_lgkm0<G::XI + G::WIH>();
        else wait_vm_lgkm0<G::XI + G::WIL>();
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int u = 0; u < TN; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Software pipeline over 16-row batch tiles: the scale FMAs of a tile's
    // MFMA results are issued two tiles later (between the MFMAs of that
    // tile), when those results are complete, so the VALU work of a wave runs
    // while its own MFMAs execute.  Steps s = (block in stage) * TM + t use
    // result slot s % 4 (TM * KC is a multiple of 4, so the slots repeat per
    // stage); sP: the scales of the previous block, whose last two tiles are
    // pending when a block starts.
    static_assert(TM % 2 == 0 && (TM * KC) % 4 == 0, "result ring");
    f32x4 dR[4][TN];
    float sP[TN];
#pragma unroll
    for (int u = 0; u < TN; u++) {
#pragma unroll
        for (int q = 0; q < 4; q++) dR[q][u] = f32x4{0.f, 0.f, 0.f, 0.f};
        sP[u] = 0.f;
    }
    auto compute = [&](auto bsel, int c) {
        const uint8_t* buf = qg_stage<decltype(bsel)::value, G::SMALL>();
        const int cb = b_begin + c * KC;
        // one block at a time where the slots do not depend on the block
        // (unrolled over blocks, the scheduler hoists both blocks' fragment
        // reads and spills)
        constexpr int UJ = TM % 4 == 0 ? 1 : KC;
#pragma unroll UJ
        for (int j = 0; j < KC; j++) {
            if (cb + j >= b_end) {  // uniform: past the split's range (stage padding)
#pragma unroll
                for (int t = 0; t < 2; t++)  // only the previous block's pending tiles
#pragma unroll
                    for (int u = 0; u < TN; u++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            acc[TM - 2 + t][u][r] =
                                __builtin_fmaf(dR[(j * TM + t + 2) & 3][u][r], sP[u], acc[TM - 2 + t][u][r]);
#pragma unroll
                for (int u = 0; u < TN; u++) sP[u] = 0.f;  // later pending reads add nothing
                continue;
            }
            bf16x8 wf[TN];
            f16x8 wh[TN];
            float sc[TN];
#pragma unroll
            for (int u = 0; u < TN; u++) {
                const uint8_t* tb = buf + 2 * G::XPL + ((wn * TN + u) * KC + j) * TB;
                WRaw<FMT> r;
                if (FMT == 8) {
                    r.scale = *(const uint32_t*)(tb + 4 * l16);
                    const uint2 q = *(const uint2*)(tb + 64 + 32 * l16 + 8 * seg);
                    reinterpret_cast<uint32_t*>(&r)[1] = q.x;
                    reinterpret_cast<uint32_t*>(&r)[2] = q.y;
                } else {
                    r.scale = *(const uint16_t*)(tb + 2 * l16);
                    reinterpret_cast<uint32_t*>(&r)[1] = *(const uint32_t*)(tb + 32 + 16 * l16 + 4 * seg);
                }
                convert<FMT>(r, wf[u], wh[u], sc[u]);
            }
            // The block's MFMAs at raised wave priority: the SIMD's other wave,
            // in its own weight conversion or LDS reads, issues into their gaps
            // (MI355X, Q4 at 128 rows, GEMM + partial sums: 11008 x 2048
            // 30.9 -> 30.0 us, 2048 x 11008 28.0 -> 26.6 us)
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int t = 0; t < TM; t++) {
                const int row = (wm * TM + t) * 16 + l16;
                const int slot = (4 * j + seg) ^ (row & 7);
                const bf16x8 ah = *(const bf16x8*)(buf + row * G::XROW + 16 * slot);
                const f16x8 al = *(const f16x8*)(buf + G::XPL + row * G::XROW + 16 * slot);
                const int q = (j * TM + t) & 3, pq = (q + 2) & 3;  // this step's slot, the pending one's
                const int pt = t >= 2 ? t - 2 : TM - 2 + t;         // pending tile
#pragma unroll
                for (int u = 0; u < TN; u++) {
                    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wf[u], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    dR[q][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, wh[u], d, 0, 0, 0);
                    const float ps = t >= 2 ? sc[u] : sP[u];
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[pt][u][r] = __builtin_fmaf(dR[pq][u][r], ps, acc[pt][u][r]);
                }
            }
            __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int u = 0; u < TN; u++) sP[u] = sc[u];
        }
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    issue(B0{}, 0);
    issue(B1{}, 1);
    for (int c = 0; c < nstages; c += 3) {
        wait_stage();
        lds_barrier();
        issue(B2{}, c + 2);
        compute(B0{}, c);
        wait_stage();
        lds_barrier();
        issue(B0{}, c + 3);
        compute(B1{}, c + 1);
        wait_stage();
        lds_barrier();
        issue(B1{}, c + 4);
        compute(B2{}, c + 2);
    }
    wait_vm_lgkm0<0>();  // drain the past-the-end stages before the workgroup exits
#pragma unroll
    for (int u = 0; u < TN; u++)  // the last block's last two tiles (slots 2, 3)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            acc[TM - 2][u][r] = __builtin_fmaf(dR[2][u][r], sP[u], acc[TM - 2][u][r]);
            acc[TM - 1][u][r] = __builtin_fmaf(dR[3][u][r], sP[u], acc[TM - 1][u][r]);
        }

    if (act_hi) {
        // SwiGLU front (mlp_forward, attention.cpp:172-178) on complete sums of
        // interleaved rows (2i = gate_i, 2i+1 = up_i), written as the hi/lo
        // planes [M][N/2] of the next GEMM.  The two lanes of a pair exchange
        // their 4 sums; the even lane writes batch rows r = 0, 1 of its 4 and
        // the odd lane rows 2, 3.
        const int F2 = N >> 1;
        const bool odd = l16 & 1;
        const bool full = m0 + (wm + 1) * TM * 16 <= M && n0 + (wn + 1) * TN * 16 <= N;  // uniform
#pragma unroll
        for (int t = 0; t < TM; t++) {
#pragma unroll
            for (int u = 0; u < TN; u++) {
                const int n2 = (n0 + (wn * TN + u) * 16 + l16) >> 1;  // the pair's output column
                float p[4];
#pragma unroll
                for (int r = 0; r < 4; r++) p[r] = __shfl_xor(acc[t][u][r], 1);
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const float g = odd ? p[2 + k] : acc[t][u][k];
                    const float up = odd ? acc[t][u][2 + k] : p[k];
                    const int m = m0 + (wm * TM + t) * 16 + seg * 4 + (odd ? 2 + k : k);
                    if (full || (m < M && 2 * n2 < N)) {
                        const size_t e = (size_t)m * F2 + n2;
                        split_bf16(silu_gate(g, up), &act_hi[e], &act_lo[e]);
                    }
                }
            }
        }
        return;
    }
    if constexpr (AMAX) {
        // greedy head (Sampler::argmax, sampler.cpp:25-35) on complete sums:
        // per batch row, the workgroup's largest logit as an argmax_key, written
        // to amax[tile][m] (no split, no stream-K: the launcher guarantees it).
        // Each lane takes the best of its TN columns; a prefix max over the
        // 16 lanes of a DPP row (the lanes that share the row's batch rows,
        // row_shr 1, 2, 4, 8, all 4*TM keys interleaved) leaves the 16
        // columns' best in lane 15; the WN waves then meet in stage buffer 0,
        // free once every wave has drained its loads and passed the barrier.
        uint64_t* keys = (uint64_t*)qg_stage<0, G::SMALL>();
        static_assert(WN * MW * 8 <= QG_STAGE_SMALL, "argmax keys must fit a stage buffer");
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TM; t++) {
            uint64_t best[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                best[r] = 0;
#pragma unroll
                for (int u = 0; u < TN; u++) {
                    const int n = n0 + (wn * TN + u) * 16 + l16;
                    const uint64_t k = n < N ? argmax_key(acc[t][u][r], (uint32_t)n) : 0;
                    best[r] = k > best[r] ? k : best[r];
                }
            }
            key_row_max<0x111>(best);
            key_row_max<0x112>(best);
            key_row_max<0x114>(best);
            key_row_max<0x118>(best);
            if (l16 == 15)
#pragma unroll
                for (int r = 0; r < 4; r++) keys[wn * MW + (wm * TM + t) * 16 + seg * 4 + r] = best[r];
        }
        __syncthreads();
        for (int i = tid; i < MW; i += 64 * NWV) {
            if (m0 + i >= M) break;
            uint64_t b = 0;
#pragma unroll
            for (int w = 0; w < WN; w++) {
                const uint64_t k = keys[w * MW + i];
                b = k > b ? k : b;
            }
            amax[(size_t)blockIdx.x * M + m0 + i] = b;
        }
        return;
    }
    // epilogue: direct (+ residual) or a partial tile
    store_tiles<TM, TN>(acc, dst, addp, M, N, m0 + wm * TM * 16, n0 + wn * TN * 16, seg, l16);
    };  // segment

    if constexpr (!SK) {  // uniform split: workgroup (tile, split, batch chunk)
        const int b_begin = blockIdx.y * bps;  // bps: a positive multiple of KC
        segment(blockIdx.x * NW, blockIdx.z * MW, b_begin, min(nb, b_begin + bps),
                part ? part + (size_t)blockIdx.y * M * N : Y, part ? nullptr : add);
        return;
    } else {
    // stream-K: this workgroup's equal share of the (tile, block) pairs, one
    // segment per tile it touches; segment k of a tile writes partial slice k
    // (or Y itself when no tile is shared, skS == 1), and the tile's last
    // segment zeroes the slices past the tile's segment count
    const long long T = (long long)sk_ntiles * ((M + MW - 1) / MW) * nb;
    const int w = blockIdx.x;
    long long lo = (long long)w * T / skG;
    const long long hi = (long long)(w + 1) * T / skG;
    while (lo < hi) {
        const long long u = lo / nb;
        const int b0 = (int)(lo % nb);
        const int b1 = (int)min((long long)nb, b0 + (hi - lo));
        const int tile = (int)(u % sk_ntiles), mc = (int)(u / sk_ntiles);
        const int first = sk_owner(u * nb, T, skG);
        const int k = w - first, nseg = sk_owner(u * nb + nb - 1, T, skG) - first + 1;
        lds_barrier();  // every wave is done with the stage buffers of the previous segment
        if (!part) {  // no tile is shared (skS == 1)
            segment(tile * NW, mc * MW, b0, b1, Y, add);
        } else {
            segment(tile * NW, mc * MW, b0, b1, part + (size_t)k * M * N, nullptr);
            if (k == nseg - 1) {
                for (int sl = nseg; sl < skS; sl++) {
                    float* z = part + (size_t)sl * M * N;
#pragma unroll
                    for (int t = 0; t < TM; t++)
#pragma unroll
                        for (int uu = 0; uu < TN; uu++) {
                            const int n = tile * NW + (wn * TN + uu) * 16 + l16;
#pragma unroll
                            for (int r = 0; r < 4; r++) {
                                const int m = mc * MW + (wm * TM + t) * 16 + seg * 4 + r;
                                if (m < M && n < N) z[(size_t)m * N + n] = 0.f;
                            }
                        }
                }
            }
        }
        lo += b1 - b0;
    }
    }
}

// ---------------------------------------------------------------------------
// Row-split GEMM with LDS-shared activations (qgemm_kx_kernel): tile-major
// weights, 128-row batch chunks.
//
// A workgroup (4 waves) owns 4R weight tiles (64R rows) x 16T batch rows over
// a range of quant blocks; wave w computes tiles 4R.. of its own R tiles for
// all 16T batch rows, so each X fragment it reads feeds R weight tiles and
// each converted weight fragment T batch tiles.  X and the weights come
// through a 3-stage LDS ring filled by direct-to-LDS loads, KC quant blocks a
// stage: X fragment-major (one 1 KB load instruction = one 16x32 fragment of
// one plane, lane l's 16 bytes at lane offset 16 l, so the MFMA operand reads
// are conflict-free without a swizzle), the 4R tile-blocks of each block in
// the tile-major order.  One barrier per stage, after the wave's own loads of
// the stage have landed; stages c+1 and c+2 stay in flight while c computes.
// Epilogue as the other tiled kernels: Y (+ add), a partial slice, or the
// SwiGLU front of interleaved gate/up rows.
// ---------------------------------------------------------------------------
template <int FMT, int R, int T, int KC>
struct KxGeom {
    static constexpr int TB = tile_block_bytes(FMT);
    static constexpr int SB = FMT == 8 ? 4 : 2, QB = FMT == 8 ? 32 : 16;
    static constexpr int XI = KC * 2 * T;               // X load instructions per stage (1 KB each)
    static constexpr int XW = XI / 4;                   // ... per wave
    static constexpr int WBYTES = KC * 4 * R * TB;      // weight bytes per stage
    static constexpr int WI = (WBYTES + 1023) / 1024;   // weight load instructions per stage
    static constexpr int WL = WI / 4, WEXTRA = WI % 4;  // waves < WEXTRA issue WL + 1
    static constexpr int XBYTES = XI * 1024;
    static constexpr int STAGE = XBYTES + WI * 1024;
    static_assert(XI % 4 == 0, "X stage must split evenly over the 4 waves");
};
constexpr int KX_STAGE_MAX = 24576;  // Q8_0, R = 3, T = 8, KC = 1: 16 KB of X + 7 KB of weights
__shared__ __align__(16) uint8_t kx_s0[KX_STAGE_MAX];
__shared__ __align__(16) uint8_t kx_s1[KX_STAGE_MAX];
__shared__ __align__(16) uint8_t kx_s2[KX_STAGE_MAX];
template <int B>
__device__ __forceinline__ uint8_t* kx_stage() {
    return B == 0 ? kx_s0 : B == 1 ? kx_s1 : kx_s2;
}

// part != nullptr: split-K partial slice blockIdx.y of [S][M][N]; act_hi: SwiGLU planes (one split)
template <int FMT, int R, int T, int KC>
__global__ __launch_bounds__(256, 2) void qgemm_kx_kernel(const uint8_t* __restrict__ Wt, int N, int nb,
                                                          const uint16_t* __restrict__ xh,
                                                          const uint16_t* __restrict__ xl, int K, int M, float* Y,
                                                          const float* add, int bps, float* __restrict__ part,
                                                          uint16_t* __restrict__ act_hi,
                                                          uint16_t* __restrict__ act_lo) {
    using G = KxGeom<FMT, R, T, KC>;
    static_assert(G::STAGE <= KX_STAGE_MAX, "stage buffer too small");
    static_assert(T % 2 == 0, "the result ring alternates between two batch tiles");
    constexpr int TB = G::TB;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int seg = lane >> 4, l16 = lane & 15;
    const int ntile16 = (N + 15) / 16;
    const int n0 = blockIdx.x * 64 * R, m0 = blockIdx.z * 16 * T;
    const int b_begin = blockIdx.y * bps, b_end = min(nb, b_begin + bps);
    const bool wextra = wave < G::WEXTRA;
    const uint32_t xbytes = (uint32_t)((size_t)M * K * 2);
    const v4i xrs[2] = {make_rsrc_words(xh, xbytes), make_rsrc_words(xl, xbytes)};
    const v4i wrs = make_rsrc_words(Wt, (uint32_t)min((size_t)ntile16 * nb * TB, (size_t)0xFFFFFFFFu));

    // per-lane source offsets of this wave's load instructions (a stage's first
    // block adds cb * 64 (X) or cb * TB (weights))
    uint32_t xo[G::XW];
#pragma unroll
    for (int i = 0; i < G::XW; i++) {
        const int q = wave + 4 * i;  // ((kc * 2 + plane) * T + t)
        const int t = q % T, kc = q / (2 * T);
        const int row = min(m0 + 16 * t + l16, M - 1);
        xo[i] = (uint32_t)((size_t)row * K * 2) + 64u * kc + 16u * seg;
    }
    uint32_t wo[G::WL + 1];
#pragma unroll
    for (int i = 0; i <= G::WL; i++) {
        const int f = min((wave + 4 * i) * 1024 + 16 * lane, G::WBYTES - 16);  // bytes past the stage re-read the last piece
        const int kc = f / (4 * R * TB), rem = f % (4 * R * TB);
        const int j = rem / TB, off = rem % TB;
        const int tile = min((int)blockIdx.x * 4 * R + j, ntile16 - 1);
        wo[i] = (uint32_t)((size_t)tile * nb * TB) + (uint32_t)(kc * TB + off);
    }
    auto issue = [&](auto bsel, int c) {
        uint8_t* buf = kx_stage<decltype(bsel)::value>();
        const int cb = min(b_begin + c * KC, b_end - 1);  // stages past the range re-read a valid block
#pragma unroll
        for (int i = 0; i < G::XW; i++) {
            const int q = wave + 4 * i;
            const int plane = (q / T) & 1;  // wave-uniform
            dma16(xrs[plane], xo[i] + (uint32_t)cb * 64u, buf + q * 1024);
        }
#pragma unroll
        for (int i = 0; i < G::WL; i++) dma16(wrs, wo[i] + (uint32_t)cb * TB, buf + G::XBYTES + (wave + 4 * i) * 1024);
        if (G::WEXTRA && wextra)
            dma16(wrs, wo[G::WL] + (uint32_t)cb * TB, buf + G::XBYTES + (wave + 4 * G::WL) * 1024);
    };
    // this wave's loads of the oldest stage in flight have landed (one stage may remain outstanding)
    auto wait_stage = [&]() {
        if (wextra) wait_vm_lgkm0<G::XW + G::WL + 1>();
        else wait_vm_lgkm0<G::XW + G::WL>();
    };

    f32x4 acc[T][R];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int u = 0; u < R; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 dR[2][R];  // MFMA results of the previous and current batch tile
    float sP[R];     // scales of the previous block (its last tile is pending when a block starts)
#pragma unroll
    for (int u = 0; u < R; u++) {
        dR[0][u] = dR[1][u] = f32x4{0.f, 0.f, 0.f, 0.f};
        sP[u] = 0.f;
    }
    auto compute = [&](auto bsel, int c) {
        const uint8_t* buf = kx_stage<decltype(bsel)::value>();
        const int cb = b_begin + c * KC;
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            if (cb + kc >= b_end) break;  // uniform: past the split's range (stage padding)
            bf16x8 wf[R];
            f16x8 wh[R];
            float sc[R];
#pragma unroll
            for (int u = 0; u < R; u++) {
                const uint8_t* tb = buf + G::XBYTES + (kc * 4 * R + wave * R + u) * TB;
                WRaw<FMT> r;
                if (FMT == 8) {
                    r.scale = *(const uint32_t*)(tb + 4 * l16);
                    const uint2 q = *(const uint2*)(tb + 64 + 32 * l16 + 8 * seg);
                    reinterpret_cast<uint32_t*>(&r)[1] = q.x;
                    reinterpret_cast<uint32_t*>(&r)[2] = q.y;
                } else {
                    r.scale = *(const uint16_t*)(tb + 2 * l16);
                    reinterpret_cast<uint32_t*>(&r)[1] = *(const uint32_t*)(tb + 32 + 16 * l16 + 4 * seg);
                }
                convert<FMT>(r, wf[u], wh[u], sc[u]);
            }
            const uint8_t* xa = buf + (kc * 2 * T) * 1024 + 16 * lane;
#pragma unroll
            for (int t = 0; t < T; t++) {
                const bf16x8 ah = *(const bf16x8*)(xa + t * 1024);
                const f16x8 al = *(const f16x8*)(xa + (T + t) * 1024);
                const int q = t & 1, pq = q ^ 1;
                const int pt = t > 0 ? t - 1 : T - 1;
#pragma unroll
                for (int u = 0; u < R; u++) {
                    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wf[u], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    dR[q][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, wh[u], d, 0, 0, 0);
                }
#pragma unroll
                for (int u = 0; u < R; u++) {
                    const float ps = t > 0 ? sc[u] : sP[u];
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[pt][u][r] = __builtin_fmaf(dR[pq][u][r], ps, acc[pt][u][r]);
                }
                // issue order of the tile: its X fragment reads, then each of its
                // 2R MFMAs followed by two of the pending tile's 4R scale FMAs, so
                // the wave's VALU work runs in the shadow of its own MFMAs
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
                for (int i = 0; i < 2 * R; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int u = 0; u < R; u++) sP[u] = sc[u];
        }
    };

    const int nstages = ((b_end - b_begin + KC - 1) / KC + 2) / 3 * 3;  // whole trips of the 3-stage loop
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    issue(B0{}, 0);
    issue(B1{}, 1);
    for (int c = 0; c < nstages; c += 3) {
        wait_stage();
        lds_barrier();
        issue(B2{}, c + 2);
        compute(B0{}, c);
        wait_stage();
        lds_barrier();
        issue(B0{}, c + 3);
        compute(B1{}, c + 1);
        wait_stage();
        lds_barrier();
        issue(B1{}, c + 4);
        compute(B2{}, c + 2);
    }
    wait_vm_lgkm0<0>();  // drain the past-the-end stages before any other memory access
#pragma unroll
    for (int u = 0; u < R; u++)  // the last block's last tile
#pragma unroll
        for (int r = 0; r < 4; r++) acc[T - 1][u][r] = __builtin_fmaf(dR[(T - 1) & 1][u][r], sP[u], acc[T - 1][u][r]);

    const int nw = n0 + wave * R * 16;  // this wave's first weight row
    if (act_hi) {
        // SwiGLU front (mlp_forward, attention.cpp:172-178) on interleaved rows
        // (2i = gate_i, 2i+1 = up_i): the two lanes of a pair exchange their 4
        // sums; the even lane writes batch rows 0, 1 of its 4, the odd lane 2, 3
        const int F2 = N >> 1;
        const bool odd = l16 & 1;
#pragma unroll
        for (int t = 0; t < T; t++) {
#pragma unroll
            for (int u = 0; u < R; u++) {
                const int n2 = (nw + u * 16 + l16) >> 1;
                float pv[4];
#pragma unroll
                for (int r = 0; r < 4; r++) pv[r] = __shfl_xor(acc[t][u][r], 1);
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const float g = odd ? pv[2 + k] : acc[t][u][k];
                    const float up = odd ? acc[t][u][2 + k] : pv[k];
                    const int m = m0 + t * 16 + seg * 4 + (odd ? 2 + k : k);
                    if (m < M && 2 * n2 < N) {
                        const size_t e = (size_t)m * F2 + n2;
                        split_bf16(silu_gate(g, up), &act_hi[e], &act_lo[e]);
                    }
                }
            }
        }
        return;
    }
    float* dst = part ? part + (size_t)blockIdx.y * M * N : Y;
    store_tiles<T, R>(acc, dst, part ? nullptr : add, M, N, m0, nw, seg, l16);
}

// ---------------------------------------------------------------------------
// Wave-split GEMM for tile-major weights (qgemm_kw_kernel): batches of up to
// 128 rows per workgroup.
//
// A workgroup owns R weight tiles (16R rows) x 16T batch rows over a range of
// quant blocks; its 4 waves take the range's blocks in turn (wave w: blocks
// b0 + w, b0 + w + 4, ...) and every wave computes the whole 16R x 16T tile
// for its blocks.  Weight fragments and X fragments are loaded by each wave
// straight into registers (weights three blocks ahead in a register ring, X
// fragments reloaded for the next block right after their MFMAs), so the
// main loop holds no LDS access and no barrier: a wave
// waits only on its own loads.  Each converted weight fragment feeds T batch
// tiles; each X fragment feeds R weight tiles.  The scale FMAs of a batch
// tile issue after the next tile's MFMAs, when its results are complete.
// At the end the four waves' sums meet in LDS and are added in wave order
// ((w0 + w1) + w2) + w3, a fixed order: a result does not depend on
// scheduling.  The epilogue stores coalesced rows of the tile: Y (+ add),
// a partial slice, or the SwiGLU front of interleaved gate/up rows written as
// the next GEMM's hi/lo planes.
// ---------------------------------------------------------------------------
constexpr int KW_WAVES = 4;

template <int FMT, int R, int T>
struct KwGeom {
    static constexpr int TB = tile_block_bytes(FMT);
    static constexpr int SB = FMT == 8 ? 4 : 2, QB = FMT == 8 ? 32 : 16;
    // result tiles per wave per reduction pass: the largest divisor of T with
    // R * TC <= 32 (at most 128 KB of LDS)
    static constexpr int TC = (R * T <= 32) ? T : (R * (T / 2) <= 32) ? T / 2 : (R * (T / 4) <= 32) ? T / 4 : 1;
    static_assert(T % TC == 0 && R * TC <= 32, "reduction pass");
    static constexpr size_t LDS = (size_t)KW_WAVES * R * TC * 64 * 16;
    // two workgroups per CU where the registers (<= 256 per lane) and the LDS allow
    static constexpr int MINB = (R * T <= 16 && 2 * LDS <= 160 * 1024) ? 2 : 1;
};

// mode 0: Y[m][n] (+ add[m][n]) of the split's sums, Y offset by blockIdx.y * slice
// (slice = M*N for split-K partials, 0 for a single split); mode 1: SwiGLU front
// of interleaved gate/up rows (2i = gate_i, 2i+1 = up_i) written as the hi/lo planes
// act_hi/act_lo [M][N/2] (one split only).  Dynamic LDS: KwGeom::LDS bytes.
template <int FMT, int R, int T>
__global__ __launch_bounds__(256, (KwGeom<FMT, R, T>::MINB)) void qgemm_kw_kernel(
    const uint8_t* __restrict__ Wt, int N, int nb, const uint16_t* __restrict__ xh, const uint16_t* __restrict__ xl,
    int K, int M, int bps, float* Y, const float* add, size_t slice, int mode, uint16_t* __restrict__ act_hi,
    uint16_t* __restrict__ act_lo) {
    using G = KwGeom<FMT, R, T>;
    constexpr int TB = G::TB;
    extern __shared__ __align__(16) f32x4 kw_red[];
    static_assert(T % 2 == 0, "the result ring alternates between two batch tiles");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int seg = lane >> 4, l16 = lane & 15;
    const int ntile16 = (N + 15) / 16;
    const int n0 = blockIdx.x * 16 * R, m0 = blockIdx.z * 16 * T;
    const int b0 = blockIdx.y * bps, b1 = min(nb, b0 + bps);
    const int nblk = b1 - b0 > wave ? (b1 - b0 - wave + KW_WAVES - 1) / KW_WAVES : 0;  // this wave's blocks

    const rsrc_t wrs = make_rsrc(Wt, (uint32_t)min((size_t)ntile16 * nb * TB, (size_t)0xFFFFFFFFu));
    const uint32_t xbytes = (uint32_t)((size_t)M * K * 2);
    const rsrc_t xrh = make_rsrc(xh, xbytes), xrl = make_rsrc(xl, xbytes);
    // lane offsets: the scale and 8 quants of row l16 within a tile-block; X row
    // m0 + 16t + l16 (clamped), elements 8*seg.. of a block
    const uint32_t wsc = (uint32_t)(G::SB * l16), wqo = (uint32_t)(16 * G::SB + G::QB * l16 + (G::QB / 4) * seg);
    const uint32_t xo0 = (uint32_t)((size_t)min(m0 + l16, M - 1) * K * 2) + 16u * seg;
    auto xoff = [&](int t) {  // X row offset of batch tile t (rows past M read row M - 1)
        return t == 0 ? xo0 : (uint32_t)((size_t)min(m0 + 16 * t + l16, M - 1) * K * 2) + 16u * seg;
    };
    uint32_t tbase[R];  // uniform: byte offset of each weight tile's first tile-block
#pragma unroll
    for (int u = 0; u < R; u++) tbase[u] = (uint32_t)((size_t)min((int)blockIdx.x * R + u, ntile16 - 1) * nb * TB);

    // block of this wave's i-th step (clamped for the loads past the end)
    auto blk = [&](int i) { return b0 + wave + KW_WAVES * min(i, max(nblk - 1, 0)); };
    auto load_w = [&](WRaw<FMT>(&wr)[R], int i) {
        const uint32_t k = (uint32_t)blk(i);
#pragma unroll
        for (int u = 0; u < R; u++) load_tiled<FMT>(wrs, wsc, wqo, tbase[u] + k * TB, wr[u]);
    };
    u32x4 xa[T], xb[T];  // X fragments of the current block; tile t reloads for the next block after its MFMAs
    auto load_xt = [&](int t, int i) {
        const uint32_t koff = (uint32_t)blk(i) * 64u, o = xoff(t);
        xa[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrh, o, koff, 0));
        xb[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrl, o, koff, 0));
    };

    f32x4 acc[T][R];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int u = 0; u < R; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 dR[2][R];  // MFMA results of the previous and current batch tile
    float sP[R];     // scales of the previous block (its last tile is pending when a block starts)
#pragma unroll
    for (int u = 0; u < R; u++) {
        dR[0][u] = dR[1][u] = f32x4{0.f, 0.f, 0.f, 0.f};
        sP[u] = 0.f;
    }

    // Weight ring: the raw fragments of steps i .. i+3 (the loads of step i + 3
    // are requested when step i begins), rotated by register moves.
    WRaw<FMT> w0[R], w1[R], w2[R];
    load_w(w0, 0);
    load_w(w1, 1);
    load_w(w2, 2);
#pragma unroll
    for (int t = 0; t < T; t++) load_xt(t, 0);
    for (int i = 0; i < nblk; i++) {
        WRaw<FMT> w3[R];
        load_w(w3, i + 3);
        __builtin_amdgcn_sched_barrier(0);
        // convert the weights of step i; per batch tile t the MFMAs, the reload
        // of its X fragment with block i + 1, the scale FMAs of tile t - 1 (of
        // the previous block for t = 0)
        bf16x8 wf[R];
        f16x8 wh[R];
        float sc[R];
#pragma unroll
        for (int u = 0; u < R; u++) convert<FMT>(w0[u], wf[u], wh[u], sc[u]);
#pragma unroll
        for (int t = 0; t < T; t++) {
            const bf16x8 ah = __builtin_bit_cast(bf16x8, xa[t]);
            const f16x8 al = __builtin_bit_cast(f16x8, xb[t]);
            const int q = t & 1, pq = q ^ 1;
            const int pt = t > 0 ? t - 1 : T - 1;
#pragma unroll
            for (int u = 0; u < R; u++) {
                const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, wf[u], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                dR[q][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, wh[u], d, 0, 0, 0);
            }
            load_xt(t, i + 1);
#pragma unroll
            for (int u = 0; u < R; u++) {
                const float ps = t > 0 ? sc[u] : sP[u];
#pragma unroll
                for (int r = 0; r < 4; r++) acc[pt][u][r] = __builtin_fmaf(dR[pq][u][r], ps, acc[pt][u][r]);
            }
            // keep each tile's reload behind its MFMAs (hoisted reloads would
            // hold a second block of X fragments in registers)
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int u = 0; u < R; u++) {
            sP[u] = sc[u];
            w0[u] = w1[u];
            w1[u] = w2[u];
            w2[u] = w3[u];
        }
    }
    // the last block's last tile (a wave without blocks adds zeros)
#pragma unroll
    for (int u = 0; u < R; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[T - 1][u][r] = __builtin_fmaf(dR[(T - 1) & 1][u][r], sP[u], acc[T - 1][u][r]);

    // ---- reduction over the waves and epilogue, TC batch tiles per pass
    constexpr int TC = G::TC;
    float* dst = mode == 0 ? Y + (size_t)blockIdx.y * slice : nullptr;
    const int F2 = N >> 1;
#pragma unroll
    for (int t0 = 0; t0 < T; t0 += TC) {
        if (t0) __syncthreads();  // the previous pass's reads are done
#pragma unroll
        for (int tt = 0; tt < TC; tt++)
#pragma unroll
            for (int u = 0; u < R; u++) kw_red[((wave * TC + tt) * R + u) * 64 + lane] = acc[t0 + tt][u];
        __syncthreads();
        if (mode == 0) {
            // unit j: (tile tt, segment sg, weight tile u, row c16): 4 batch rows of one column
            for (int j = tid; j < TC * 4 * R * 16; j += 256) {
                const int c16 = j & 15, u = (j >> 4) % R, sg = (j / (16 * R)) & 3, tt = j / (64 * R);
                const int e = (tt * R + u) * 64 + sg * 16 + c16;
                f32x4 v = kw_red[e];
#pragma unroll
                for (int w = 1; w < KW_WAVES; w++) v += kw_red[w * TC * R * 64 + e];
                const int n = n0 + 16 * u + c16;
                if (n < N) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int m = m0 + 16 * (t0 + tt) + 4 * sg + r;
                        if (m < M) {
                            const size_t o = (size_t)m * N + n;
                            dst[o] = add ? v[r] + add[o] : v[r];
                        }
                    }
                }
            }
        } else {
            // unit j: (tile tt, segment sg, weight tile u, pair p): the gate row
            // 16u + 2p and the up row 16u + 2p + 1 of 4 batch rows
            for (int j = tid; j < TC * 4 * R * 8; j += 256) {
                const int p = j & 7, u = (j >> 3) % R, sg = (j / (8 * R)) & 3, tt = j / (32 * R);
                const int e = (tt * R + u) * 64 + sg * 16 + 2 * p;
                f32x4 g = kw_red[e], up = kw_red[e + 1];
#pragma unroll
                for (int w = 1; w < KW_WAVES; w++) {
                    g += kw_red[w * TC * R * 64 + e];
                    up += kw_red[w * TC * R * 64 + e + 1];
                }
                const int c = (n0 + 16 * u) / 2 + p;
                if (2 * c < N) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int m = m0 + 16 * (t0 + tt) + 4 * sg + r;
                        if (m < M) {
                            const size_t o = (size_t)m * F2 + c;
                            split_bf16(silu_gate(g[r], up[r]), &act_hi[o], &act_lo[o]);
                        }
                    }
                }
            }
        }
    }
}

// Y = sum_{s < S} part[s] (+ add), in split order.
__global__ __launch_bounds__(256) void qgemm_reduce_kernel(const float* __restrict__ part, int S, size_t MN, float* Y,
                                                           const float* add) {
    const size_t n4 = MN / 4;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        f32x4 v = ((const f32x4*)part)[i];
        for (int s = 1; s < S; s++) {
            const f32x4 p = ((const f32x4*)(part + (size_t)s * MN))[i];
            v[0] += p[0];
            v[1] += p[1];
            v[2] += p[2];
            v[3] += p[3];
        }
        if (add) {
            const f32x4 a = ((const f32x4*)add)[i];
            v[0] += a[0];
            v[1] += a[1];
            v[2] += a[2];
            v[3] += a[3];
        }
        ((f32x4*)Y)[i] = v;
    }
    for (size_t i = n4 * 4 + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN;
         i += (size_t)gridDim.x * blockDim.x) {
        float v = part[i];
        for (int s = 1; s < S; s++) v += part[(size_t)s * MN + i];
        if (add) v += add[i];
        Y[i] = v;
    }
}

int launch_reduce_slices(const float* part, int S, size_t MN, float* Y, const float* add, hipStream_t s) {
    const int rgrid = (int)min((MN / 4 + 255) / 256 + 1, (size_t)2048);
    hipLaunchKernelGGL(qgemm_reduce_kernel, dim3(rgrid), dim3(256), 0, s, part, S, MN, Y, add);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

struct QgPlan {
    int WM, WN, TM, TN, KC, MW, NW, ntiles, mchunks, S, bps;
    bool pipe;  // qgemm_pipe_kernel (tile-major weights, batch tiles over 32 rows)
    int kwR, kwT;  // kwR > 0: qgemm_kw_kernel<FMT, kwR, kwT> (tile-major weights)
    int kxT;       // > 0: qgemm_kx_kernel<FMT, 3, kxT, 1> (tile-major weights)
    int skG;    // > 0: stream-K over skG workgroups (pipelined kernel only); S = the slices a tile may need
    size_t ws_bytes;
};

// Tuning overrides (qraf_hip_set_qgemm_tuning): 0 = automatic.
static int g_qg_waves = 0;   // 4 or 8 waves per workgroup for batch tiles > 32 rows
static int g_qg_splits = 0;  // forced split count
static int g_qg_pipe = 0;    // 1: pipelined kernel for every tiled batch over 32 rows, 2: its narrow
                             // 4-wave form, -1: never
static int g_qg_mchunk = 0;  // batch rows per workgroup at most (0: QG_MCHUNK)
static int g_qg_sched = 0;   // pipelined kernel: 0 automatic (the uniform split), 1 stream-K, 2 uniform split
static int g_qg_skmin = 0;   // stream-K: quant blocks per workgroup at least (0: 16)
static int g_qg_kw = 0;      // wave-split kernel: 0 automatic, 1 for every tiled batch over 16 rows, -1 never
static int g_qg_kwR = 0;     // wave-split kernel: weight tiles per workgroup (0: automatic, else 2, 3 or 4)

static int qg_cu_count() {
    static int n = 0;
    if (!n) {
        int d = 0;
        hipDeviceProp_t pr;
        if (hipGetDevice(&d) == hipSuccess && hipGetDeviceProperties(&pr, d) == hipSuccess) n = pr.multiProcessorCount;
        if (n <= 0) n = 256;
    }
    return n;
}

// Stream-K for a pipelined plan (g_qg_sched == 1): `slots` workgroups
// resident at once, each an equal share of the (tile, block) pairs (at least
// g_qg_skmin blocks), so every CU gets the same work whatever the tile count;
// S becomes the most segments any tile has.  Not the automatic choice: on
// MI355X at the continuous-batch shapes (128 rows) it was slower than the
// uniform grid (Q4 11008 x 2048: 37.6 against 33.0 us; a 128-sequence decode
// step 6.34 against 5.96 ms), since shares of 11-21 blocks pay a pipeline
// prologue per segment and more partial slices than the balance saves.
static void qgemm_stream(QgPlan& p, int nb, int slots) {
    if (g_qg_sched != 1 || g_qg_splits > 0) return;
    const long long units = (long long)p.ntiles * p.mchunks, T = units * nb;
    const int minb = g_qg_skmin > 0 ? g_qg_skmin : 16;
    const int G = (int)std::max(1LL, std::min((long long)slots, T / minb));
    int smax = 1;
    for (long long u = 0; u < units; u++)
        smax = std::max(smax, sk_owner(u * nb + nb - 1, T, G) - sk_owner(u * nb, T, G) + 1);
    p.skG = G;
    p.S = smax;
}

// The wave-split kernel for a tiled N x K product of M rows.  Automatic
// choice (MI355X, Q4_0 and Q8_0 at the Qwen2.5-3B shapes, GEMM + partial sums,
// graph-timed): batches of 17-32 rows on every shape (Q4 11008 x 2048 14.8 us
// against 20.8 for the 32-row-chunk kernel, 2048 x 2048 8.3 against 12.2) and
// of 33-64 rows below 16384 weight rows (11008 x 2048 23.0 against 25.7, 2048 x
// 11008 22.7 against 28.9); from 65 rows, and for the 22016-row gate/up
// product at 33-64 rows (42.1 against 37.4), the LDS-shared pipelined kernels,
// whose X fragments each feed 8 waves (here each wave reads its own: 5x the X
// bytes per MFMA at 128 rows, 40-83 us against 29-49).
static bool kw_wanted(int N, int M) {
    if (g_qg_kw < 0 || (g_qg_pipe != 0 && g_qg_kw == 0)) return false;  // an older form forced
    if (g_qg_kw > 0) return M > 16;
    return M > 16 && (M <= 32 || (M <= 64 && N < 16384));
}

// Wave-split plan: batch tiles T = 2, 4 or 8 (chunks of up to 128 rows),
// R = 2, 3 or 4 weight tiles per workgroup and S splits of the quant blocks,
// chosen for the fewest rounds of workgroups (one per CU) x the time of one,
// modelled as (steps per wave) x (R + 2) + 3R: a step costs its R tiles'
// MFMAs plus a fixed part (X loads, FMAs), the reduction and stores about 3
// steps per weight tile (fitted to the measured best R on the Qwen2.5-3B
// shapes at 32 and 64 rows).  Splits (not with the SwiGLU epilogue, which
// needs whole sums) fill the CUs when the weight tiles alone do not, keeping
// at least 8 blocks (2 per wave) per split.
static void kw_plan(QgPlan& p, int N, int nb, int M, bool whole) {
    const int ntile16 = (N + 15) / 16, cu = qg_cu_count();
    p.kwT = M > 64 ? 8 : M > 32 ? 4 : 2;
    if (g_qg_mchunk) p.kwT = std::max(2, std::min(p.kwT, g_qg_mchunk / 16));
    p.mchunks = (M + 16 * p.kwT - 1) / (16 * p.kwT);
    double best = 1e30;
    for (int R = 2; R <= 4; R++) {  // ties go to the smaller R (fewer registers, two workgroups per CU)
        if (g_qg_kwR && R != g_qg_kwR) continue;
        const long long base = (long long)((ntile16 + R - 1) / R) * p.mchunks;
        int S = 1;
        if (!whole) {
            if (g_qg_splits > 0) S = g_qg_splits;
            else S = (int)std::max(1LL, std::min((long long)cu / base, (long long)nb / 8));
        }
        int bps = (nb + S - 1) / S;
        S = (nb + bps - 1) / bps;
        const long long rounds = (base * S + cu - 1) / cu;
        const double cost = (double)rounds * ((double)((bps + KW_WAVES - 1) / KW_WAVES) * (R + 2) + 3 * R);
        if (cost < best) {
            best = cost;
            p.kwR = R;
            p.S = S;
            p.bps = bps;
            p.ntiles = (ntile16 + R - 1) / R;
        }
    }
    p.NW = 16 * p.kwR;
    p.MW = 16 * p.kwT;
    p.ws_bytes = p.S > 1 ? (size_t)p.S * M * N * 4 : 0;
}

// Tile shape and split count for an N x K matrix times M rows.  Batch tiles
// of more than 32 rows use 2 x WN waves of 64 weight rows each; smaller ones
// 4 waves of 32 weight rows.  Splits are added (powers of two, at most 64)
// while the grid has fewer workgroups than the chip has slots for and every
// split keeps at least one ping-pong pair of stages.
// Row-split LDS-shared plan (qgemm_kx_kernel, 3 weight tiles per wave):
// batch chunks of 128 (64) rows, S splits of the quant blocks so that the
// grid holds at least one workgroup per CU, at least 8 blocks per split.
static void kx_plan(QgPlan& p, int N, int nb, int M, bool whole) {
    const int ntile16 = (N + 15) / 16, cu = qg_cu_count();
    p.kxT = M > 64 ? 8 : 4;
    p.MW = 16 * p.kxT;
    p.NW = 64 * 3;
    p.mchunks = (M + p.MW - 1) / p.MW;
    p.ntiles = (ntile16 + 11) / 12;
    const long long base = (long long)p.ntiles * p.mchunks;
    int S = 1;
    if (!whole) {
        if (g_qg_splits > 0) S = g_qg_splits;
        else S = (int)std::max(1LL, std::min((cu + base - 1) / base, (long long)nb / 8));
    }
    p.bps = (nb + S - 1) / S;
    p.S = (nb + p.bps - 1) / p.bps;
    p.ws_bytes = p.S > 1 ? (size_t)p.S * M * N * 4 : 0;
}

// The row-split LDS-shared kernel where it measured faster than the other
// forms (MI355X, tiled, GEMM + partial sums, graph-timed): 33-64 rows on
// products of 16384 rows and more (Q4 22016 x 2048 at 64 rows 29.9 us against
// 38.3 for the pipelined kernel and 42.1 for the wave-split one), and Q8_0
// products with a long in_dim from 65 rows (2048 x 11008 at 128 / 256 rows
// 34.1 / 54.9 against 41.8 / 65.2); the SwiGLU-epilogue entry from 256 rows
// (22016 x 2048 at 256 rows: Q4 78.7 against 84.7, Q8 81.1 against 122.7).
// At 128 rows on the Q4 shapes it ties or trails the pipelined kernel.
static bool kx_wanted(uint32_t dtype, int N, int K, int M) {
    if (g_qg_pipe == 3) return M > 16;
    if (g_qg_pipe != 0 || g_qg_kw != 0) return false;
    return (M > 32 && M <= 64 && N >= 16384) || (M > 64 && dtype == DT_Q8_0 && K >= 8192);
}

static QgPlan qgemm_plan(uint32_t dtype, int N, int K, int M, size_t row_bytes, bool tiled) {
    QgPlan p{};
    if (tiled && kx_wanted(dtype, N, K, M)) {
        kx_plan(p, N, K / 32, M, false);
        return p;
    }
    if (tiled && kw_wanted(N, M)) {
        kw_plan(p, N, K / 32, M, false);
        return p;
    }
    int Mc = min(M, g_qg_mchunk ? g_qg_mchunk : QG_MCHUNK);
    const bool pipe = g_qg_pipe == 1 || (g_qg_pipe == 0 && N >= 8192);
    // the narrow form is the default for narrow products at > 64 rows except
    // the smallest at <= 128 rows (MI355X, Q4, partial reduction included:
    // down 2048 x 11008 at 128/256/512 rows 36/61/105 -> 29/43/76 us, QKV
    // 2560 x 2048 19/28/39 -> 18/23/31 us, O 2048 x 2048 at 256/512 rows
    // 22/28 -> 20/23 us; O at 128 rows stays at 14 us on qgemm_kernel)
    const bool narrow = g_qg_pipe == 2 || (g_qg_pipe == 0 && !g_qg_mchunk && N < 8192 && Mc > 64 &&
                                           (M > 128 || (size_t)N * K > (size_t)4608 * 1024));
    if (tiled && Mc > 32 && narrow) {
        // narrow pipelined kernel: 4 waves side by side, 128 weight rows, all
        // 16*TM batch rows per wave (64 or 128); two workgroups per CU when
        // the 64-row stages fit the small LDS set
        p.pipe = true;
        p.KC = 2;
        p.WM = 1;
        p.WN = 4;
        p.TN = 2;
        p.TM = g_qg_mchunk == 128 ? 8 : 4;  // 64-row chunks, two workgroups per CU (measured best)
        p.MW = 16 * p.TM;
        p.NW = 128;
        p.ntiles = (N + p.NW - 1) / p.NW;
        p.mchunks = (M + p.MW - 1) / p.MW;
        const int nb = K / 32;
        const size_t tiles = (size_t)p.ntiles * p.mchunks;
        const size_t slots = p.TM == 4 ? 512 : 256;
        int S = 1;
        if (g_qg_splits > 0) S = g_qg_splits;
        else  // at most one round of workgroups, at least 16 blocks per split
            while (S < 64 && tiles * S * 2 <= slots && nb >= 32 * S) S *= 2;
        p.bps = ((nb + S - 1) / S + p.KC - 1) / p.KC * p.KC;
        p.S = (nb + p.bps - 1) / p.bps;
        qgemm_stream(p, nb, qg_cu_count() * (p.TM == 4 ? 2 : 1));
        p.ws_bytes = p.S > 1 ? (size_t)p.S * M * N * 4 : 0;
        return p;
    }
    if (tiled && Mc > 32 && pipe) {
        // pipelined kernel, 3-stage LDS ring, 1 workgroup per CU, 256 weight rows:
        // up to 64 batch rows 2 x 4 waves of 16*TM x 64 rows; beyond, 8 waves
        // side by side of all 128 batch rows x 32 weight rows (each converted
        // weight fragment then feeds 8 batch tiles instead of 4), or for Q4_0
        // x 48 weight rows (384 per workgroup; Q8_0's stages would not fit
        // the LDS) when that grid fills more CUs in one round
        p.pipe = true;
        p.KC = 2;
        const int nb = K / 32;
        const int unit = 3 * p.KC;  // blocks per trip of the 3-stage loop
        auto fill = [&](int tn, int& S) {  // workgroups of the tn form, S its split count
            const size_t tiles = (size_t)((N + 16 * tn * 8 - 1) / (16 * tn * 8)) * ((M + 127) / 128);
            S = 1;
            if (g_qg_splits > 0) S = g_qg_splits;
            else if (tn == 3)  // at most one round of workgroups (one per CU)
                while (S < 64 && tiles * S * 2 <= (size_t)qg_cu_count() && nb >= 2 * S * unit) S *= 2;
            else  // about one round of workgroups (one per CU): a second, partial round costs a full stage loop
                while (S < 64 && tiles * S * 2 <= 200 && nb >= 2 * S * unit) S *= 2;
            return tiles * S;
        };
        int S = 1;
        if (Mc > 64) {
            p.WM = 1;
            p.WN = 8;
            p.TM = 8;
            p.MW = 128;
            // the form with the smaller rounds of workgroups x work per
            // workgroup, (weight tiles) x (blocks per split + 10: the pipeline's
            // fill and drain and the partial tile, in blocks); MI355X, Q4_0 at 128
            // rows: 22016 x 2048 232 workgroups of 384 rows against 172 of 256
            // (the 128-row decode step 5.67 -> 5.56 ms); 11008 x 2048 172 of 256
            // rows in 4 splits (30.7 us) against 232 of 384 rows in 8 (32.5 us)
            int S3 = 1;
            const size_t cu = (size_t)qg_cu_count(), g2 = fill(2, S), g3 = fill(3, S3);
            const double t2 = (double)((g2 + cu - 1) / cu) * 2 * ((double)nb / S + 10),
                         t3 = (double)((g3 + cu - 1) / cu) * 3 * ((double)nb / S3 + 10);
            p.TN = row_bytes == (size_t)nb * 18 && t3 < t2 ? 3 : 2;
            if (p.TN == 3) S = S3;
        } else {
            p.WM = 2;
            p.WN = 4;
            p.TM = 2;  // 33..64 rows
            p.TN = 4;
            p.MW = 32 * p.TM;
            const size_t tiles = (size_t)((N + 255) / 256) * ((M + p.MW - 1) / p.MW);
            if (g_qg_splits > 0) S = g_qg_splits;
            else
                while (S < 64 && tiles * S * 2 <= 200 && nb >= 2 * S * unit) S *= 2;
        }
        p.NW = 16 * p.TN * p.WN;
        p.ntiles = (N + p.NW - 1) / p.NW;
        p.mchunks = (M + p.MW - 1) / p.MW;
        // whole stages per split; the kernel rounds its stage loop up to whole
        // trips and skips the blocks past the split
        p.bps = ((nb + S - 1) / S + p.KC - 1) / p.KC * p.KC;
        p.S = (nb + p.bps - 1) / p.bps;
        qgemm_stream(p, nb, qg_cu_count());
        p.ws_bytes = p.S > 1 ? (size_t)p.S * M * N * 4 : 0;
        return p;
    }
    // Narrow products (the non-pipelined path) at batches over 32 rows run in
    // 32-row chunks: four times the workgroups of one 128-row chunk and a
    // quarter of the split-K partials (measured on MI355X at the continuous-
    // batch shapes: QKV 2560x2048 25 -> 19 us, O 2048x2048 22 -> 14 us,
    // down 2048x11008 37 -> 34 us, partial reduction included).
    if (!g_qg_mchunk && tiled) Mc = min(Mc, 32);
    p.WM = Mc > 32 ? 2 : 1;
    p.TM = (Mc + 16 * p.WM - 1) / (16 * p.WM);
    p.TN = p.WM == 2 ? 4 : 2;
    p.WN = p.WM == 2 ? (g_qg_waves == 8 ? 4 : 2) : 4;
    p.MW = p.WM * p.TM * 16;
    p.NW = p.WN * p.TN * 16;
    p.KC = p.MW <= 32 ? 8 : p.MW <= 64 ? 4 : 2;  // keep the X stage near 16-32 KB
    p.ntiles = (N + p.NW - 1) / p.NW;
    p.mchunks = (M + p.MW - 1) / p.MW;
    const int nb = K / 32;
    const size_t tiles = (size_t)p.ntiles * p.mchunks;
    const size_t slots = p.WM * p.WN == 8 ? 256 : 512;  // workgroups resident at once (LDS / waves)
    (void)row_bytes;
    const int pair = 2 * p.KC;  // blocks per ping-pong pair of stages
    int S = 1;
    if (g_qg_splits > 0) {
        S = g_qg_splits;
    } else {
        while (S < 64 && tiles * S < slots && nb >= 2 * S * pair) S *= 2;
    }
    p.bps = ((nb + S - 1) / S + pair - 1) / pair * pair;
    p.S = (nb + p.bps - 1) / p.bps;  // no empty splits
    p.ws_bytes = p.S > 1 ? (size_t)p.S * M * N * 4 : 0;
    return p;
}

int set_qgemm_schedule(int mode, int min_blocks) {
    QH_REQUIRE(mode >= 0 && mode <= 2 && min_blocks >= 0 && min_blocks <= 4096, QRAF_HIP_ERR_INVALID,
               "qgemm schedule: mode %d, min_blocks %d", mode, min_blocks);
    g_qg_sched = mode;
    g_qg_skmin = min_blocks;
    bump_tuning_generation();
    return QRAF_HIP_OK;
}

int set_qgemm_kw(int mode, int tiles) {
    QH_REQUIRE(mode >= -1 && mode <= 1 && (tiles == 0 || (tiles >= 2 && tiles <= 4)), QRAF_HIP_ERR_INVALID,
               "qgemm kw: mode %d, tiles %d", mode, tiles);
    g_qg_kw = mode;
    g_qg_kwR = tiles;
    bump_tuning_generation();
    return QRAF_HIP_OK;
}

int set_qgemm_tuning(int waves, int splits, int pipe, int mchunk) {
    QH_REQUIRE(waves == 0 || waves == 4 || waves == 8, QRAF_HIP_ERR_INVALID, "qgemm tuning: waves %d", waves);
    QH_REQUIRE(mchunk == 0 || mchunk == 16 || mchunk == 32 || mchunk == 64 || mchunk == 128, QRAF_HIP_ERR_INVALID,
               "qgemm tuning: batch chunk %d", mchunk);
    QH_REQUIRE(splits >= 0 && splits <= 256, QRAF_HIP_ERR_INVALID, "qgemm tuning: splits %d", splits);
    QH_REQUIRE(pipe >= -1 && pipe <= 3, QRAF_HIP_ERR_INVALID, "qgemm tuning: pipe %d", pipe);
    g_qg_waves = waves;
    g_qg_splits = splits;
    g_qg_pipe = pipe;
    g_qg_mchunk = mchunk;
    bump_tuning_generation();
    return QRAF_HIP_OK;
}

size_t qgemm_workspace_bytes(uint32_t dtype, int N, int K, int M, bool tiled) {
    if ((dtype != DT_Q8_0 && dtype != DT_Q4_0) || N <= 0 || K <= 0 || K % 32 || M <= 0) return 0;
    return qgemm_plan(dtype, N, K, M, q_row_bytes(dtype, 32, K), tiled).ws_bytes;
}

size_t qgemm_partials_bytes(uint32_t dtype, int N, int K, int M, bool tiled) {
    if ((dtype != DT_Q8_0 && dtype != DT_Q4_0) || N <= 0 || K <= 0 || K % 32 || M <= 0) return 0;
    return (size_t)qgemm_plan(dtype, N, K, M, q_row_bytes(dtype, 32, K), tiled).S * M * N * 4;
}

int launch_split_bf16(const float* x, uint16_t* hi, uint16_t* lo, int M, int K, int op, float* xout, hipStream_t s,
                      int S, size_t slice) {
    QH_REQUIRE(x && hi && lo && M > 0 && K > 0 && S >= 1, QRAF_HIP_ERR_INVALID, "split: bad arguments");
    const size_t n = (size_t)M * K;
    if (op == 1 && !xout && S <= 4 && K % 4 == 0 && n < ((size_t)1 << 31) && (((uintptr_t)x) & 15) == 0 &&
        (S == 1 || slice % 4 == 0) && (((uintptr_t)hi) & 7) == 0 && (((uintptr_t)lo) & 7) == 0) {
        const int grid4 = (int)min((n / 4 + 255) / 256, (size_t)4096);
#define QH_S4(Sv) hipLaunchKernelGGL(silu_split4_kernel<Sv>, dim3(grid4), dim3(256), 0, s, x, hi, lo, M, K, slice)
        if (S == 1) QH_S4(1);
        else if (S == 2) QH_S4(2);
        else if (S == 3) QH_S4(3);
        else QH_S4(4);
#undef QH_S4
        QH_CHECK_HIP(hipGetLastError());
        return QRAF_HIP_OK;
    }
    const int grid = (int)min((n + 255) / 256, (size_t)4096);
    hipLaunchKernelGGL(split_bf16_kernel, dim3(grid), dim3(256), 0, s, x, hi, lo, M, K, op, xout, S, slice);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

size_t tiled_weight_bytes(uint32_t dtype, int N, int K) {
    if ((dtype != DT_Q8_0 && dtype != DT_Q4_0) || N <= 0 || K <= 0 || K % 32) return 0;
    return (size_t)((N + 15) / 16) * (K / 32) * tile_block_bytes(dtype == DT_Q8_0 ? 8 : 4);
}

int launch_repack_tiles(const void* W, uint32_t dtype, int N, int K, void* dst, hipStream_t s) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "repack: unsupported dtype %u", dtype);
    QH_REQUIRE(K % 32 == 0 && K > 0 && N > 0, QRAF_HIP_ERR_INVALID, "repack: K=%d must be a positive multiple of 32", K);
    QH_REQUIRE(W && dst && (((uintptr_t)W) & 1) == 0 && (((uintptr_t)dst) & 15) == 0, QRAF_HIP_ERR_INVALID,
               "repack: null or misaligned pointer");
    const size_t total = (size_t)((N + 15) / 16) * (K / 32) * 16;
    const int grid = (int)min((total + 255) / 256, (size_t)8192);
    if (dtype == DT_Q8_0)
        hipLaunchKernelGGL(repack_tiles_kernel<8>, dim3(grid), dim3(256), 0, s, (const uint8_t*)W, N, K / 32,
                           (uint8_t*)dst);
    else
        hipLaunchKernelGGL(repack_tiles_kernel<4>, dim3(grid), dim3(256), 0, s, (const uint8_t*)W, N, K / 32,
                           (uint8_t*)dst);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

// One launch of qgemm_kw_kernel<F, R, T>; dynamic LDS beyond 64 KB is opted
// into once per instantiation.
template <int F, int R, int T>
static int kw_attr() {
    static bool done = false;
    if (!done) {
        QH_CHECK_HIP(hipFuncSetAttribute((const void*)qgemm_kw_kernel<F, R, T>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)KwGeom<F, R, T>::LDS));
        done = true;
    }
    return QRAF_HIP_OK;
}

template <int F, int R>
static int kw_attr_t() {
    QH_TRY((kw_attr<F, R, 2>()));
    QH_TRY((kw_attr<F, R, 4>()));
    return kw_attr<F, R, 8>();
}

// Called by qraf_hip_init (the first launch of each form also does it), so
// that no attribute call happens while a caller captures a graph.
int qgemm_kw_init() {
    QH_TRY((kw_attr_t<4, 2>()));
    QH_TRY((kw_attr_t<4, 3>()));
    QH_TRY((kw_attr_t<4, 4>()));
    QH_TRY((kw_attr_t<8, 2>()));
    QH_TRY((kw_attr_t<8, 3>()));
    return kw_attr_t<8, 4>();
}

template <int F, int R, int T>
static int kw_go(dim3 grid, const uint8_t* W, int N, int nb, const uint16_t* xh, const uint16_t* xl, int K, int M,
                 int bps, float* Y, const float* add, size_t slice, int mode, uint16_t* act_hi, uint16_t* act_lo,
                 hipStream_t s) {
    constexpr size_t lds = KwGeom<F, R, T>::LDS;
    QH_TRY((kw_attr<F, R, T>()));
    hipLaunchKernelGGL((qgemm_kw_kernel<F, R, T>), grid, dim3(64 * KW_WAVES), lds, s, W, N, nb, xh, xl, K, M, bps, Y,
                       add, slice, mode, act_hi, act_lo);
    return QRAF_HIP_OK;
}

// qgemm_kw_kernel<FMT, p.kwR, p.kwT> (mode 0: Y / partial slices, 1: SwiGLU planes).
static int launch_kw(uint32_t dtype, const QgPlan& p, dim3 grid, const uint8_t* W, int N, int nb, const uint16_t* xh,
                     const uint16_t* xl, int K, int M, float* Y, const float* add, size_t slice, int mode,
                     uint16_t* act_hi, uint16_t* act_lo, hipStream_t s) {
#define QH_KW(F, R_, T_) \
    QH_TRY((kw_go<F, R_, T_>(grid, W, N, nb, xh, xl, K, M, p.bps, Y, add, slice, mode, act_hi, act_lo, s)))
#define QH_KWT(F, R_)                       \
    if (p.kwT == 2) { QH_KW(F, R_, 2); }      \
    else if (p.kwT == 4) { QH_KW(F, R_, 4); } \
    else { QH_KW(F, R_, 8); }
#define QH_KWR(F)                   \
    if (p.kwR == 2) { QH_KWT(F, 2) }      \
    else if (p.kwR == 3) { QH_KWT(F, 3) } \
    else { QH_KWT(F, 4) }
    if (dtype == DT_Q8_0) {
        QH_KWR(8)
    } else {
        QH_KWR(4)
    }
#undef QH_KWR
#undef QH_KWT
#undef QH_KW
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

// qgemm_pipe_kernel at plan p's geometry; amax: the greedy-head epilogue
// (uniform split grid, one split, no Y).
static void launch_pipe(uint32_t dtype, const QgPlan& p, dim3 grid, const void* W, int N, int nb, const uint16_t* xh,
                        const uint16_t* xl, int K, int M, float* Y, const float* add, float* part, uint64_t* amax,
                        hipStream_t s) {
#define QH_P(F, TM_, TN_, WN_, WM_)                                                                            \
    do {                                                                                                      \
        if (amax)                                                                                             \
            hipLaunchKernelGGL((qgemm_pipe_kernel<F, TM_, TN_, 2, WN_, WM_, false, true>), grid,               \
                               dim3(64 * WN_ * WM_), 0, s, (const uint8_t*)W, N, nb, xh, xl, K, M, nullptr,     \
                               nullptr, p.bps, nullptr, 0, p.ntiles, 1, nullptr, nullptr, amax);              \
        else if (p.skG > 0)                                                                                   \
            hipLaunchKernelGGL((qgemm_pipe_kernel<F, TM_, TN_, 2, WN_, WM_, true>), grid, dim3(64 * WN_ * WM_), 0, \
                               s, (const uint8_t*)W, N, nb, xh, xl, K, M, Y, add, p.bps, part, p.skG, p.ntiles,  \
                               p.S, nullptr, nullptr, nullptr);                                               \
        else                                                                                                  \
            hipLaunchKernelGGL((qgemm_pipe_kernel<F, TM_, TN_, 2, WN_, WM_, false>), grid, dim3(64 * WN_ * WM_),  \
                               0, s, (const uint8_t*)W, N, nb, xh, xl, K, M, Y, add, p.bps, part, 0, p.ntiles,  \
                               p.S, nullptr, nullptr, nullptr);                                               \
    } while (0)
    if (dtype == DT_Q8_0) {
        if (p.WN == 4 && p.WM == 1) {
            if (p.TM == 8) QH_P(8, 8, 2, 4, 1);
            else QH_P(8, 4, 2, 4, 1);
        } else if (p.WM == 1) QH_P(8, 8, 2, 8, 1);
        else QH_P(8, 2, 4, 4, 2);
    } else {
        if (p.WN == 4 && p.WM == 1) {
            if (p.TM == 8) QH_P(4, 8, 2, 4, 1);
            else QH_P(4, 4, 2, 4, 1);
        } else if (p.WM == 1) {
            if (p.TN == 3) QH_P(4, 8, 3, 8, 1);
            else QH_P(4, 8, 2, 8, 1);
        } else QH_P(4, 2, 4, 4, 2);
    }
#undef QH_P
}

int launch_qgemm(const void* W, uint32_t dtype, int bs, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                 float* Y, const float* add, void* ws, size_t ws_bytes, hipStream_t s, bool tiled, int* slices) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "qgemm: unsupported dtype %u", dtype);
    QH_REQUIRE(bs == 32, QRAF_HIP_ERR_DTYPE, "qgemm: block size %d (32 required)", bs);
    QH_REQUIRE(K % 32 == 0 && K > 0 && N > 0, QRAF_HIP_ERR_INVALID, "qgemm: K=%d must be a positive multiple of 32", K);
    QH_REQUIRE(M > 0, QRAF_HIP_ERR_INVALID, "qgemm: batch %d", M);
    QH_REQUIRE(W && xh && xl && Y, QRAF_HIP_ERR_INVALID, "qgemm: null pointer");
    // Q8 blocks are read with 4-byte loads (36-byte blocks keep rows 4-aligned),
    // Q4 blocks with 2-byte-aligned loads (18-byte blocks); X rows with 16-byte loads
    QH_REQUIRE((((uintptr_t)W) & (tiled ? 15 : dtype == DT_Q8_0 ? 3 : 1)) == 0 && (((uintptr_t)xh) & 15) == 0 &&
                   (((uintptr_t)xl) & 15) == 0,
               QRAF_HIP_ERR_INVALID, "qgemm: misaligned operands");
    const size_t rb = q_row_bytes(dtype, bs, K);
    const int nb = K / 32;
    QgPlan p = qgemm_plan(dtype, N, K, M, rb, tiled);
    float* part = nullptr;
    if (slices) {  // partials mode: S slices [S][M][N] in ws, summed by the caller's next kernel
        QH_REQUIRE(ws && ws_bytes >= (size_t)p.S * M * N * 4 && (((uintptr_t)ws) & 15) == 0 && !add,
                   QRAF_HIP_ERR_INVALID, "qgemm: partials need a workspace of %zu bytes and no residual",
                   (size_t)p.S * M * N * 4);
        part = (float*)ws;
        *slices = p.S;
    } else if (p.S > 1) {
        if (ws && ws_bytes >= p.ws_bytes && (((uintptr_t)ws) & 15) == 0) {
            part = (float*)ws;
        } else {  // no (or too small a) workspace: one split
            p.S = 1;
            p.skG = 0;
            const int unit = (p.kwR || p.kxT) ? 1 : (p.pipe ? 1 : 2) * p.KC;
            p.bps = (nb + unit - 1) / unit * unit;
        }
    }
    QH_REQUIRE(p.mchunks <= 65535, QRAF_HIP_ERR_INVALID, "qgemm: batch %d too large", M);
    const dim3 grid = p.skG > 0 ? dim3(p.skG, 1, 1) : dim3(p.ntiles, p.S, p.mchunks);
    if (p.kxT) {
#define QH_KX(F, T_)                                                                                          \
    hipLaunchKernelGGL((qgemm_kx_kernel<F, 3, T_, 1>), grid, dim3(256), 0, s, (const uint8_t*)W, N, nb, xh, xl, K, M, \
                       Y, add, p.bps, part, nullptr, nullptr)
        if (dtype == DT_Q8_0) {
            if (p.kxT == 8) QH_KX(8, 8);
            else QH_KX(8, 4);
        } else {
            if (p.kxT == 8) QH_KX(4, 8);
            else QH_KX(4, 4);
        }
#undef QH_KX
    } else if (p.kwR) {
        float* yk = part ? part : Y;
        const size_t slice = part ? (size_t)M * N : 0;
        QH_TRY(launch_kw(dtype, p, grid, (const uint8_t*)W, N, nb, xh, xl, K, M, yk, part ? nullptr : add, slice, 0,
                         nullptr, nullptr, s));
    } else if (p.pipe) {
        launch_pipe(dtype, p, grid, W, N, nb, xh, xl, K, M, Y, add, part, nullptr, s);
    } else {
#define QH_G(F, WM_, WN_, TM_, TN_, KC_)                                                                           \
    if (tiled)                                                                                                     \
        hipLaunchKernelGGL((qgemm_kernel<F, WM_, WN_, TM_, TN_, KC_, true>), grid, dim3(64 * WM_ * WN_), 0, s,       \
                           (const uint8_t*)W, rb, N, nb, xh, xl, K, M, Y, add, p.bps, part);                       \
    else                                                                                                           \
        hipLaunchKernelGGL((qgemm_kernel<F, WM_, WN_, TM_, TN_, KC_, false>), grid, dim3(64 * WM_ * WN_), 0, s,      \
                           (const uint8_t*)W, rb, N, nb, xh, xl, K, M, Y, add, p.bps, part)
#define QH_GW(F, WN_)                               \
    if (p.TM == 2) QH_G(F, 2, WN_, 2, 4, 4);        \
    else if (p.TM == 3) QH_G(F, 2, WN_, 3, 4, 2);   \
    else QH_G(F, 2, WN_, 4, 4, 2);
#define QH_GF(F)                                    \
    if (p.WM == 1) {                                \
        if (p.TM == 1) QH_G(F, 1, 4, 1, 2, 8);      \
        else QH_G(F, 1, 4, 2, 2, 8);                \
    } else if (p.WN == 4) {                         \
        QH_GW(F, 4)                                 \
    } else {                                        \
        QH_GW(F, 2)                                 \
    }
    if (dtype == DT_Q8_0) {
        QH_GF(8)
    } else {
        QH_GF(4)
    }
#undef QH_GF
#undef QH_GW
#undef QH_G
    }
    QH_CHECK_HIP(hipGetLastError());
    if (part && !slices) {
        const size_t MN = (size_t)M * N;
        const int rgrid = (int)min((MN / 4 + 255) / 256 + 1, (size_t)2048);
        hipLaunchKernelGGL(qgemm_reduce_kernel, dim3(rgrid), dim3(256), 0, s, part, p.S, MN, Y, add);
        QH_CHECK_HIP(hipGetLastError());
    }
    return QRAF_HIP_OK;
}

// Row m's token: the largest of the per-workgroup keys [tiles][M] of
// qgemm_pipe_kernel's argmax epilogue (0 for a key past the N rows, as
// argmax_rows_kernel clamps).
__global__ __launch_bounds__(256) void argmax_keys_kernel(const uint64_t* __restrict__ keys, int tiles, int M, int N,
                                                          uint32_t* __restrict__ out) {
    __shared__ uint64_t wb[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    uint64_t best = 0;
    for (int t = tid; t < tiles; t += 256) {
        const uint64_t k = keys[(size_t)t * M + m];
        best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t k = __shfl_xor(best, o);
        best = k > best ? k : best;
    }
    if ((tid & 63) == 0) wb[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; w++) best = wb[w] > best ? wb[w] : best;
        const uint32_t idx = 0xFFFFFFFFu - (uint32_t)best;
        out[m] = best != 0 && idx < (uint32_t)N ? idx : 0u;
    }
}

size_t qgemm_argmax_keys_bytes(int N, int M) {
    // pipelined tiles hold at least 128 weight rows
    return (size_t)((N + 127) / 128) * (size_t)M * 8;
}

// Greedy head: the argmax (Sampler::argmax) of each of the M rows of
// X W^T over the N weight rows, with no product written: where the tiled plan
// is the pipelined form, qgemm_pipe_kernel in one split writes each
// workgroup's best key per row to keys [tiles][M] and argmax_keys_kernel
// reduces them to out [M]; *done = false and nothing launched otherwise (the
// caller then writes the products and takes their argmax).
// the pipelined plan of the fused head, unsplit (false: not the pipelined form,
// or the keys do not fit)
static bool argmax_plan(uint32_t dtype, int N, int K, int M, size_t keys_bytes, QgPlan& p) {
    if ((dtype != DT_Q8_0 && dtype != DT_Q4_0) || K <= 0 || K % 32 || N <= 0 || M <= 0) return false;
    p = qgemm_plan(dtype, N, K, M, q_row_bytes(dtype, 32, K), true);
    if (!p.pipe || p.kwR || p.kxT) return false;
    p.S = 1;  // complete sums in every workgroup
    p.skG = 0;
    p.bps = K / 32;
    return p.mchunks <= 65535 && keys_bytes >= (size_t)p.ntiles * M * 8;
}

bool qgemm_argmax_fits(uint32_t dtype, int N, int K, int M, size_t keys_bytes) {
    QgPlan p;
    return argmax_plan(dtype, N, K, M, keys_bytes, p);
}

int launch_qgemm_argmax(const void* Wt, uint32_t dtype, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                        uint64_t* keys, size_t keys_bytes, uint32_t* out, hipStream_t s, bool* done) {
    *done = false;
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "qgemm argmax: unsupported dtype %u", dtype);
    QH_REQUIRE(K % 32 == 0 && K > 0 && N > 0 && M > 0, QRAF_HIP_ERR_INVALID, "qgemm argmax: N=%d K=%d M=%d", N, K, M);
    QH_REQUIRE(Wt && xh && xl && keys && out, QRAF_HIP_ERR_INVALID, "qgemm argmax: null pointer");
    QH_REQUIRE((((uintptr_t)Wt) & 15) == 0 && (((uintptr_t)xh) & 15) == 0 && (((uintptr_t)xl) & 15) == 0 &&
                   (((uintptr_t)keys) & 7) == 0,
               QRAF_HIP_ERR_INVALID, "qgemm argmax: misaligned operands");
    QgPlan p;
    if (!argmax_plan(dtype, N, K, M, keys_bytes, p)) return QRAF_HIP_OK;
    launch_pipe(dtype, p, dim3(p.ntiles, 1, p.mchunks), Wt, N, K / 32, xh, xl, K, M, nullptr, nullptr, nullptr, keys,
                s);
    QH_CHECK_HIP(hipGetLastError());
    hipLaunchKernelGGL(argmax_keys_kernel, dim3(M), dim3(256), 0, s, keys, p.ntiles, M, N, out);
    QH_CHECK_HIP(hipGetLastError());
    *done = true;
    return QRAF_HIP_OK;
}

// Gate/up projection of interleaved rows with the SwiGLU front in the
// epilogue: the narrow pipelined form (4 waves x 128 weight rows, 64-row
// batch chunks, one workgroup per (tile, chunk), no split) so that every
// workgroup holds complete sums; act_hi/act_lo [M][N/2] must not overlap xh/xl.
int launch_qgemm_silu(const void* Wt, uint32_t dtype, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                      uint16_t* act_hi, uint16_t* act_lo, hipStream_t s) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "qgemm silu: unsupported dtype %u", dtype);
    QH_REQUIRE(K % 32 == 0 && K > 0 && N > 0 && N % 2 == 0 && M > 0, QRAF_HIP_ERR_INVALID,
               "qgemm silu: N=%d (even), K=%d (multiple of 32), M=%d", N, K, M);
    QH_REQUIRE(Wt && xh && xl && act_hi && act_lo, QRAF_HIP_ERR_INVALID, "qgemm silu: null pointer");
    QH_REQUIRE(((((uintptr_t)Wt) | ((uintptr_t)xh) | ((uintptr_t)xl)) & 15) == 0, QRAF_HIP_ERR_INVALID,
               "qgemm silu: misaligned operands");
    const int nb = K / 32, KC = 2;
    if (g_qg_pipe == 3 ? M > 16 : (g_qg_pipe == 0 && g_qg_kw == 0 && M >= 256)) {
        QgPlan p{};
        kx_plan(p, N, nb, M, true);
        QH_REQUIRE(p.mchunks <= 65535, QRAF_HIP_ERR_INVALID, "qgemm silu: batch %d too large", M);
        const dim3 g(p.ntiles, 1, p.mchunks);
#define QH_KXS(F, T_)                                                                                            \
    hipLaunchKernelGGL((qgemm_kx_kernel<F, 3, T_, 1>), g, dim3(256), 0, s, (const uint8_t*)Wt, N, nb, xh, xl, K, M, \
                       nullptr, nullptr, nb, nullptr, act_hi, act_lo)
        if (dtype == DT_Q8_0) {
            if (p.kxT == 8) QH_KXS(8, 8);
            else QH_KXS(8, 4);
        } else {
            if (p.kxT == 8) QH_KXS(4, 8);
            else QH_KXS(4, 4);
        }
#undef QH_KXS
        QH_CHECK_HIP(hipGetLastError());
        return QRAF_HIP_OK;
    }
    if (kw_wanted(N, M)) {
        QgPlan p{};
        kw_plan(p, N, nb, M, true);
        QH_REQUIRE(p.mchunks <= 65535, QRAF_HIP_ERR_INVALID, "qgemm silu: batch %d too large", M);
        return launch_kw(dtype, p, dim3(p.ntiles, 1, p.mchunks), (const uint8_t*)Wt, N, nb, xh, xl, K, M, nullptr,
                         nullptr, 0, 1, act_hi, act_lo, s);
    }
    const dim3 grid((N + 127) / 128, 1, (M + 63) / 64);
    QH_REQUIRE(grid.z <= 65535, QRAF_HIP_ERR_INVALID, "qgemm silu: batch %d too large", M);
    const int bps = (nb + KC - 1) / KC * KC;
    if (dtype == DT_Q8_0)
        hipLaunchKernelGGL((qgemm_pipe_kernel<8, 4, 2, 2, 4, 1, false>), grid, dim3(256), 0, s, (const uint8_t*)Wt, N, nb, xh, xl,
                           K, M, nullptr, nullptr, bps, nullptr, 0, 0, 1, act_hi, act_lo, nullptr);
    else
        hipLaunchKernelGGL((qgemm_pipe_kernel<4, 4, 2, 2, 4, 1, false>), grid, dim3(256), 0, s, (const uint8_t*)Wt, N, nb, xh, xl,
                           K, M, nullptr, nullptr, bps, nullptr, 0, 0, 1, act_hi, act_lo, nullptr);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip

extern "C" {

int qraf_hip_split_bf16_dev(const float* x, uint16_t* x_hi, uint16_t* x_lo, int32_t rows, int32_t cols, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_split_bf16(x, x_hi, x_lo, rows, cols, 0, nullptr, qraf_hip::as_stream(stream));
}

int qraf_hip_qgemm_tiled_silu_dev(const void* w_tiled, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                                  const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, uint16_t* out_hi,
                                  uint16_t* out_lo, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_qgemm_silu(w_tiled, dtype, (int)out_dim, (int)in_dim, x_hi, x_lo, batch, out_hi, out_lo,
                                       qraf_hip::as_stream(stream));
}

int qraf_hip_set_qgemm_schedule(int32_t mode, int32_t min_blocks) {
    qraf_hip::clear_error();
    return qraf_hip::set_qgemm_schedule(mode, min_blocks);
}

int qraf_hip_set_qgemm_tuning(int waves, int splits, int pipe, int batch_chunk) {
    qraf_hip::clear_error();
    return qraf_hip::set_qgemm_tuning(waves, splits, pipe, batch_chunk);
}

int qraf_hip_set_qgemm_kw(int32_t mode, int32_t tiles_per_workgroup) {
    qraf_hip::clear_error();
    return qraf_hip::set_qgemm_kw(mode, tiles_per_workgroup);
}

uint64_t qraf_hip_qgemm_workspace_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim, int32_t batch) {
    return qraf_hip::qgemm_workspace_bytes(dtype, (int)out_dim, (int)in_dim, batch, false);
}

uint64_t qraf_hip_qgemm_tiled_workspace_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim, int32_t batch) {
    return qraf_hip::qgemm_workspace_bytes(dtype, (int)out_dim, (int)in_dim, batch, true);
}

int qraf_hip_qgemm_dev(const void* w, uint32_t dtype, uint32_t block_size, uint32_t out_dim, uint32_t in_dim,
                       const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, float* y, const float* add,
                       void* workspace, uint64_t workspace_bytes, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_qgemm(w, dtype, block_size ? (int)block_size : 32, (int)out_dim, (int)in_dim, x_hi, x_lo,
                                  batch, y, add, workspace, workspace_bytes, qraf_hip::as_stream(stream), false);
}

uint64_t qraf_hip_tiled_weight_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim) {
    return qraf_hip::tiled_weight_bytes(dtype, (int)out_dim, (int)in_dim);
}

int qraf_hip_repack_tiles_dev(const void* w, uint32_t dtype, uint32_t out_dim, uint32_t in_dim, void* dst,
                              void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_repack_tiles(w, dtype, (int)out_dim, (int)in_dim, dst, qraf_hip::as_stream(stream));
}

int qraf_hip_qgemm_tiled_dev(const void* w_tiled, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                             const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, float* y, const float* add,
                             void* workspace, uint64_t workspace_bytes, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_qgemm(w_tiled, dtype, 32, (int)out_dim, (int)in_dim, x_hi, x_lo, batch, y, add, workspace,
                                  workspace_bytes, qraf_hip::as_stream(stream), true);
}

uint64_t qraf_hip_qgemm_tiled_argmax_keys_bytes(uint32_t out_dim, int32_t batch) {
    return batch > 0 ? qraf_hip::qgemm_argmax_keys_bytes((int)out_dim, batch) : 0;
}

int qraf_hip_qgemm_tiled_argmax_dev(const void* w_tiled, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                                    const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, void* keys,
                                    uint64_t keys_bytes, uint32_t* tokens, int32_t* fused, void* stream) {
    qraf_hip::clear_error();
    bool done = false;
    const int rc = qraf_hip::launch_qgemm_argmax(w_tiled, dtype, (int)out_dim, (int)in_dim, x_hi, x_lo, batch,
                                                 (uint64_t*)keys, keys_bytes, tokens, qraf_hip::as_stream(stream),
                                                 &done);
    if (fused) *fused = done ? 1 : 0;
    return rc;
}

}  // extern "C"
