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
// and loads each unit with two dwordx4 loads + one dword (4-byte aligned),
// so a wave reads 2304 contiguous bytes per row step.  The activation vector
// is staged once per workgroup in LDS, padded to 36 floats per 32-element
// block (16-byte aligned, free of bank conflicts for ds_read_b128), for Q4
// with every odd element pre-scaled by 1/16 (see q4_compute).
// Dequantisation happens in registers: v_cvt_f32_i32 with an SDWA byte select
// for Q8; for Q4 one mask per two nibbles and v_fma_mix_f32, which reads the
// masked nibble as an fp16 subnormal (the -8 offset is applied once per block
// through the staged block sum).  Accumulation is fp32; each wave reduces its
// R rows with a transposing butterfly.
#include "common.h"

#include <atomic>

namespace qraf_hip {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int XS8 = 36;  // staged floats per Q8 block  (32 + pad)
constexpr int XS4 = 76;  // staged floats per Q4 block pair (2 x (32 + sum + pad) + pad)
constexpr int WG = 256;  // 4 waves

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// Q4 staging of x: elements in order, odd ones times 1/16 (exact: a power of
// two).  q4_compute reads nibble pairs as fp16 subnormals: masking a dword of
// 8 nibbles with 0x000F000F leaves elements 0 and 4 as n * 2^-24 in its two
// halves, with 0x00F000F0 elements 1 and 5 as 16n * 2^-24, and the same masks
// of the dword shifted right by 8 give elements 2/6 and 3/7.  With the odd
// elements' x staged as x / 16 every product is n * x * 2^-24 exactly.
__device__ __forceinline__ f32x4 q4_stage4(float a, float b, float c, float d) {
    return f32x4{a, b * 0.0625f, c, d * 0.0625f};
}
__device__ __forceinline__ float half_lo(uint32_t t) { return (float)__builtin_bit_cast(_Float16, (uint16_t)t); }
__device__ __forceinline__ float half_hi(uint32_t t) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(t >> 16)); }

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
//
// Latency hiding: the first unit's weights are requested before x is staged,
// and every iteration requests the next unit's weights before it computes the
// current one, so each wave keeps two units x R rows of loads in flight.
// ----------------------------------------------------------------------------
// A unit's 36 bytes as the hardware loads them: bytes 0-15, 16-31, 32-35.
// (Declared in this order on purpose: a layout that does not match the load
// split makes the compiler copy registers right after the loads, which waits
// for them.)  dword(w, r, i) is dword i (0..8) of row r's unit.
template <int R>
struct Units {
    u32x4a4 a[R], b[R];
    uint32_t c[R];
};
template <int R>
__device__ __forceinline__ uint32_t dword(const Units<R>& w, int r, int i) {
    return i < 4 ? w.a[r][i] : i < 8 ? w.b[r][i - 4] : w.c[r];
}

template <int R>
__device__ __forceinline__ void load_units(Units<R>& w, const uint8_t* const (&rowp)[R], int u) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t* p = rowp[r] + (size_t)u * 36;
        w.a[r] = *(const u32x4a4*)p;
        w.b[r] = *(const u32x4a4*)(p + 16);
        w.c[r] = *(const uint32_t*)(p + 32);
    }
}

template <int R>
__device__ __forceinline__ void q8_compute(const Units<R>& w, const float* xs, float (&acc)[R]) {
    const f32x4* xv = (const f32x4*)xs;
    f32x4 xr[8];
#pragma unroll
    for (int j = 0; j < 8; j++) xr[j] = xv[j];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float bs = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t d = dword(w, r, 1 + j);
#pragma unroll
            for (int k = 0; k < 4; k++) bs = __builtin_fmaf((float)(int8_t)(d >> (8 * k)), xr[j][k], bs);
        }
        acc[r] = __builtin_fmaf(bs, __builtin_bit_cast(float, dword(w, r, 0)), acc[r]);
    }
}

// The nibbles of one dword (elements 8k..8k+7 of a block) as the four masked
// dwords q4_compute multiplies: halves (e0, e4), (16 e1, 16 e5), (e2, e6),
// (16 e3, 16 e7), each an fp16 subnormal of value half * 2^-24.
__device__ __forceinline__ void q4_split(uint32_t d, uint32_t (&t)[4]) {
    const uint32_t u = d >> 8;
    t[0] = d & 0x000F000Fu;
    t[1] = d & 0x00F000F0u;
    t[2] = u & 0x000F000Fu;
    t[3] = u & 0x00F000F0u;
}

// Block sums of the unit's two blocks: every product is n * x * 2^-24 (exact
// inside the fma), so be and bo are the sums of n * x scaled by 2^-24 -- the
// same roundings, as binary scaling commutes with them while values stay
// normal -- and the -8 offset and the block scale are applied at that scale
// (8 * sum * 2^-24 = sum * 2^-21; scale * 2^24), so acc gets the unscaled
// arithmetic's value.
template <int R>
__device__ __forceinline__ void q4_compute(const Units<R>& w, const float* xu, float (&acc)[R]) {
    f32x4 xe[8], xo[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        xe[j] = ((const f32x4*)xu)[j];
        xo[j] = ((const f32x4*)(xu + 36))[j];
    }
    const float se8 = 0x1p-21f * xu[32], so8 = 0x1p-21f * xu[36 + 32];
#pragma unroll
    for (int r = 0; r < R; r++) {
        // unit dwords: s = 0, a = 1..4, b = 5..8
        uint32_t dw[9];
#pragma unroll
        for (int i = 0; i < 9; i++) dw[i] = dword(w, r, i);
        float be = 0.f, bo = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t te[4], to[4];
            q4_split(__builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2), te);  // even block, nibble bytes 4k..4k+3
            q4_split(dw[5 + k], to);                                         // odd block, nibble bytes 4k..4k+3
#pragma unroll
            for (int q = 0; q < 4; q++) {
                be = __builtin_fmaf(half_lo(te[q]), xe[2 * k][q], be);
                bo = __builtin_fmaf(half_lo(to[q]), xo[2 * k][q], bo);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                be = __builtin_fmaf(half_hi(te[q]), xe[2 * k + 1][q], be);
                bo = __builtin_fmaf(half_hi(to[q]), xo[2 * k + 1][q], bo);
            }
        }
        const float se = half_bits_to_float(dw[0]) * 0x1p24f, so = half_bits_to_float(dw[4] >> 16) * 0x1p24f;
        acc[r] = __builtin_fmaf(be - se8, se, acc[r]);
        acc[r] = __builtin_fmaf(bo - so8, so, acc[r]);
    }
}

// ---- forming x while staging it (MvPrep): element i of x from its source
template <int XP>
__device__ __forceinline__ float x_elem(const float* __restrict__ x, int i, float r, const float* __restrict__ w) {
    if (XP == XP_NORM) return __fmul_rn(__fmul_rn(x[i], r), w[i]);
    if (XP == XP_SILU_GATE) return silu_gate(x[2 * i], x[2 * i + 1]);
    return x[i];
}
// elements i..i+3 (i % 4 == 0, i + 3 < K, x and w 16-byte aligned)
template <int XP>
__device__ __forceinline__ f32x4 x_vec4(const float* __restrict__ x, int i, float r, const float* __restrict__ w) {
    if (XP == XP_SILU_GATE) {
        const f32x4 a = *(const f32x4*)(x + 2 * i), b = *(const f32x4*)(x + 2 * i + 4);
        return f32x4{silu_gate(a[0], a[1]), silu_gate(a[2], a[3]), silu_gate(b[0], b[1]), silu_gate(b[2], b[3])};
    }
    f32x4 v = *(const f32x4*)(x + i);
    if (XP == XP_NORM) {
        const f32x4 ww = *(const f32x4*)(w + i);
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = __fmul_rn(__fmul_rn(v[e], r), ww[e]);
    }
    return v;
}
// 1 / sqrt(mean(x^2) + eps) for a 256-thread workgroup: the reduction of the
// engine's rmsnorm_rows_kernel (strided fma per thread, wave butterfly, the
// four waves in pairs), so a fused norm equals the separate one bit for bit
__device__ __forceinline__ float norm_r_256(const float* __restrict__ x, int K, float eps) {
    __shared__ float red[4];
    float ss = 0.f;
    for (int i = threadIdx.x; i < K; i += 256) ss = __builtin_fmaf(x[i], x[i], ss);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    return 1.0f / sqrtf(ss / (float)K + eps);
}

template <int FMT, int XP = XP_NONE>
__device__ __forceinline__ void stage_x(float* sx, const float* __restrict__ x, int K, int nb,
                                        const float* __restrict__ xw = nullptr, float eps = 0.f) {
    const float r = XP == XP_NORM ? norm_r_256(x, K, eps) : 1.f;
    const bool vec = (((uintptr_t)x) & 15) == 0 && (XP != XP_NORM || (((uintptr_t)xw) & 15) == 0);
    if (FMT == 8) {
        // thread t stages elements 4t..4t+3 (one float4, inside one block)
        for (int i = threadIdx.x * 4; i < nb * 32; i += WG * 4) {
            f32x4 v;
            if (i + 3 < K && vec) {
                v = x_vec4<XP>(x, i, r, xw);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = (i + e < K) ? x_elem<XP>(x, i + e, r, xw) : 0.f;
            }
            *(f32x4*)(sx + (i >> 5) * XS8 + (i & 31)) = v;
        }
    } else {
        // thread t stages elements 8t..8t+7 (odd ones scaled, q4_stage4) and
        // the four threads of a block reduce its sum.  Keff drops the odd tail
        // element the reference never reads (quantize.cpp:227).
        const int Keff = K & ~1;
        const int nthr = nb * 4;  // 8 elements per thread
        for (int base = 0; base < nthr; base += WG) {
            const int t = base + threadIdx.x;
            const int i = t * 8;
            float v[8];
            if (t < nthr && i + 7 < Keff && vec) {
                f32x4 a = x_vec4<XP>(x, i, r, xw), b = x_vec4<XP>(x, i + 4, r, xw);
                v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
                v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (t < nthr && i + e < Keff) ? x_elem<XP>(x, i + e, r, xw) : 0.f;
            }
            float part = ((v[0] + v[2]) + (v[4] + v[6])) + ((v[1] + v[3]) + (v[5] + v[7]));
            part += __shfl_xor(part, 1);
            part += __shfl_xor(part, 2);
            if (t < nthr) {
                const int blk = i >> 5, g = (i & 31) >> 3;
                float* dst = sx + (blk >> 1) * XS4 + (blk & 1) * 36;
                *(f32x4*)(dst + g * 8) = q4_stage4(v[0], v[1], v[2], v[3]);
                *(f32x4*)(dst + g * 8 + 4) = q4_stage4(v[4], v[5], v[6], v[7]);
                if ((t & 3) == 0) dst[32] = part;
            }
        }
    }
}

// Q8 staging of x in two phases, for K == nb * 32 <= 2048 * JX and 16-byte
// aligned x (and xw): issue() requests every load the staging needs (the
// norm's strided elements, the float4s to stage), each index clamped into x
// so that no load sits in a branch; finish() forms and stores them.  A caller
// that requests its weights between the two waits for x with the weights
// still in flight (the wait counter is in order).  The values are those of
// stage_x<8, XP>: the same strided fma order and reduction for the norm, the
// same products per element.
template <int XP, int JX>
struct XStage8 {
    static constexpr int NI = 2 * JX;                      // float4 steps of 1024 elements
    static constexpr int NN = XP == XP_NORM ? 8 * JX : 1;  // strided norm elements per thread
    f32x4 a[NI], b[XP == XP_NONE ? 1 : NI];                // x, and the SiLU-gate's second float4 or xw
    float n[NN];
    __device__ __forceinline__ void issue(const float* __restrict__ x, const float* __restrict__ xw, int K) {
        const int t = threadIdx.x;
        if (XP == XP_NORM) {
#pragma unroll
            for (int k = 0; k < NN; k++) n[k] = x[min(t + 256 * k, K - 1)];
        }
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int i = min(4 * t + 1024 * k, K - 4);
            if (XP == XP_SILU_GATE) {
                a[k] = *(const f32x4*)(x + 2 * i);
                b[k] = *(const f32x4*)(x + 2 * i + 4);
            } else {
                a[k] = *(const f32x4*)(x + i);
                if (XP == XP_NORM) b[k] = *(const f32x4*)(xw + i);
            }
        }
    }
    __device__ __forceinline__ void finish(float* sx, int K, float eps) {
        const int t = threadIdx.x;
        float r = 1.f;
        if (XP == XP_NORM) {  // norm_r_256's sums in its order
            __shared__ float red[4];
            float ss = 0.f;
#pragma unroll
            for (int k = 0; k < NN; k++) ss = t + 256 * k < K ? __builtin_fmaf(n[k], n[k], ss) : ss;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
            if ((t & 63) == 0) red[t >> 6] = ss;
            __syncthreads();
            ss = (red[0] + red[1]) + (red[2] + red[3]);
            r = 1.0f / sqrtf(ss / (float)K + eps);
        }
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int i = 4 * t + 1024 * k;
            f32x4 v;
            if (XP == XP_SILU_GATE) {
                v = f32x4{silu_gate(a[k][0], a[k][1]), silu_gate(a[k][2], a[k][3]), silu_gate(b[k][0], b[k][1]),
                          silu_gate(b[k][2], b[k][3])};
            } else if (XP == XP_NORM) {
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = __fmul_rn(__fmul_rn(a[k][e], r), b[k][e]);
            } else {
                v = a[k];
            }
            if (i < K) *(f32x4*)(sx + (i >> 5) * XS8 + (i & 31)) = v;
        }
    }
};

// The row of its group that lane `lane` holds after wave_reduce_rows<R>.
template <int R>
__device__ __forceinline__ int reduced_row_of_lane(int lane) {
    int r = 0;
#pragma unroll
    for (int m = 32, c = R; c > 1; c >>= 1, m >>= 1) r = r * 2 + ((lane & m) != 0 ? 1 : 0);
    return r;
}

// FMT 8: unit = one Q8_0 block; FMT 4: unit = a pair of Q4_0 blocks.
template <int FMT, int R>
__global__ __launch_bounds__(WG) void qmv_stream_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes, int N,
                                                     int K, int nb, const float* __restrict__ x,
                                                     float* __restrict__ y, const float* __restrict__ add,
                                                     const float*, float) {
    extern __shared__ __align__(16) float sx[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    const int U = FMT == 8 ? nb : nb >> 1;

    const uint8_t* rowp[R];
#pragma unroll
    for (int r = 0; r < R; r++) rowp[r] = W + (size_t)min(row0 + r, N - 1) * row_bytes;

    // Loads are unconditional, with the unit index clamped into the row, so
    // they never sit in a divergent branch (whose join would force a full
    // vmcnt wait); clamped duplicates re-read bytes already in flight.
    Units<R> b0, b1;
    load_units<R>(b0, rowp, min(lane, U - 1));  // in flight while x is staged

    stage_x<FMT>(sx, x, K, nb);
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

    // Two-deep ping-pong pipeline: unit u+64 is requested before unit u is used.
    for (int u = lane; u < U; u += 128) {
        load_units<R>(b1, rowp, min(u + 64, U - 1));
        if (FMT == 8) q8_compute<R>(b0, sx + u * XS8, acc);
        else q4_compute<R>(b0, sx + u * XS4, acc);
        if (u + 64 >= U) break;
        load_units<R>(b0, rowp, min(u + 128, U - 1));
        if (FMT == 8) q8_compute<R>(b1, sx + (u + 64) * XS8, acc);
        else q4_compute<R>(b1, sx + (u + 64) * XS4, acc);
    }
    int rr;
    float v = wave_reduce_rows<R>(acc, lane, &rr);
    if ((lane & (64 / R - 1)) == 0 && row0 + rr < N) y[row0 + rr] = add ? v + add[row0 + rr] : v;
}

// ----------------------------------------------------------------------------
// One-shot kernel (J <= 8 units per lane per row): every wave requests all
// R x J units it will use at entry, before x is staged, so the whole matrix is
// in flight almost at once; staging x (float4 loads) overlaps those loads.
// This is the main path: for the shapes of the decode path the kernel is a
// few microseconds long, and a load -> use -> load chain per wave would pay
// the HBM latency several times.
// ----------------------------------------------------------------------------
// The rows of one wave: returns row row0 + *rr's sum on the lanes with
// (lane & (64/R - 1)) == 0 (sx: the workgroup's x staging).  Q8 with whole
// blocks and aligned x requests x first, then the weights, then whatever
// tail() requests (the epilogue's operands), so the wait for x leaves the
// weights in flight and the epilogue finds its operands arrived.
template <int FMT, int R, int J, int XP, typename Tail>
__device__ __forceinline__ float oneshot_rows(const uint8_t* __restrict__ W, uint32_t row_bytes, int N, int K, int nb,
                                              const float* __restrict__ x, const float* __restrict__ xw, float eps,
                                              float* sx, int row0, int lane, int* rr, Tail&& tail) {
    const int U = FMT == 8 ? nb : nb >> 1;
    const bool two_phase = FMT == 8 && K == nb * 32 && (((uintptr_t)x) & 15) == 0 &&
                           (XP != XP_NORM || (((uintptr_t)xw) & 15) == 0);  // uniform

    const uint8_t* rowp[R];
#pragma unroll
    for (int r = 0; r < R; r++) rowp[r] = W + (size_t)min(row0 + r, N - 1) * row_bytes;

    XStage8<XP, J> xs;
    if (two_phase) xs.issue(x, xw, K);
    Units<R> w[J];
#pragma unroll
    for (int j = 0; j < J; j++) load_units<R>(w[j], rowp, min(lane + 64 * j, U - 1));
    __builtin_amdgcn_sched_barrier(0);  // tail's loads (and any wait they need) behind the weights
    tail();

    if (two_phase) xs.finish(sx, K, eps);
    else stage_x<FMT, XP>(sx, x, K, nb, xw, eps);
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int u = lane + 64 * j;
        if (u < U) {
            if (FMT == 8) q8_compute<R>(w[j], sx + u * XS8, acc);
            else q4_compute<R>(w[j], sx + u * XS4, acc);
        }
    }
    return wave_reduce_rows<R>(acc, lane, rr);
}

template <int FMT, int R, int J, int XP = XP_NONE>
__global__ __launch_bounds__(WG) void qmv_oneshot_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes, int N,
                                                        int K, int nb, const float* __restrict__ x,
                                                        float* __restrict__ y, const float* __restrict__ add,
                                                        const float* __restrict__ xw, float eps) {
    extern __shared__ __align__(16) float sx[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    // the residual of the row this lane stores, requested behind the weights
    // (without a residual the load reads x[0] and is not used)
    const float* ap = add ? add + min(row0 + reduced_row_of_lane<R>(lane), N - 1) : x;
    float addv = 0.f;
    int rr;
    const float v = oneshot_rows<FMT, R, J, XP>(W, row_bytes, N, K, nb, x, xw, eps, sx, row0, lane, &rr,
                                                [&]() { addv = *ap; });
    if ((lane & (64 / R - 1)) == 0 && row0 + rr < N) y[row0 + rr] = add ? v + addv : v;
}

// The one-shot kernel with the QKV epilogue (MvRope): a workgroup's 4R rows
// (an even count starting at an even row, so whole RoPE pairs) pass through
// LDS, and thread t < 2R takes the pair 2t, 2t+1: bias, rotation of q and k
// pairs (unfused products, the host-libm table), stores of q, k and v.
template <int FMT, int R, int J, int XP>
__global__ __launch_bounds__(WG) void qmv_oneshot_rope_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes,
                                                             int N, int K, int nb, const float* __restrict__ x,
                                                             const float* __restrict__ xw, float eps, MvRope rp) {
    extern __shared__ __align__(16) float sx[];
    __shared__ float s_y[4 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    const int t = threadIdx.x, r = blockIdx.x * 4 * R + 2 * t;
    const int hd = rp.hd, qd = rp.H * hd, kvd = rp.Hkv * hd, ps = rp.page_size;
    // the epilogue's operands, requested behind the weights: the position,
    // its page, the pair's bias and rotation (at a pair index clamped into
    // the rows; without a bias those loads read x and are not used)
    const int rc = min(r, N - 2);
    int p = 0, page = 0;
    float ba = 0.f, bb = 0.f, c = 0.f, sn = 0.f;
    int rr;
    const float v = oneshot_rows<FMT, R, J, XP>(W, row_bytes, N, K, nb, x, xw, eps, sx, row0, lane, &rr, [&]() {
        p = *rp.pos;
        page = rp.page_table[p / ps];
        const float* bp = rp.bias ? rp.bias + rc : x;
        ba = bp[0];
        bb = bp[1];
        const float* cs = rp.rope + (size_t)p * hd + rc % hd;
        c = cs[0];
        sn = cs[1];
    });
    if ((lane & (64 / R - 1)) == 0) s_y[wave * R + rr] = v;
    __syncthreads();
    if (t >= 2 * R || r >= N) return;
    float a = s_y[2 * t], b = s_y[2 * t + 1];
    if (rp.bias) {
        a = __fadd_rn(a, ba);
        b = __fadd_rn(b, bb);
    }
    const int off = p % ps;
    if (r < qd + kvd) {
        const int i = r % hd;  // even index inside the head
        const float ra = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, sn));
        const float rb = __fadd_rn(__fmul_rn(a, sn), __fmul_rn(b, c));
        if (r < qd) {
            rp.q_out[r] = ra;
            rp.q_out[r + 1] = rb;
        } else {
            const size_t o = (((size_t)page * rp.Hkv + (r - qd) / hd) * ps + off) * hd + i;
            if (rp.kv_dtype == DT_F16) {
                ((_Float16*)rp.kc)[o] = (_Float16)ra;
                ((_Float16*)rp.kc)[o + 1] = (_Float16)rb;
            } else {
                ((float*)rp.kc)[o] = ra;
                ((float*)rp.kc)[o + 1] = rb;
            }
        }
    } else {
        const int j = r - qd - kvd, vh = j / hd, dd = j % hd;
        if (rp.kv_dtype == DT_F16) {  // fp16 pages keep V dimension-major
            const size_t o = (((size_t)page * rp.Hkv + vh) * hd + dd) * ps + off;
            ((_Float16*)rp.vc)[o] = (_Float16)a;
            ((_Float16*)rp.vc)[o + ps] = (_Float16)b;
        } else {
            const size_t o = (((size_t)page * rp.Hkv + vh) * ps + off) * hd + dd;
            ((float*)rp.vc)[o] = a;
            ((float*)rp.vc)[o + 1] = b;
        }
    }
}

// ----------------------------------------------------------------------------
// Persistent streaming kernel: a grid of a few workgroups per CU; each WG
// stages x once, then each wave walks its share of (row group, unit column)
// steps with a two-deep ping-pong prefetch.  Waves drift out of phase, so
// one wave's dequantise-and-FMA work overlaps other waves' loads.
// ----------------------------------------------------------------------------
template <int FMT, int R>
__global__ __launch_bounds__(WG) void qmv_persist_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes, int N,
                                                        int K, int nb, const float* __restrict__ x,
                                                        float* __restrict__ y, const float* __restrict__ add,
                                                        const float*, float) {
    extern __shared__ __align__(16) float sx[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int U = FMT == 8 ? nb : nb >> 1;
    const int J = (U + 63) >> 6;
    const int ngroups = (N + R - 1) / R;
    const int gw = blockIdx.x * 4 + wave, nw = gridDim.x * 4;
    const int my_groups = gw < ngroups ? (ngroups - 1 - gw) / nw + 1 : 0;
    const int n_it = my_groups * J;

    // step it -> row group gw + (it / J) * nw, unit column it % J
    auto rows_of = [&](int it, const uint8_t* (&rp)[R]) {
        const int g = gw + (it / J) * nw;
#pragma unroll
        for (int r = 0; r < R; r++) rp[r] = W + (size_t)min(g * R + r, N - 1) * row_bytes;
    };
    auto unit_of = [&](int it) { return min(lane + 64 * (it % J), U - 1); };

    Units<R> b0, b1;
    const uint8_t* rp0[R];
    const uint8_t* rp1[R];
    if (n_it > 0) {
        rows_of(0, rp0);
        load_units<R>(b0, rp0, unit_of(0));
    }
    stage_x<FMT>(sx, x, K, nb);
    __syncthreads();
    if (n_it == 0) return;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

    auto finish = [&](int it) {  // after the last unit column of a row group
        const int g = gw + (it / J) * nw;
        int rr;
        float v = wave_reduce_rows<R>(acc, lane, &rr);
        if ((lane & (64 / R - 1)) == 0 && g * R + rr < N) y[g * R + rr] = add ? v + add[g * R + rr] : v;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
    };
    auto compute = [&](const Units<R>& b, int it) {
        const int u = lane + 64 * (it % J);
        if (u < U) {
            if (FMT == 8) q8_compute<R>(b, sx + u * XS8, acc);
            else q4_compute<R>(b, sx + u * XS4, acc);
        }
        if (it % J == J - 1) finish(it);
    };

    for (int it = 0; it < n_it; it += 2) {
        const int i1 = min(it + 1, n_it - 1);
        rows_of(i1, rp1);
        load_units<R>(b1, rp1, unit_of(i1));
        compute(b0, it);
        if (it + 1 >= n_it) break;
        const int i2 = min(it + 2, n_it - 1);
        rows_of(i2, rp0);
        load_units<R>(b0, rp0, unit_of(i2));
        compute(b1, it + 1);
    }
}

// ----------------------------------------------------------------------------
// Ring kernel (the default fast path).  What decides its speed, measured with
// per-wave timestamps on MI355X:
//  * x must reach LDS before the weight flood.  Every workgroup reads the same
//    x; requested behind ~10 MB of first weight loads it arrives ~3 us late and
//    holds every wave at the staging barrier.  Each thread's x loads are issued
//    first (XJ float4 per thread, branch-free: addresses are clamped and
//    out-of-range stores go to a spare LDS slot), and larger workgroups (NW
//    waves) cut the number of times the same x lines are requested.
//  * the weight ring must stay full: every step issues the loads of the step
//    D-1 ahead before touching the current one (a scheduling barrier keeps the
//    compiler from hoisting the current step's use above them), the loop body
//    has no branch around loads or their uses (ragged unit columns are masked
//    with a select, steps past the end recompute a duplicate and skip only the
//    store), and the residual values are loaded at entry, before x, so no late
//    load forces a full wait at the end of a row.
//  * every wave owns the same number of row groups (the launcher sizes the grid
//    so), otherwise the waves holding one extra group finish alone.
// Step it of a wave: row group gw + (it / J) * nw, unit column it % J.
// ----------------------------------------------------------------------------
constexpr int RING_KA = 4;  // row groups per wave whose residual values are preloaded

// Opaque redefinition of a step's registers: their uses cannot move above this
// point, so the compiler's wait for them lands here (after the next step's
// loads are issued), not at the loop latch where it would drain the ring.
template <int R>
__device__ __forceinline__ void pin_units(Units<R>& b) {
#pragma unroll
    for (int r = 0; r < R; r++) __asm__ volatile("" : "+v"(b.a[r]), "+v"(b.b[r]), "+v"(b.c[r])::"memory");
}

template <int R>
__device__ __forceinline__ void q8_compute_masked(const Units<R>& w, const float* xs, float (&acc)[R], bool valid) {
    const f32x4* xv = (const f32x4*)xs;
    f32x4 xr[8];
#pragma unroll
    for (int j = 0; j < 8; j++) xr[j] = xv[j];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float bs = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t d = dword(w, r, 1 + j);
#pragma unroll
            for (int k = 0; k < 4; k++) bs = __builtin_fmaf((float)(int8_t)(d >> (8 * k)), xr[j][k], bs);
        }
        const float t = __builtin_fmaf(bs, __builtin_bit_cast(float, dword(w, r, 0)), acc[r]);
        acc[r] = valid ? t : acc[r];
    }
}

template <int R>
__device__ __forceinline__ void q4_compute_masked(const Units<R>& w, const float* xu, float (&acc)[R], bool valid) {
    float t[R];
#pragma unroll
    for (int r = 0; r < R; r++) t[r] = acc[r];
    q4_compute<R>(w, xu, t);
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = valid ? t[r] : acc[r];
}

template <int FMT, int R, int XJ, int D, int NW, int XP = XP_NONE>
__global__ __launch_bounds__(64 * NW) void qmv_ring_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes, int N,
                                                          int K, int nb, const float* __restrict__ x, float* y,
                                                          const float* add, const float* __restrict__ xw, float eps) {
    extern __shared__ __align__(16) float sx[];
    constexpr int NT = 64 * NW;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int U = FMT == 8 ? nb : nb >> 1;
    const int J = (U + 63) >> 6;
    const int ngroups = (N + R - 1) / R;
    const int gw = blockIdx.x * NW + wave, nw = gridDim.x * NW;
    const int my_groups = gw < ngroups ? (ngroups - 1 - gw) / nw + 1 : 0;
    const int n_it = my_groups * J;
    const int t = threadIdx.x;
    const int rr = lane / (64 / R);  // the row of its group this lane stores after the reduction

    // 0. residual values of this lane's rows (the launcher guarantees my_groups <= RING_KA when add is set)
    float addv[RING_KA];
#pragma unroll
    for (int i = 0; i < RING_KA; i++)
        addv[i] = add ? add[min((gw + i * nw) * R + rr, N - 1)] : 0.f;

    // 1. x loads.  Q8: float4 f = t + NT i holds elements 4f..4f+3;
    //    Q4: 8-element group g = t + NT i = float4s 2g, 2g+1.  (K % 32 == 0,
    //    x 16-byte aligned.)  Slot k of xr holds x float4 xf[k]; the source
    //    is read raw first (twice the floats for the SiLU-gate), then x formed.
    constexpr int XL = FMT == 8 ? XJ : 2 * XJ;
    constexpr int SL = XP == XP_SILU_GATE ? 2 * XL : XL;
    const int n4 = K >> 2;
    int xf[XL];
    bool xok[XL];
#pragma unroll
    for (int i = 0; i < XJ; i++) {
        if (FMT == 8) {
            xok[i] = t + NT * i < n4;
            xf[i] = min(t + NT * i, n4 - 1);
        } else {
            const int g = t + NT * i;
            xok[2 * i] = xok[2 * i + 1] = g < (n4 >> 1);
            xf[2 * i] = 2 * min(g, (n4 >> 1) - 1);
            xf[2 * i + 1] = xf[2 * i] + 1;
        }
    }
    f32x4 raw[SL];
    f32x4 wr[XP == XP_NORM ? XL : 1];
#pragma unroll
    for (int k = 0; k < XL; k++) {
        if (XP == XP_SILU_GATE) {
            raw[2 * k] = *(const f32x4*)(x + 8 * xf[k]);
            raw[2 * k + 1] = *(const f32x4*)(x + 8 * xf[k] + 4);
        } else {
            raw[k] = *(const f32x4*)(x + 4 * xf[k]);
            if (XP == XP_NORM) wr[k] = *(const f32x4*)(xw + 4 * xf[k]);
        }
    }

    // Q8 requests the weight ring's first units right behind the x loads, so
    // the two round trips overlap (faster at 4096 x 4096 and 11008 x 4096); on Q4 the same
    // order measured 2-4% slower, so Q4 requests them after x is staged.
    constexpr bool early_ring = FMT == 8;
    const int last = max(n_it - 1, 0);
    auto issue = [&](int it, Units<R>& b) {
        const int i = min(it, last);
        const int g = gw + (i / J) * nw, j = i % J;
        const uint8_t* rp[R];
#pragma unroll
        for (int r = 0; r < R; r++) rp[r] = W + (size_t)min(g * R + r, N - 1) * row_bytes;
        load_units<R>(b, rp, min(lane + 64 * j, U - 1));
    };
    Units<R> buf[D];
    if constexpr (early_ring) {
#pragma unroll
        for (int d = 0; d < D - 1; d++) issue(d, buf[d]);
        __builtin_amdgcn_sched_barrier(0);
    }

    f32x4 xr[XL];
    if (XP == XP_NORM) {
        // 1 / sqrt(mean(x^2) + eps): this thread's elements, then the waves in order
        __shared__ float red[NW];
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < XL; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) ss = xok[k] ? __builtin_fmaf(raw[k][e], raw[k][e], ss) : ss;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = red[0];
#pragma unroll
        for (int w = 1; w < NW; w++) ss += red[w];
        const float r = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
        for (int k = 0; k < XL; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) xr[k][e] = __fmul_rn(__fmul_rn(raw[k][e], r), wr[k][e]);
    } else if (XP == XP_SILU_GATE) {
#pragma unroll
        for (int k = 0; k < XL; k++)
            xr[k] = f32x4{silu_gate(raw[2 * k][0], raw[2 * k][1]), silu_gate(raw[2 * k][2], raw[2 * k][3]),
                          silu_gate(raw[2 * k + 1][0], raw[2 * k + 1][1]), silu_gate(raw[2 * k + 1][2], raw[2 * k + 1][3])};
    } else {
#pragma unroll
        for (int k = 0; k < XL; k++) xr[k] = raw[k];
    }
    // 2. x into LDS (Q8: 36-float blocks; Q4: block pairs, odd elements
    //    scaled, plus block sums), the layout stage_x builds.
    if (FMT == 8) {
        const int spare = nb * XS8;
#pragma unroll
        for (int i = 0; i < XJ; i++) {
            const int f = t + NT * i;
            const int off = f < n4 ? (f >> 3) * XS8 + ((f & 7) << 2) : spare;
            *(f32x4*)(sx + off) = xr[i];
        }
    } else {
        const int spare = (nb >> 1) * XS4;
#pragma unroll
        for (int i = 0; i < XJ; i++) {
            const int g = t + NT * i;
            const f32x4 a = xr[2 * i], b = xr[2 * i + 1];
            float part = ((a[0] + a[2]) + (b[0] + b[2])) + ((a[1] + a[3]) + (b[1] + b[3]));
            part += __shfl_xor(part, 1);
            part += __shfl_xor(part, 2);
            const int blk = g >> 2, gg = g & 3;
            const bool ok = g < (n4 >> 1);
            const int base = ok ? (blk >> 1) * XS4 + (blk & 1) * 36 : spare;
            *(f32x4*)(sx + base + (ok ? gg * 8 : 0)) = q4_stage4(a[0], a[1], a[2], a[3]);
            *(f32x4*)(sx + base + (ok ? gg * 8 + 4 : 4)) = q4_stage4(b[0], b[1], b[2], b[3]);
            if (gg == 0) sx[base + (ok ? 32 : 8)] = part;
        }
    }

    // 3. the weight ring
    if constexpr (!early_ring) {
#pragma unroll
        for (int d = 0; d < D - 1; d++) issue(d, buf[d]);
    }
    __syncthreads();
    if (add) {
        // the residual values were requested before x: take them now, while
        // only the ring prologue is in flight behind them
#pragma unroll
        for (int i = 0; i < RING_KA; i++) __asm__ volatile("" : "+v"(addv[i]));
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    float add_cur = addv[0];
    float v_done = 0.f;  // the last finished row group's value (re-stored by steps past the end)
    // The loop body is branch-free: a branch inside it splits the live ranges of
    // the ring registers and the copies that follow wait for their loads.  So
    // every step reduces and stores: a row group's partial sums are stored
    // before its final sum (the same wave, the same address, in order), and a
    // step past the end stores the last finished value again.  (R divides N on
    // this path, so every stored row exists.)
    for (int it0 = 0; it0 < n_it; it0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int it = it0 + d;
            issue(it + D - 1, buf[(d + D - 1) % D]);
            __builtin_amdgcn_sched_barrier(0);
            pin_units<R>(buf[d]);
            const int i = min(it, last);
            const int j = i % J;
            const int u = lane + 64 * j;
            const bool valid = u < U && it < n_it;
            const int uc = min(u, U - 1);
            if (FMT == 8) q8_compute_masked<R>(buf[d], sx + uc * XS8, acc, valid);
            else q4_compute_masked<R>(buf[d], sx + uc * XS4, acc, valid);
            float red[R];
#pragma unroll
            for (int r = 0; r < R; r++) red[r] = acc[r];
            int rrr;
            const float v = wave_reduce_rows<R>(red, lane, &rrr) + add_cur;
            const bool fin = j == J - 1;
            const float vs = it < n_it ? v : v_done;
            const int g = gw + (i / J) * nw;
            y[g * R + rr] = vs;
            v_done = fin ? vs : v_done;
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = fin ? 0.f : acc[r];
#pragma unroll
            for (int k = 0; k + 1 < RING_KA; k++) addv[k] = fin ? addv[k + 1] : addv[k];
            add_cur = fin ? addv[0] : add_cur;
        }
    }
}

// ----------------------------------------------------------------------------
// General path: any block size, any alignment (byte loads).  One wave per row;
// lane l takes blocks l, l+64, ...  Follows the reference's block geometry
// exactly, including the Q4 odd-tail rule (this_block/2 pairs).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(WG) void qmv_generic_kernel(const uint8_t* __restrict__ W, uint32_t dtype,
                                                        int bs, size_t row_bytes, int N, int K,
                                                        const float* __restrict__ x, float* __restrict__ y,
                                                        const float* __restrict__ add) {
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
    if (lane == 0) y[row] = add ? part + add[row] : part;
}

// f32 weights (reference dispatch_matvec_opt, backend.cpp:62-105; used for F32
// projection weights and the tied f32 lm_head).  One wave per row, float4 loads.
__global__ __launch_bounds__(WG) void mv_f32_kernel(const float* __restrict__ W, const float* __restrict__ x,
                                                   float* __restrict__ y, int N, int K, const float* __restrict__ add) {
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
    if (lane == 0) y[row] = add ? part + add[row] : part;
}

// ----------------------------------------------------------------------------
// Launchers
// ----------------------------------------------------------------------------
static int g_rows_per_wave = 0;  // 0: automatic; else 1, 2, 4 or 8
static int g_kernel = 0;         // 0: automatic, 1: one-shot, 2: persistent streaming, 3 / 4: ring, 8 / 4 waves per workgroup
static int g_wgs_per_cu = 0;     // persistent / ring grid size per CU (0: automatic)

static std::atomic<uint32_t> g_tuning_gen{0};
uint32_t tuning_generation() { return g_tuning_gen.load(std::memory_order_relaxed); }
void bump_tuning_generation() { g_tuning_gen.fetch_add(1, std::memory_order_relaxed); }

int set_matvec_tuning(int kernel, int r, int wgs_per_cu) {
    QH_REQUIRE(r == 0 || r == 1 || r == 2 || r == 4 || r == 8, QRAF_HIP_ERR_INVALID,
               "rows per wave must be 0 (auto), 1, 2, 4 or 8");
    QH_REQUIRE(kernel >= 0 && kernel <= 4, QRAF_HIP_ERR_INVALID, "kernel must be 0..4");
    QH_REQUIRE(wgs_per_cu >= 0 && wgs_per_cu <= 16, QRAF_HIP_ERR_INVALID, "workgroups per CU must be 0..16");
    g_rows_per_wave = r;
    g_kernel = kernel;
    g_wgs_per_cu = wgs_per_cu;
    bump_tuning_generation();
    return QRAF_HIP_OK;
}

static int cu_count() {
    static int n = 0;
    if (!n) {
        int d = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&d) == hipSuccess && hipGetDeviceProperties(&p, d) == hipSuccess) n = p.multiProcessorCount;
        if (n <= 0) n = 256;
    }
    return n;
}

typedef void (*qmv_fn)(const uint8_t*, uint32_t, int, int, int, const float*, float*, const float*, const float*,
                       float);

// workgroups of `threads` threads and `lds` bytes of LDS that fit on one CU at
// once (cached per kernel and LDS size: the launch path calls this per matvec)
static hipError_t resident_wgs(const void* kf, int threads, size_t lds, int* out) {
    struct Entry { const void* k; size_t lds; int n; };
    thread_local Entry cache[64];
    thread_local int used = 0;
    for (int i = 0; i < used; i++)
        if (cache[i].k == kf && cache[i].lds == lds) { *out = cache[i].n; return hipSuccess; }
    int n = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kf, threads, lds);
    if (e != hipSuccess) return e;
    if (used < 64) cache[used++] = {kf, lds, n};
    *out = n;
    return hipSuccess;
}

// one-shot instances: R * J <= 8; with x formed in the kernel (XP) for J <= 4
template <int FMT, int R, int J, int XP>
static qmv_fn oneshot_if_valid() {
    if constexpr (R * J <= 8 && (XP == XP_NONE || J <= 4)) return qmv_oneshot_kernel<FMT, R, J, XP>;
    else return nullptr;
}
template <int FMT, int R, int XP>
static qmv_fn pick_oneshot(int J) {
    switch (J) {
        case 1: return oneshot_if_valid<FMT, R, 1, XP>();
        case 2: return oneshot_if_valid<FMT, R, 2, XP>();
        case 3: return oneshot_if_valid<FMT, R, 3, XP>();
        case 4: return oneshot_if_valid<FMT, R, 4, XP>();
        case 5: return oneshot_if_valid<FMT, R, 5, XP>();
        case 6: return oneshot_if_valid<FMT, R, 6, XP>();
        case 7: return oneshot_if_valid<FMT, R, 7, XP>();
        case 8: return oneshot_if_valid<FMT, R, 8, XP>();
        default: return nullptr;
    }
}
template <int FMT, int XP>
static qmv_fn pick_oneshot_r(int R, int J) {
    switch (R) {
        case 1: return pick_oneshot<FMT, 1, XP>(J);
        case 2: return pick_oneshot<FMT, 2, XP>(J);
        case 4: return pick_oneshot<FMT, 4, XP>(J);
        default: return pick_oneshot<FMT, 8, XP>(J);
    }
}
template <int FMT>
static qmv_fn pick_oneshot_xp(int R, int J, int xp) {
    if (xp == XP_NORM) return pick_oneshot_r<FMT, XP_NORM>(R, J);
    if (xp == XP_SILU_GATE) return pick_oneshot_r<FMT, XP_SILU_GATE>(R, J);
    return pick_oneshot_r<FMT, XP_NONE>(R, J);
}
// one-shot instances with the QKV epilogue: x formed as RMSNorm(x) * w in
// staging (the layer's attention norm), R * J <= 8, J <= 4
typedef void (*qmv_rope_fn)(const uint8_t*, uint32_t, int, int, int, const float*, const float*, float, MvRope);
template <int FMT, int R, int J>
static qmv_rope_fn rope_if_valid() {
    if constexpr (R * J <= 8 && J <= 4) return qmv_oneshot_rope_kernel<FMT, R, J, XP_NORM>;
    else return nullptr;
}
template <int FMT, int R>
static qmv_rope_fn pick_rope_j(int J) {
    switch (J) {
        case 1: return rope_if_valid<FMT, R, 1>();
        case 2: return rope_if_valid<FMT, R, 2>();
        case 3: return rope_if_valid<FMT, R, 3>();
        case 4: return rope_if_valid<FMT, R, 4>();
        default: return nullptr;
    }
}
template <int FMT>
static qmv_rope_fn pick_rope(int R, int J) {
    switch (R) {
        case 1: return pick_rope_j<FMT, 1>(J);
        case 2: return pick_rope_j<FMT, 2>(J);
        case 4: return pick_rope_j<FMT, 4>(J);
        default: return pick_rope_j<FMT, 8>(J);
    }
}

template <int FMT>
static qmv_fn pick_stream(int R) {
    switch (R) {
        case 1: return qmv_stream_kernel<FMT, 1>;
        case 2: return qmv_stream_kernel<FMT, 2>;
        default: return qmv_stream_kernel<FMT, 4>;
    }
}

// ring kernel instances: XJ in {1, 2, 4, 8, 12} (x loads per thread, rounded
// up; the extra loads are clamped duplicates), R in {1, 2}, D = 2, NW in
// {4, 8}; x formed in the kernel (XP) with NW = 8 only
template <int FMT, int R, int NW, int XP>
static qmv_fn pick_ring_xj(int xj) {
    if constexpr (NW == 4 && XP != XP_NONE) {
        return nullptr;
    } else {
        if (xj <= 1) return qmv_ring_kernel<FMT, R, 1, 2, NW, XP>;
        if (xj <= 2) return qmv_ring_kernel<FMT, R, 2, 2, NW, XP>;
        if (xj <= 4) return qmv_ring_kernel<FMT, R, 4, 2, NW, XP>;
        if (xj <= 8) return qmv_ring_kernel<FMT, R, 8, 2, NW, XP>;
        if (xj <= 12) return qmv_ring_kernel<FMT, R, 12, 2, NW, XP>;
        return nullptr;
    }
}
template <int FMT, int XP>
static qmv_fn pick_ring_r(int R, int NW, int xj) {
    if (R == 1) return NW == 4 ? pick_ring_xj<FMT, 1, 4, XP>(xj) : pick_ring_xj<FMT, 1, 8, XP>(xj);
    return NW == 4 ? pick_ring_xj<FMT, 2, 4, XP>(xj) : pick_ring_xj<FMT, 2, 8, XP>(xj);
}
template <int FMT>
static qmv_fn pick_ring(int R, int NW, int xj, int xp) {
    if (xp == XP_NORM) return pick_ring_r<FMT, XP_NORM>(R, NW, xj);
    if (xp == XP_SILU_GATE) return pick_ring_r<FMT, XP_SILU_GATE>(R, NW, xj);
    return pick_ring_r<FMT, XP_NONE>(R, NW, xj);
}

// x formed by a kernel of its own (for the matvec kernels that cannot form it)
__global__ __launch_bounds__(256) void xprep_norm_kernel(const float* __restrict__ x, const float* __restrict__ w, int K,
                                                         float eps, float* __restrict__ out) {
    const float r = norm_r_256(x, K, eps);
    for (int i = threadIdx.x; i < K; i += 256) out[i] = __fmul_rn(__fmul_rn(x[i], r), w[i]);
}
__global__ void xprep_silu_gate_kernel(const float* __restrict__ x, int K, float* __restrict__ out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < K; i += gridDim.x * blockDim.x)
        out[i] = silu_gate(x[2 * i], x[2 * i + 1]);
}
static int launch_xprep(const float* x, const MvPrep& p, int K, hipStream_t s) {
    QH_REQUIRE(p.xbuf, QRAF_HIP_ERR_INVALID, "matvec: this kernel needs a scratch buffer to form x");
    if (p.op == XP_NORM) {
        QH_REQUIRE(p.w, QRAF_HIP_ERR_INVALID, "matvec: norm weights missing");
        hipLaunchKernelGGL(xprep_norm_kernel, dim3(1), dim3(256), 0, s, x, p.w, K, p.eps, p.xbuf);
    } else {
        hipLaunchKernelGGL(xprep_silu_gate_kernel, dim3(std::min((K + 255) / 256, 1024)), dim3(256), 0, s, x, K, p.xbuf);
    }
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_matvec_q(const void* Wv, uint32_t dtype, int bs, uint32_t N, uint32_t K, const float* x, float* y,
                    hipStream_t s, const float* add, const MvPrep* prep, const MvRope* rope, bool* fused) {
    if (fused) *fused = false;
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "unsupported weight dtype %u", dtype);
    QH_REQUIRE(bs > 0 && bs <= 4096, QRAF_HIP_ERR_INVALID, "bad block size %d", bs);
    QH_REQUIRE(K > 0 && N > 0, QRAF_HIP_ERR_INVALID, "empty matvec (%u x %u)", N, K);
    QH_REQUIRE(Wv && x && y, QRAF_HIP_ERR_INVALID, "null pointer");
    int xp = prep ? prep->op : XP_NONE;
    QH_REQUIRE(xp == XP_NONE || xp == XP_NORM || xp == XP_SILU_GATE, QRAF_HIP_ERR_INVALID, "matvec: bad x op %d", xp);
    QH_REQUIRE(xp != XP_NORM || prep->w, QRAF_HIP_ERR_INVALID, "matvec: norm weights missing");
    const float* xw = xp == XP_NORM ? prep->w : nullptr;
    const float eps = xp == XP_NORM ? prep->eps : 0.f;
    // kernels that cannot form x: a prep kernel writes it to the scratch buffer first
    auto plain_x = [&]() -> int {
        if (xp == XP_NONE) return QRAF_HIP_OK;
        QH_TRY(launch_xprep(x, *prep, (int)K, s));
        x = prep->xbuf;
        xp = XP_NONE;
        xw = nullptr;
        return QRAF_HIP_OK;
    };
    const uint8_t* W = (const uint8_t*)Wv;
    const size_t rb = q_row_bytes(dtype, bs, K);
    const int nb = (int)((K + bs - 1) / bs);
    const size_t lds = dtype == DT_Q8_0 ? (size_t)nb * XS8 * 4 : (size_t)(nb / 2) * XS4 * 4;
    const bool fast = bs == 32 && (((uintptr_t)W) & 3) == 0 && (dtype == DT_Q8_0 || (nb % 2) == 0) &&
                      lds <= 160 * 1024 && rb <= 0xFFFFFFFFu;
    if (fast) {
        const int U = dtype == DT_Q8_0 ? nb : nb / 2;
        const int J = (U + 63) / 64;
        // Automatic choice (measured on MI355X, weights streamed from HBM): the
        // one-shot kernel below ~6 MB of weights (it has the whole matrix in
        // flight at once), else the ring kernel: Q8 one row per wave, 8-wave
        // workgroups, 2 per CU; Q4 one row per wave, 1 such workgroup per CU,
        // or for N >= 8192 two rows per wave in 4-wave workgroups, 4 per CU
        // (8-wave workgroups when the kernel forms x itself).
        const bool big = (size_t)N * rb >= ((size_t)6 << 20);
        const bool q4_wide = dtype == DT_Q4_0 && N >= 8192;
        int kern_req = g_kernel;
        if (kern_req == 0 && big) kern_req = q4_wide && xp == XP_NONE ? 4 : 3;
        const int NWr = kern_req == 4 && xp == XP_NONE ? 4 : 8;  // waves per workgroup
        const int xj = dtype == DT_Q8_0 ? (int)((K + 64 * NWr * 4 - 1) / (64 * NWr * 4))
                                        : (int)((K + 64 * NWr * 8 - 1) / (64 * NWr * 8));
        // the ring kernel needs whole blocks, a 16-byte aligned x and x within its staging
        const bool ring_ok = (K % 32) == 0 && (((uintptr_t)x) & 15) == 0 && (((uintptr_t)xw) & 15) == 0 &&
                             xj <= 12 && lds + 64 <= 160 * 1024;
        int kern = kern_req;
        if (kern == 0) kern = (N >= 8192 && J <= 8) ? 2 : 1;
        if ((kern == 3 || kern == 4) && ring_ok) {
            // two rows per wave for short rows too (at most 32 units: most lanes
            // would hold no unit of a single row)
            int R = g_rows_per_wave ? min(g_rows_per_wave, 2)
                                    : (g_kernel == 0 && ((q4_wide && NWr == 4) || U <= 32) ? 2 : 1);
            if (N % R) R = 1;  // every stored row must exist
            qmv_fn kf = dtype == DT_Q8_0 ? pick_ring<8>(R, NWr, xj, xp) : pick_ring<4>(R, NWr, xj, xp);
            QH_REQUIRE(kf, QRAF_HIP_ERR_INVALID, "no ring matvec kernel for K=%u", K);
            const size_t lds_r = lds + 16 * sizeof(float);  // + the spare slot for out-of-range x stores
            if (lds_r > 65536)
                QH_CHECK_HIP(hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_r));
            // never more workgroups per CU than fit at once (the rest would run as a second round)
            int fit = 0;
            QH_CHECK_HIP(resident_wgs((const void*)kf, 64 * NWr, lds_r, &fit));
            const int dflt = dtype == DT_Q8_0 ? 16 / NWr : (q4_wide && NWr == 4 ? 4 : 1);
            const int wgs_per_cu = max(1, min(g_wgs_per_cu ? g_wgs_per_cu : dflt, fit));
            // equal row groups per wave: k = ceil(groups / max waves), then as few waves as hold k
            // each; with a residual every wave must hold at most RING_KA groups
            const int ngroups = (int)((N + R - 1) / R);
            int wmax = wgs_per_cu * NWr * cu_count();
            if (add) wmax = max(wmax, (ngroups + RING_KA - 1) / RING_KA);
            const int k = (ngroups + wmax - 1) / wmax;
            const int waves = (ngroups + k - 1) / k;
            const int grid = (waves + NWr - 1) / NWr;
            hipLaunchKernelGGL(kf, dim3(grid), dim3(64 * NWr), lds_r, s, W, (uint32_t)rb, (int)N, (int)K, nb, x, y, add,
                               xw, eps);
            QH_CHECK_HIP(hipGetLastError());
            return QRAF_HIP_OK;
        }
        // persistent kernel when the ring does not apply and there are many rows, else one-shot
        if (kern >= 3) kern = (N >= 8192 && J <= 8) ? 2 : 1;
        if (kern == 2 || J > 8) {
            QH_TRY(plain_x());
            const int R = g_rows_per_wave ? min(g_rows_per_wave, 4) : (dtype == DT_Q8_0 ? 1 : 2);
            const int ngroups = (int)((N + R - 1) / R);
            const int per_cu = g_wgs_per_cu ? g_wgs_per_cu : (dtype == DT_Q8_0 ? 4 : 2);
            const int grid = max(1, min((ngroups + 3) / 4, per_cu * cu_count()));
            qmv_fn k = nullptr;
            if (dtype == DT_Q8_0) k = R == 1 ? qmv_persist_kernel<8, 1> : R == 2 ? qmv_persist_kernel<8, 2> : qmv_persist_kernel<8, 4>;
            else k = R == 1 ? qmv_persist_kernel<4, 1> : R == 2 ? qmv_persist_kernel<4, 2> : qmv_persist_kernel<4, 4>;
            if (lds > 65536)
                QH_CHECK_HIP(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
            hipLaunchKernelGGL(k, dim3(grid), dim3(WG), lds, s, W, (uint32_t)rb, (int)N, (int)K, nb, x, y, add, xw, eps);
            QH_CHECK_HIP(hipGetLastError());
            return QRAF_HIP_OK;
        }
        int R = g_rows_per_wave;
        if (R == 0) {
            // as many rows per wave as the register budget allows (R*J <= 8),
            // but keep at least ~256 workgroups so every CU streams
            R = 8;
            while (R > 1 && (R * J > 8 || (N + 4 * R - 1) / (4 * R) < 256)) R >>= 1;
        } else {
            while (R > 1 && R * J > 8) R >>= 1;
        }
        if (rope && fused && xp == XP_NORM && !add && (N % 2) == 0 && rope->hd % 2 == 0 &&
            (int)N == (rope->H + 2 * rope->Hkv) * rope->hd &&
            (rope->kv_dtype == DT_F32 || rope->kv_dtype == DT_F16)) {
            const qmv_rope_fn kr = dtype == DT_Q8_0 ? pick_rope<8>(R, J) : pick_rope<4>(R, J);
            if (kr) {
                if (lds > 65536)
                    QH_CHECK_HIP(hipFuncSetAttribute((const void*)kr, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)lds));
                hipLaunchKernelGGL(kr, dim3((N + 4 * R - 1) / (4 * R)), dim3(WG), lds, s, W, (uint32_t)rb, (int)N,
                                   (int)K, nb, x, xw, eps, *rope);
                QH_CHECK_HIP(hipGetLastError());
                *fused = true;
                return QRAF_HIP_OK;
            }
        }
        qmv_fn k = dtype == DT_Q8_0 ? pick_oneshot_xp<8>(R, J, xp) : pick_oneshot_xp<4>(R, J, xp);
        if (!k) {  // no one-shot instance forms this x (J > 4): prepare it separately
            QH_TRY(plain_x());
            k = dtype == DT_Q8_0 ? pick_oneshot_xp<8>(R, J, XP_NONE) : pick_oneshot_xp<4>(R, J, XP_NONE);
        }
        QH_REQUIRE(k, QRAF_HIP_ERR_INVALID, "no matvec kernel for R=%d J=%d", R, J);
        if (lds > 65536)
            QH_CHECK_HIP(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(k, dim3((N + 4 * R - 1) / (4 * R)), dim3(WG), lds, s, W, (uint32_t)rb, (int)N, (int)K, nb,
                           x, y, add, xw, eps);
        QH_CHECK_HIP(hipGetLastError());
        return QRAF_HIP_OK;
    }
    QH_TRY(plain_x());
    hipLaunchKernelGGL(qmv_generic_kernel, dim3((N + 3) / 4), dim3(WG), 0, s, W, dtype, bs, rb, (int)N, (int)K, x, y,
                       add);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

// ----------------------------------------------------------------------------
// Several vectors at once (dispatch_matvec_q, backend.cpp:131-199, applied to
// each of nv rows of x): the persistent streaming form above with NV >= nv x
// vectors staged in LDS (each formed as the batch-1 kernels form x: as is,
// RMSNorm or SiLU-gate), each weight unit loaded once and applied to every
// vector.  A unit's quants are converted to floats once; each vector's sum
// then runs the batch-1 compute's exact sequence (q8_compute / q4_compute,
// R = 1), so a row's result is the batch-1 persistent kernel's.  For batches
// below the matrix cores' reach: no split-K partials, no activation planes,
// one launch.  Vectors past nv repeat the last one and are not stored.
// ----------------------------------------------------------------------------
// Staging of NV vectors at once (rows min(v, nv - 1) of x, ldx floats apart)
// into sx + v * S in stage_x's layout and arithmetic, with every thread's
// loads of up to 8 elements groups requested together (a chunk of 8 per
// thread per round trip over all vectors), where stage_x's loop would wait
// for each group: vector-major (v, group) indices, so the four threads of a
// Q4 block are consecutive lanes of one vector.  The RMSNorm factors come
// first, from norm_r_256's strided sums for all vectors in one pass.
template <int FMT, int XP, int NV>
__device__ __forceinline__ void stage_x_batch(float* sx, int S, const float* __restrict__ x, int ldx, int nv, int K,
                                              int nb, const float* __restrict__ xw, float eps) {
    __shared__ float red[NV][4];
    __shared__ float s_r[NV];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (XP == XP_NORM) {
        float ss[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) ss[v] = 0.f;
#pragma unroll 4
        for (int i = tid; i < K; i += 256)
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const float a = x[(size_t)min(v, nv - 1) * ldx + i];
                ss[v] = __builtin_fmaf(a, a, ss[v]);
            }
#pragma unroll
        for (int v = 0; v < NV; v++) {
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss[v] += __shfl_xor(ss[v], o);
            if (lane == 0) red[v][wave] = ss[v];
        }
        __syncthreads();
        if (tid < NV) s_r[tid] = 1.0f / sqrtf(((red[tid][0] + red[tid][1]) + (red[tid][2] + red[tid][3])) / (float)K + eps);
        __syncthreads();
    }
    const bool vec = (((uintptr_t)x) & 15) == 0 && (ldx & 3) == 0 && (XP != XP_NORM || (((uintptr_t)xw) & 15) == 0);
    constexpr int CH = 8;  // element groups per thread per round trip
    if (FMT == 8) {
        const int n4 = nb * 8;  // float4 groups per vector (K padded to whole blocks)
        const int total = NV * n4;
        for (int base = 0; base < total; base += 256 * CH) {
            f32x4 g[CH];
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int c = min(base + tid + 256 * u, total - 1);
                const int v = c / n4, i = 4 * (c - v * n4);
                const float* xs = x + (size_t)min(v, nv - 1) * ldx;
                const float r = XP == XP_NORM ? s_r[v] : 1.f;
                if (i + 3 < K && vec) {
                    g[u] = x_vec4<XP>(xs, i, r, xw);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) g[u][e] = (i + e < K) ? x_elem<XP>(xs, i + e, r, xw) : 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int c = base + tid + 256 * u;
                if (c < total) {
                    const int v = c / n4, i = 4 * (c - v * n4);
                    *(f32x4*)(sx + v * S + (i >> 5) * XS8 + (i & 31)) = g[u];
                }
            }
        }
    } else {
        const int Keff = K & ~1;
        const int ng = nb * 4;  // 8-element groups per vector
        const int total = NV * ng;
        for (int base = 0; base < total; base += 256 * CH) {
            float g[CH][8];
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int c = min(base + tid + 256 * u, total - 1);
                const int v = c / ng, i = 8 * (c - v * ng);
                const float* xs = x + (size_t)min(v, nv - 1) * ldx;
                const float r = XP == XP_NORM ? s_r[v] : 1.f;
                if (i + 7 < Keff && vec) {
                    const f32x4 a = x_vec4<XP>(xs, i, r, xw), b = x_vec4<XP>(xs, i + 4, r, xw);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        g[u][e] = a[e];
                        g[u][4 + e] = b[e];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) g[u][e] = (i + e < Keff) ? x_elem<XP>(xs, i + e, r, xw) : 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int c = base + tid + 256 * u;  // lanes of a block: consecutive, one vector (ng % 4 == 0)
                const float* v8 = g[u];
                float part = ((v8[0] + v8[2]) + (v8[4] + v8[6])) + ((v8[1] + v8[3]) + (v8[5] + v8[7]));
                part += __shfl_xor(part, 1);
                part += __shfl_xor(part, 2);
                if (c < total) {
                    const int v = c / ng, t = c - v * ng, i = 8 * t;
                    const int blk = i >> 5, gg = (i & 31) >> 3;
                    float* dst = sx + v * S + (blk >> 1) * XS4 + (blk & 1) * 36;
                    *(f32x4*)(dst + gg * 8) = q4_stage4(v8[0], v8[1], v8[2], v8[3]);
                    *(f32x4*)(dst + gg * 8 + 4) = q4_stage4(v8[4], v8[5], v8[6], v8[7]);
                    if ((t & 3) == 0) dst[32] = part;
                }
            }
        }
    }
}

template <int FMT, int NV, int XP>
__global__ __launch_bounds__(WG) void qmv_batch_kernel(const uint8_t* __restrict__ W, uint32_t row_bytes, int N, int K,
                                                       int nb, const float* __restrict__ x, int ldx, int nv,
                                                       float* __restrict__ y, int ldy, const float* __restrict__ add,
                                                       const float* __restrict__ xw, float eps) {
    extern __shared__ __align__(16) float sx[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int U = FMT == 8 ? nb : nb >> 1;
    const int J = (U + 63) >> 6;
    const int S = FMT == 8 ? nb * XS8 : (nb >> 1) * XS4;  // staged floats per vector
    const int gw = blockIdx.x * 4 + wave, nw = gridDim.x * 4;
    const int my_rows = gw < N ? (N - 1 - gw) / nw + 1 : 0;
    const int n_it = my_rows * J;

    // step it -> row gw + (it / J) * nw, unit column it % J
    auto row_of = [&](int it) { return W + (size_t)min(gw + (it / J) * nw, N - 1) * row_bytes; };
    auto unit_of = [&](int it) { return min(lane + 64 * (it % J), U - 1); };

    Units<1> b0, b1;
    if (n_it > 0) {
        const uint8_t* rp[1] = {row_of(0)};
        load_units<1>(b0, rp, unit_of(0));
    }
    stage_x_batch<FMT, XP, NV>(sx, S, x, ldx, nv, K, nb, xw, eps);
    __syncthreads();
    if (n_it == 0) return;

    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) acc[v] = 0.f;

    auto compute = [&](const Units<1>& w, int it) {
        const int u = lane + 64 * (it % J);
        if (u < U) {
            if (FMT == 8) {
                float q[32];
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int k = 0; k < 4; k++) q[4 * j + k] = (float)(int8_t)(dword(w, 0, 1 + j) >> (8 * k));
                const float sc = __builtin_bit_cast(float, dword(w, 0, 0));
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const f32x4* xv = (const f32x4*)(sx + v * S + u * XS8);
                    f32x4 xr[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) xr[j] = xv[j];
                    float bs = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; j++)
#pragma unroll
                        for (int k = 0; k < 4; k++) bs = __builtin_fmaf(q[4 * j + k], xr[j][k], bs);
                    acc[v] = __builtin_fmaf(bs, sc, acc[v]);
                }
            } else {
                uint32_t dw[9];
#pragma unroll
                for (int i = 0; i < 9; i++) dw[i] = dword(w, 0, i);
                // the even and odd block's nibbles in element order, as the values
                // q4_compute multiplies (n * 2^-24, odd elements 16n * 2^-24)
                float we[32], wo[32];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    uint32_t te[4], to[4];
                    q4_split(__builtin_amdgcn_alignbyte(dw[k + 1], dw[k], 2), te);
                    q4_split(dw[5 + k], to);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        we[8 * k + q] = half_lo(te[q]);
                        we[8 * k + 4 + q] = half_hi(te[q]);
                        wo[8 * k + q] = half_lo(to[q]);
                        wo[8 * k + 4 + q] = half_hi(to[q]);
                    }
                }
                const float se = half_bits_to_float(dw[0]) * 0x1p24f, so = half_bits_to_float(dw[4] >> 16) * 0x1p24f;
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const float* xu = sx + v * S + u * XS4;
                    f32x4 xe[8], xo[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        xe[j] = ((const f32x4*)xu)[j];
                        xo[j] = ((const f32x4*)(xu + 36))[j];
                    }
                    const float se8 = 0x1p-21f * xu[32], so8 = 0x1p-21f * xu[36 + 32];
                    float be = 0.f, bo = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; j++)
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            be = __builtin_fmaf(we[4 * j + q], xe[j][q], be);
                            bo = __builtin_fmaf(wo[4 * j + q], xo[j][q], bo);
                        }
                    acc[v] = __builtin_fmaf(be - se8, se, acc[v]);
                    acc[v] = __builtin_fmaf(bo - so8, so, acc[v]);
                }
            }
        }
        if (it % J == J - 1) {  // the row's last unit column: reduce and store each vector's sum
            const int row = gw + (it / J) * nw;
#pragma unroll
            for (int v = 0; v < NV; v++) {
                float a1[1] = {acc[v]};
                int rr;
                const float t = wave_reduce_rows<1>(a1, lane, &rr);
                if (lane == 0 && v < nv && row < N) {
                    const size_t e = (size_t)v * ldy + row;
                    y[e] = add ? t + add[e] : t;
                }
                acc[v] = 0.f;
            }
        }
    };

    for (int it = 0; it < n_it; it += 2) {
        const uint8_t* rp1[1] = {row_of(min(it + 1, n_it - 1))};
        load_units<1>(b1, rp1, unit_of(min(it + 1, n_it - 1)));
        compute(b0, it);
        if (it + 1 >= n_it) break;
        const uint8_t* rp0[1] = {row_of(min(it + 2, n_it - 1))};
        load_units<1>(b0, rp0, unit_of(min(it + 2, n_it - 1)));
        compute(b1, it + 1);
    }
}

// bytes of LDS the batch kernel stages nv vectors of K elements in (0: not coverable)
static size_t batch_lds(uint32_t dtype, uint32_t K, int nv) {
    if ((dtype != DT_Q8_0 && dtype != DT_Q4_0) || K == 0 || K % 32 != 0 || nv < 1 || nv > MV_BATCH_MAX) return 0;
    const int nb = (int)(K / 32);
    if (dtype == DT_Q4_0 && nb % 2 != 0) return 0;
    const int NV = nv <= 2 ? 2 : nv <= 4 ? 4 : nv <= 8 ? 8 : 16;
    const size_t per = dtype == DT_Q8_0 ? (size_t)nb * XS8 * 4 : (size_t)(nb / 2) * XS4 * 4;
    const size_t lds = per * NV;
    return lds <= MV_BATCH_LDS ? lds : 0;
}

bool matvec_batch_ok(uint32_t dtype, uint32_t K, int nv) { return batch_lds(dtype, K, nv) != 0; }

int launch_matvec_q_batch(const void* Wv, uint32_t dtype, uint32_t N, uint32_t K, const float* x, int ldx, int nv,
                          float* y, int ldy, hipStream_t s, const float* add, const MvPrep* prep) {
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "batch matvec: unsupported dtype %u", dtype);
    QH_REQUIRE(Wv && x && y && N > 0 && K > 0, QRAF_HIP_ERR_INVALID, "batch matvec: null pointer or empty shape");
    QH_REQUIRE(nv >= 1 && nv <= MV_BATCH_MAX, QRAF_HIP_ERR_INVALID, "batch matvec: %d vectors (1..%d)", nv,
               MV_BATCH_MAX);
    const int xp = prep ? prep->op : XP_NONE;
    QH_REQUIRE(xp == XP_NONE || xp == XP_NORM || xp == XP_SILU_GATE, QRAF_HIP_ERR_INVALID, "batch matvec: x op %d", xp);
    QH_REQUIRE(xp != XP_NORM || prep->w, QRAF_HIP_ERR_INVALID, "batch matvec: norm weights missing");
    const int xlen = xp == XP_SILU_GATE ? 2 * (int)K : (int)K;
    QH_REQUIRE(ldx >= xlen && ldy >= (int)N, QRAF_HIP_ERR_INVALID, "batch matvec: row strides %d / %d too short", ldx,
               ldy);
    const size_t lds = batch_lds(dtype, K, nv);
    QH_REQUIRE(lds, QRAF_HIP_ERR_INVALID,
               "batch matvec: K=%u (a multiple of 32; of 64 for Q4_0) and %d vectors must fit %d bytes of LDS", K, nv,
               MV_BATCH_LDS);
    QH_REQUIRE((((uintptr_t)Wv) & 3) == 0, QRAF_HIP_ERR_INVALID, "batch matvec: weights must be 4-byte aligned");
    const int NV = nv <= 2 ? 2 : nv <= 4 ? 4 : nv <= 8 ? 8 : 16;
    const float* xw = xp == XP_NORM ? prep->w : nullptr;
    const float eps = xp == XP_NORM ? prep->eps : 0.f;
    typedef void (*fn)(const uint8_t*, uint32_t, int, int, int, const float*, int, int, float*, int, const float*,
                       const float*, float);
    fn k = nullptr;
#define QH_MB(F, N_)                                                                                 \
    if (NV == N_) k = xp == XP_NORM ? qmv_batch_kernel<F, N_, XP_NORM>                               \
                      : xp == XP_SILU_GATE ? qmv_batch_kernel<F, N_, XP_SILU_GATE> : qmv_batch_kernel<F, N_, XP_NONE>;
    if (dtype == DT_Q8_0) {
        QH_MB(8, 2) QH_MB(8, 4) QH_MB(8, 8) QH_MB(8, 16)
    } else {
        QH_MB(4, 2) QH_MB(4, 4) QH_MB(4, 8) QH_MB(4, 16)
    }
#undef QH_MB
    const int nb = (int)(K / 32);
    const size_t rb = q_row_bytes(dtype, 32, K);
    QH_REQUIRE(rb <= 0xFFFFFFFFu, QRAF_HIP_ERR_INVALID, "batch matvec: rows too long");
    if (lds > 65536) QH_CHECK_HIP(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int fit = 0;
    QH_CHECK_HIP(resident_wgs((const void*)k, WG, lds, &fit));
    const int grid = max(1, min((int)((N + 3) / 4), max(1, fit) * cu_count()));
    hipLaunchKernelGGL(k, dim3(grid), dim3(WG), lds, s, (const uint8_t*)Wv, (uint32_t)rb, (int)N, (int)K, nb, x, ldx,
                       nv, y, ldy, add, xw, eps);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_matvec_f32(const float* W, const float* x, float* y, uint32_t N, uint32_t K, hipStream_t s,
                      const float* add) {
    QH_REQUIRE(W && x && y && N > 0 && K > 0, QRAF_HIP_ERR_INVALID, "bad f32 matvec arguments");
    hipLaunchKernelGGL(mv_f32_kernel, dim3((N + 3) / 4), dim3(WG), 0, s, W, x, y, (int)N, (int)K, add);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip
