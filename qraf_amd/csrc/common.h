// common.h -- shared definitions for the gfx950 QRAF decode library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/qraf_hip.h"
#include "status.h"

namespace qraf_hip {

// QRAF dtype codes (reference include/core/types.h:27-39).
constexpr uint32_t DT_F32 = 0, DT_F16 = 1, DT_Q8_0 = 10, DT_Q4_0 = 20, DT_I8 = 102;  // types.h:27-38


#define QH_CHECK_HIP(expr)                                                              \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return ::qraf_hip::set_error(QRAF_HIP_ERR_HIP, "%s failed: %s (%s:%d)", #expr, \
                                         hipGetErrorString(e_), __FILE__, __LINE__);     \
    } while (0)


// Bytes of one quantized block (reference quantize.cpp:107, :146).
__host__ __device__ inline size_t q_block_bytes(uint32_t dtype, int bs) {
    if (dtype == DT_Q8_0) return 4 + (size_t)bs;
    if (dtype == DT_Q4_0) return 2 + (size_t)(bs / 2);
    return 0;
}
// Bytes of one weight row of in_dim elements (reference backend.cpp:137-140, :166-169).
__host__ __device__ inline size_t q_row_bytes(uint32_t dtype, int bs, uint32_t in_dim) {
    return ((size_t)(in_dim + bs - 1) / bs) * q_block_bytes(dtype, bs);
}

// Kernel launchers (device pointers; stream-ordered; no synchronisation).
// add (optional, may alias y): y[i] = dot(row_i, x) + add[i]
// How a batch-1 matvec forms its x while staging it, instead of a separate
// kernel writing x first (x then names the source):
//   XP_NONE       x as is
//   XP_NORM       rms_norm(x) * w  (ops.cpp:107-118), x of K elements
//   XP_SILU_GATE  silu(x[2i]) * x[2i+1]  (x: interleaved gate/up rows, 2K elements)
// Kernels that cannot form x themselves get it from a prep kernel writing
// `xbuf` (K floats) first.
enum { XP_NONE = 0, XP_NORM = 1, XP_SILU_GATE = 2 };
struct MvPrep {
    int op = XP_NONE;
    const float* w = nullptr;  // XP_NORM weights
    float eps = 0.f;           // XP_NORM epsilon
    float* xbuf = nullptr;     // scratch for the prep-kernel fallback
};
// Epilogue of a one-token QKV projection (y = [q | k | v]): the bias, RoPE
// of q and k, and the store of k and v at the token's position in its KV
// page (rope_append_kernel's arithmetic), so no y is written.  f32 and fp16
// pages.
struct MvRope {
    const float* bias = nullptr;          // [qd + 2 kvd] F32 bias, or null
    const int32_t* pos = nullptr;         // device: the token's position
    const float* rope = nullptr;          // [positions][hd]: (cos, sin) of pair i/2 at [i], [i + 1]
    float* q_out = nullptr;               // [qd]
    void* kc = nullptr;                   // the layer's K pages
    void* vc = nullptr;                   // the layer's V pages
    const int32_t* page_table = nullptr;  // the sequence's page ids
    int H = 0, Hkv = 0, hd = 0, page_size = 0;
    uint32_t kv_dtype = 0;                // DT_F32 or DT_F16
};
// rope (optional): fuse that epilogue when the chosen kernel is the one-shot
// form; *fused says whether it was (else y holds the projection as usual)
int launch_matvec_q(const void* W, uint32_t dtype, int bs, uint32_t N, uint32_t K, const float* x,
                    float* y, hipStream_t s, const float* add = nullptr, const MvPrep* prep = nullptr,
                    const MvRope* rope = nullptr, bool* fused = nullptr);
int launch_matvec_f32(const float* W, const float* x, float* y, uint32_t N, uint32_t K, hipStream_t s,
                      const float* add = nullptr);
// nv (1..MV_BATCH_MAX) vectors at once: x rows of ldx floats (2K for the
// SiLU-gate's interleaved source), y rows of ldy floats, add likewise; the
// vectors are staged in LDS together (at most MV_BATCH_LDS bytes), so K is
// bounded; matvec_batch_ok says whether a shape is covered.  Q8_0 / Q4_0,
// block size 32.
constexpr int MV_BATCH_MAX = 16;
constexpr int MV_BATCH_SMALL = 8;  // the engine's steps of 2..8 rows (larger steps are padded for graph reuse)
// rows x N x K up to which the engine prefers it to the GEMM (split, GEMM and
// reduction launches): MI355X, Qwen2.5-3B / SmolLM2-135M projection shapes at
// 2-8 rows, e.g. 2048 x 2048 Q4_0 at 2 / 8 rows 6.7 / 10.9 us against 12.3 /
// 12.5; 22016 x 2048 at 2 / 3 rows 21.4 / 27.0 against 22.8 / 22.8
constexpr long long MV_BATCH_WORK = 96LL << 20;
constexpr int MV_BATCH_LDS = 144 * 1024;
bool matvec_batch_ok(uint32_t dtype, uint32_t K, int nv);
int launch_matvec_q_batch(const void* W, uint32_t dtype, uint32_t N, uint32_t K, const float* x, int ldx, int nv,
                          float* y, int ldy, hipStream_t s, const float* add = nullptr, const MvPrep* prep = nullptr);
int set_matvec_tuning(int kernel, int rows, int wgs_per_cu);
// Bumped by every tuning call: captured launch sequences (the engine's step
// graphs) record it and are rebuilt when it changes.
uint32_t tuning_generation();
void bump_tuning_generation();
int launch_rms_norm(float* x, const float* w, int n, float eps, hipStream_t s);
int launch_softmax(float* x, int n, hipStream_t s);
int launch_dot(const float* a, const float* b, int n, float* out, hipStream_t s);
// op: 0 silu, 1 add, 2 mul, 3 scale
int launch_ew(int op, float* x, const float* y, float sc, int n, hipStream_t s);
// streaming read of `bytes` (the plain-read ceiling); out: read_probe_out_floats() floats
int launch_read_probe(const void* p, size_t bytes, float* out, hipStream_t s);
int launch_empty(int wgs, hipStream_t s);
size_t read_probe_out_floats();

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}
// The two activation planes of the GEMM: hi = round-to-nearest-even bf16 of
// x (fp32's range), lo = round-to-nearest-even fp16 of the exact rest x - hi
// (|x - hi| <= 2^-8 |x|), clamped to the finite fp16 range.  x = hi + lo + r
// with |r| <= 2^-20 |x| + 2^-25 while |x| < 2^24 (lo normal: 2^-20 |x|; lo
// subnormal, |x| below about 2^-5: at most half the fp16 subnormal step);
// beyond 2^24 the clamp leaves |r| <= 2^-8 |x|.
__device__ __forceinline__ void split_bf16(float v, uint16_t* hi, uint16_t* lo) {
    const uint32_t h = f32_to_bf16_rne(v);
    *hi = (uint16_t)h;
    const float rest = v - __builtin_bit_cast(float, h << 16);  // exact
    *lo = __builtin_bit_cast(uint16_t, (_Float16)__builtin_fminf(__builtin_fmaxf(rest, -65504.0f), 65504.0f));
}

// SiLU-gate of one gate/up pair (ops.cpp:218-222 then :275-279): silu(g) * u
__device__ __forceinline__ float silu_gate(float g, float u) { return __fmul_rn(g / (1.0f + expf(-g)), u); }

// element e of S slices (GEMM split-K partials) of `slice` floats, summed in
// slice order.  Up to 8 slices: every load issued before the first add (one
// round trip); beyond, 8 slices per round trip.
template <int S>
__device__ __forceinline__ float sum_slices_n(const float* __restrict__ p, size_t slice, size_t e) {
    float t[S];
#pragma unroll
    for (int u = 0; u < S; u++) t[u] = p[(size_t)u * slice + e];
    float acc = t[0];
#pragma unroll
    for (int u = 1; u < S; u++) acc += t[u];
    return acc;
}
__device__ __forceinline__ float sum_slices(const float* __restrict__ p, int S, size_t slice, size_t e) {
    switch (S) {
        case 1: return p[e];
        case 2: return sum_slices_n<2>(p, slice, e);
        case 3: return sum_slices_n<3>(p, slice, e);
        case 4: return sum_slices_n<4>(p, slice, e);
        case 5: return sum_slices_n<5>(p, slice, e);
        case 6: return sum_slices_n<6>(p, slice, e);
        case 7: return sum_slices_n<7>(p, slice, e);
        case 8: return sum_slices_n<8>(p, slice, e);
        default: break;
    }
    float acc = p[e];
    int k = 1;
    for (; k + 8 <= S; k += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; u++) t[u] = p[(size_t)(k + u) * slice + e];
#pragma unroll
        for (int u = 0; u < 8; u++) acc += t[u];
    }
    for (; k < S; k++) acc += p[(size_t)k * slice + e];
    return acc;
}

// sort storage a sampling call needs (0: none): rows whose candidates may
// exceed the in-LDS limit keep rows * V (p, index) pairs twice
size_t sample_sort_bytes(int rows, int V, const qraf_sampling_params& sp);
int launch_sample(float* logits, int rows, int V, const qraf_sampling_params& sp, const uint32_t* recent,
                  const int32_t* counts, int stride, const float* uniforms, uint32_t* out, void* sort_ws,
                  size_t sort_bytes, hipStream_t s);

// x may be S slices of `slice` floats each (GEMM partials), summed in slice order
int launch_split_bf16(const float* x, uint16_t* hi, uint16_t* lo, int M, int K, int op, float* xout, hipStream_t s,
                      int S = 1, size_t slice = 0);
// split-K partial tiles go to ws when it is large enough (qgemm_workspace_bytes), else one split
int launch_qgemm(const void* W, uint32_t dtype, int bs, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                 float* Y, const float* add, void* ws, size_t ws_bytes, hipStream_t s, bool tiled = false,
                 int* slices = nullptr);
// sets the dynamic-LDS attribute of every wave-split GEMM instantiation (qraf_hip_init)
int qgemm_kw_init();
int launch_qgemm_silu(const void* Wt, uint32_t dtype, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                      uint16_t* act_hi, uint16_t* act_lo, hipStream_t s);
// greedy head: argmax of each row of X W^T without writing it (tile-major W);
// *done = false (nothing launched) where the tiled plan is not the pipelined form
size_t qgemm_argmax_keys_bytes(int N, int M);
bool qgemm_argmax_fits(uint32_t dtype, int N, int K, int M, size_t keys_bytes);
int launch_qgemm_argmax(const void* Wt, uint32_t dtype, int N, int K, const uint16_t* xh, const uint16_t* xl, int M,
                        uint64_t* keys, size_t keys_bytes, uint32_t* out, hipStream_t s, bool* done);
size_t qgemm_workspace_bytes(uint32_t dtype, int N, int K, int M, bool tiled = false);
// bytes of the [S][M][N] partial slices launch_qgemm(..., slices) writes
size_t qgemm_partials_bytes(uint32_t dtype, int N, int K, int M, bool tiled = false);
// tile-major copy of a Q8_0/Q4_0 matrix for launch_qgemm(..., tiled = true)
size_t tiled_weight_bytes(uint32_t dtype, int N, int K);
int launch_repack_tiles(const void* W, uint32_t dtype, int N, int K, void* dst, hipStream_t s);
// Y = sum of S slices [S][MN] (+ add), in slice order
int launch_reduce_slices(const float* part, int S, size_t MN, float* Y, const float* add, hipStream_t s);
size_t attn_workspace_bytes(int n, int H, int Hkv, int hd, int max_ctx);
// resolves the device address of the no-allocation attention workspace on
// `device` (current); called once per device by qraf_hip_init
int attn_scratch_init(int device);
int launch_attention(const float* q, const void* kc, const void* vc, uint32_t kv_dtype, const int32_t* page_table,
                     int max_pages, const int32_t* ctx, int n, int H, int Hkv, int hd, int page_size, float scale,
                     int max_ctx, float* out, void* ws, size_t ws_bytes, hipStream_t st, uint16_t* out_hi = nullptr,
                     uint16_t* out_lo = nullptr);
int launch_rope_append(const float* qkv, const float* bias, int n, int H, int Hkv, int hd, const int32_t* pos,
                       const float* rope, float* q_out, void* kc, void* vc, uint32_t kv_dtype,
                       const int32_t* page_table, int max_pages, int page_size, hipStream_t st, int S = 1,
                       size_t slice = 0);
int launch_gen_weights(void* dst, uint32_t dtype, uint64_t count, uint64_t seed, uint64_t stream_id, float stddev,
                       hipStream_t s);
int launch_quantize(const float* src, uint64_t count, uint32_t dtype, void* dst, hipStream_t s);

typedef int v4i __attribute__((ext_vector_type(4)));
// ---------------------------------------------------------------- LDS staging
// Direct-to-LDS 16-byte load: lane i writes LDS [lds + 16 i, +16) from its
// own voffset.  Issued as inline asm so that the compiler tracks none of these
// loads (it would otherwise wait for all of them before every LDS read it
// cannot prove disjoint): the kernel counts them itself (vmcnt) and every
// other vector memory access of the kernel happens after the final drain.
__device__ __forceinline__ v4i make_rsrc_words(const void* p, uint32_t bytes) {
    const uint64_t a = (uint64_t)p;
    return v4i{(int)(uint32_t)a, (int)(uint32_t)(a >> 32), (int)bytes, 0x00020000};
}
__device__ __forceinline__ void dma16(v4i rsrc, uint32_t voff, const void* lds) {
    const uint32_t m0v = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
    __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                     :
                     : "v"(voff), "s"(rsrc), "s"(m0v)
                     : "memory", "m0");
}

__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_barrier" ::: "memory"); }

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
}


// Library default stream of the current device (created by qraf_hip_init).
hipStream_t default_stream();
inline hipStream_t as_stream(void* s) { return s ? (hipStream_t)s : default_stream(); }

}  // namespace qraf_hip
