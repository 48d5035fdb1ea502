// engine.hip -- device-resident decode engine for LLaMA/Qwen2-family QRAF models.
//
// The MI355X counterpart of Transformer::init / forward / reset
// (reference transformer.cpp:310-439, :573-643, transformer.h:55-90) with
// the one API extension a continuous batch needs: a step that advances
// several sequences at once, each with its own token and position.
//
// Weights are uploaded (or generated) once into HBM, in the reference's
// block layout, with two layout-only changes that let one launch serve
// several reference matvecs: the q, k and v projection rows are stored
// back to back (one [q_dim + 2 kv_dim] x hidden matrix), and the gate and up
// projection rows are interleaved (row 2i = gate_i, row 2i+1 = up_i), so
// SiLU(gate) * up (attention.cpp:172-180) pairs neighbouring outputs.
//
// KV cache: a pool of pages per layer, [num_pages][Hkv][page_size][head_dim]
// (f32 or f16), or int8 blocks with a scale per position (the layout of the
// attention kernels); sequences own page lists handed out by a host-side free
// list.
// Each step: embedding row, then per layer RMSNorm -> fused QKV projection
// -> bias + RoPE + page append -> ragged paged attention -> O projection with
// the residual add in its epilogue -> RMSNorm -> gate/up projection ->
// SiLU-gate -> down projection with the residual add; final RMSNorm, LM head
// for the rows that want logits, argmax on the device.  Batch 1 runs on the
// streaming matvec, larger batches on the matrix-core GEMM.
#include <limits.h>
#include <math.h>

#include <cmath>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <string>
#include <vector>

#include "common.h"
#include "kv_pages.h"

namespace qraf_hip {

// ---------------------------------------------------------------- kernels

// embedding row of row s's token (load_tensor_f32 + Tensor::row,
// transformer.cpp:34-39, :577): dequantised values (f32)q * scale.  The token
// is tok[s], or, where src[s] >= 0, the previous step's greedy token of its
// logit row src[s] (prev, still in HBM: the token never visits the host).
// Rows of a sequence with a repetition penalty on the device (pslot[s] >= 0)
// also count their token in that sequence's occurrence counts, the
// reference's recent_for_penalty list (inference.cpp:104-108, :125) as counts.
__global__ void embed_kernel(const uint8_t* __restrict__ emb, uint32_t dtype, int bs, int D,
                             const int32_t* __restrict__ tok, const int32_t* __restrict__ src,
                             const uint32_t* __restrict__ prev, float* __restrict__ h,
                             const int32_t* __restrict__ pslot, uint32_t* __restrict__ pcounts, int V) {
    const int s = blockIdx.x;
    const int32_t from = src[s];
    const size_t row = from >= 0 ? (size_t)prev[from] : (size_t)tok[s];
    if (pcounts && threadIdx.x == 0 && pslot[s] >= 0) atomicAdd(&pcounts[(size_t)pslot[s] * V + row], 1u);
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        const size_t e = row * D + i;
        float v;
        if (dtype == DT_F32) {
            v = ((const float*)emb)[e];
        } else if (dtype == DT_F16) {
            v = (float)((const _Float16*)emb)[e];
        } else {
            const size_t b = e / bs, w = e % bs;
            const uint8_t* p = emb + b * q_block_bytes(dtype, bs);
            if (dtype == DT_Q8_0) {
                const float sc = __builtin_bit_cast(float, (uint32_t)p[0] | ((uint32_t)p[1] << 8) |
                                                               ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
                v = __fmul_rn((float)(int8_t)p[4 + w], sc);
            } else {
                const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(p[0] | (p[1] << 8)));
                const uint8_t q = p[2 + w / 2];
                v = __fmul_rn((float)((int)((w & 1) ? (q >> 4) : (q & 15)) - 8), sc);
            }
        }
        h[(size_t)s * D + i] = v;
    }
}

// rms_norm_inplace (ops.cpp:107-118) of `rows` rows, one workgroup per row
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          int D, float eps, float* __restrict__ out,
                                                          const int32_t* __restrict__ row_map) {
    __shared__ float red[4];
    const int s = blockIdx.x;
    const float* xr = x + (size_t)(row_map ? row_map[s] : s) * D;
    float ss = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) ss = __builtin_fmaf(xr[i], xr[i], ss);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += 256) out[(size_t)s * D + i] = __fmul_rn(__fmul_rn(xr[i], r), w[i]);
}

// Residual add of a projection's split-K partials, then the next RMSNorm into
// the two planes (bf16 hi, fp16 lo) the following GEMM reads (one 1024-thread workgroup per
// row, J elements per thread):
//     h += (part[0] + ... + part[S-1])        (transformer.cpp:593 / :601)
//     xh + xl = rms_norm(h) * w               (ops.cpp:107-118)
// S = 0: no residual (h as is); w = null: residual only.
template <int J>
__global__ __launch_bounds__(1024) void residual_norm_split_kernel(const float* __restrict__ part, int S, size_t slice,
                                                                  float* __restrict__ h, const float* __restrict__ w,
                                                                  int D, float eps, uint16_t* __restrict__ xh,
                                                                  uint16_t* __restrict__ xl) {
    __shared__ float red[16];
    const int m = blockIdx.x, tid = threadIdx.x;
    float* hr = h + (size_t)m * D;
    float v[J];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int i = tid + 1024 * j;
        v[j] = 0.f;
        if (i < D) {
            v[j] = hr[i];
            if (S > 0) {
                v[j] = sum_slices(part, S, slice, (size_t)m * D + i) + v[j];
                hr[i] = v[j];
            }
        }
        ss = __builtin_fmaf(v[j], v[j], ss);
    }
    if (!w) return;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) ss += red[k];
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int i = tid + 1024 * j;
        if (i < D) {
            const size_t e = (size_t)m * D + i;
            split_bf16(__fmul_rn(__fmul_rn(v[j], r), w[i]), &xh[e], &xl[e]);
        }
    }
}

// The same with elements 2t, 2t+1 per thread (8-byte loads of each slice and
// of h, half the load instructions, every slice's load issued before the
// first add); D even, D <= 2048, 8-byte aligned rows, S <= 8 or 16.
template <int S>
__global__ __launch_bounds__(1024) void residual_norm_split_v2_kernel(const float* __restrict__ part, size_t slice,
                                                                     float* __restrict__ h, const float* __restrict__ w,
                                                                     int D, float eps, uint16_t* __restrict__ xh,
                                                                     uint16_t* __restrict__ xl) {
    __shared__ float red[16];
    const int m = blockIdx.x, tid = threadIdx.x, i = 2 * tid;
    float2* hr = (float2*)(h + (size_t)m * D);
    // the norm weights of this thread's pair, requested with the sums' operands
    // (at a pair index clamped into the row; without weights the load reads h)
    const float2 wv = *(const float2*)(w ? w + min(i, D - 2) : h);
    float2 v = make_float2(0.f, 0.f);
    if (i < D) {
        v = hr[tid];
        if (S > 0) {
            float2 t[S > 0 ? S : 1];
#pragma unroll
            for (int u = 0; u < S; u++) t[u] = *(const float2*)(part + (size_t)u * slice + (size_t)m * D + i);
            float a = t[0].x, b = t[0].y;
#pragma unroll
            for (int u = 1; u < S; u++) {
                a += t[u].x;
                b += t[u].y;
            }
            v = make_float2(a + v.x, b + v.y);
            hr[tid] = v;
        }
    }
    float ss = __builtin_fmaf(v.y, v.y, v.x * v.x);
    if (!w) return;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) ss += red[k];
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    if (i < D) {
        const size_t e = (size_t)m * D + i;
        split_bf16(__fmul_rn(__fmul_rn(v.x, r), wv.x), &xh[e], &xl[e]);
        split_bf16(__fmul_rn(__fmul_rn(v.y, r), wv.y), &xh[e + 1], &xl[e + 1]);
    }
}

static int launch_residual_norm_split(const float* part, int S, size_t slice, float* h, const float* w, int D, float eps,
                                      uint16_t* xh, uint16_t* xl, int rows, hipStream_t s) {
    QH_REQUIRE(D <= 8192, QRAF_HIP_ERR_INVALID, "residual/norm: hidden size %d > 8192", D);
    if (D % 2 == 0 && D <= 2048 && (S <= 8 || S == 16) && (S == 0 || slice % 2 == 0) && (((uintptr_t)h) & 7) == 0 &&
        (((uintptr_t)part) & 7) == 0 && (((uintptr_t)w) & 7) == 0) {
#define QH_RN2(Sv) hipLaunchKernelGGL(residual_norm_split_v2_kernel<Sv>, dim3(rows), dim3(1024), 0, s, part, slice, h, w, \
                                      D, eps, xh, xl)
        switch (S) {
            case 0: QH_RN2(0); break;
            case 1: QH_RN2(1); break;
            case 2: QH_RN2(2); break;
            case 3: QH_RN2(3); break;
            case 4: QH_RN2(4); break;
            case 5: QH_RN2(5); break;
            case 6: QH_RN2(6); break;
            case 7: QH_RN2(7); break;
            case 8: QH_RN2(8); break;
            default: QH_RN2(16); break;
        }
#undef QH_RN2
        QH_CHECK_HIP(hipGetLastError());
        return QRAF_HIP_OK;
    }
#define QH_RNS(Jv) hipLaunchKernelGGL(residual_norm_split_kernel<Jv>, dim3(rows), dim3(1024), 0, s, part, S, slice, h, w, \
                                      D, eps, xh, xl)
    if (D <= 1024) QH_RNS(1);
    else if (D <= 2048) QH_RNS(2);
    else if (D <= 4096) QH_RNS(4);
    else QH_RNS(8);
#undef QH_RNS
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

// silu_inplace then mul_inplace (attention.cpp:177-178) on interleaved gate/up rows
__global__ void silu_gate_kernel(const float* __restrict__ gu, int F, int n, float* __restrict__ act) {
    const size_t total = (size_t)n * F;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t s = i / F, j = i % F;
        const float g = gu[s * 2 * F + 2 * j], u = gu[s * 2 * F + 2 * j + 1];
        act[i] = silu_gate(g, u);
    }
}

// Two-pass Sampler::argmax for long rows: 32 chunks per row, each scanned by
// one workgroup with 8 loads in flight per thread (ascending index per thread,
// so strict '>' keeps the lowest index), then a per-row pass over the chunk
// winners in chunk order.  Ties across threads/chunks go to the lower index.
constexpr int ARGMAX_CHUNKS = 32;

__device__ __forceinline__ void argmax_take(float& best, int& bi, float v, int i) {
    if (v > best || (v == best && i < bi)) {
        best = v;
        bi = i;
    }
}

__device__ __forceinline__ void argmax_block(float& best, int& bi) {
    __shared__ float sv[4];
    __shared__ int si[4];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) argmax_take(best, bi, __shfl_xor(best, o), __shfl_xor(bi, o));
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < 4; w++) argmax_take(best, bi, sv[w], si[w]);
}

__global__ __launch_bounds__(256) void argmax_chunk_kernel(const float* __restrict__ logits, int V,
                                                          float* __restrict__ pv, int* __restrict__ pi) {
    const int row = blockIdx.y, c = blockIdx.x;
    const int len = (V + ARGMAX_CHUNKS - 1) / ARGMAX_CHUNKS;
    const int c0 = c * len, c1 = min(V, c0 + len);
    const float* l = logits + (size_t)row * V;
    float best = -INFINITY;
    int bi = INT_MAX;
    for (int base = c0 + (int)threadIdx.x; base < c1; base += 256 * 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = base + 256 * u;
            v[u] = i < c1 ? l[i] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = base + 256 * u;
            if (i < c1 && (bi == INT_MAX || v[u] > best)) {
                best = v[u];
                bi = i;
            }
        }
    }
    argmax_block(best, bi);
    if (threadIdx.x == 0) {
        pv[row * ARGMAX_CHUNKS + c] = best;
        pi[row * ARGMAX_CHUNKS + c] = bi;
    }
}

__global__ void argmax_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi, int V,
                                    uint32_t* __restrict__ out) {
    const int row = blockIdx.x;
    if (threadIdx.x != 0) return;
    float best = -INFINITY;
    int bi = INT_MAX;
    for (int c = 0; c < ARGMAX_CHUNKS; c++) {
        const int i = pi[row * ARGMAX_CHUNKS + c];
        if (i == INT_MAX) continue;  // empty chunk
        if (bi == INT_MAX) {
            best = pv[row * ARGMAX_CHUNKS + c];
            bi = i;
        } else {
            argmax_take(best, bi, pv[row * ARGMAX_CHUNKS + c], i);
        }
    }
    out[row] = (uint32_t)(bi == INT_MAX || bi >= V ? 0 : bi);
}

// One pass of Sampler::argmax per row (sampler.cpp:25-35), a 1024-thread
// workgroup per row: each thread scans its 16-byte groups i, i + 1024, ... in
// ascending index order (strict '>': its lowest index of its maximum), 16
// groups in flight per round, then the workgroup keeps the maximum, ties to
// the lower index.  Needs V % 4 == 0 and 16-byte aligned rows.  A row whose
// sequence has a repetition penalty on the device (pslot of its step row
// lrows[row] >= 0) takes each logit through
// Sampler::apply_repetition_penalty (sampler.cpp:37-49) first: k times
// v > 0 ? v / penalty : v * penalty for a token fed k times (the reference
// applies it once per list entry; a value keeps its sign, so the entries of
// one token are these k steps, and distinct tokens are independent).  The
// logits in HBM stay as they are.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* __restrict__ logits, int V,
                                                          uint32_t* __restrict__ out,
                                                          const int32_t* __restrict__ lrows,
                                                          const int32_t* __restrict__ pslot,
                                                          const float* __restrict__ ppen,
                                                          const uint32_t* __restrict__ pcounts) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float4* l4 = (const float4*)(logits + (size_t)row * V);
    const int n4 = V >> 2;
    const int srow = pcounts ? lrows[row] : 0;
    const int slot = pcounts ? pslot[srow] : -1;
    const float pen = slot >= 0 ? ppen[srow] : 1.f;
    const uint4* c4 = (const uint4*)(pcounts + (size_t)(slot >= 0 ? slot : 0) * V);
    float best = -INFINITY;
    int bi = INT_MAX;
    for (int base = tid; base < n4; base += 1024 * 16) {
        float4 v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = l4[min(base + 1024 * u, n4 - 1)];
        if (slot >= 0) {  // uniform per workgroup
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const uint4 k = c4[min(base + 1024 * u, n4 - 1)];
                const uint32_t kk[4] = {k.x, k.y, k.z, k.w};
                float* e = (float*)&v[u];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    for (uint32_t r = 0; r < kk[j]; r++) e[j] = e[j] > 0.f ? e[j] / pen : e[j] * pen;
            }
        }
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int g = base + 1024 * u;
            if (g < n4) {
                const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (bi == INT_MAX || e[k] > best) {
                        best = e[k];
                        bi = 4 * g + k;
                    }
            }
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) argmax_take(best, bi, __shfl_xor(best, o), __shfl_xor(bi, o));
    if ((tid & 63) == 0) {
        sv[tid >> 6] = best;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++) argmax_take(best, bi, sv[w], si[w]);
        out[row] = (uint32_t)(bi == INT_MAX || bi >= V ? 0 : bi);
    }
}

__global__ void fill_kernel(float* p, float v, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// compact rows: dst[j] = src[rows[j]] (D floats each)
__global__ void gather_rows_kernel(const float* __restrict__ src, const int32_t* __restrict__ rows, int D,
                                   float* __restrict__ dst) {
    const int j = blockIdx.x;
    for (int i = threadIdx.x; i < D; i += blockDim.x) dst[(size_t)j * D + i] = src[(size_t)rows[j] * D + i];
}

}  // namespace qraf_hip

// ---------------------------------------------------------------- engine

using namespace qraf_hip;

struct qraf_engine {
    qraf_model_config c{};
    qraf_engine_options o{};
    int hd = 0, qd = 0, kvd = 0, qkvd = 0, capacity = 0, max_pages = 0;
    hipStream_t stream = nullptr;
    bool finalized = false;

    struct Layer {
        uint8_t* wqkv = nullptr;
        uint8_t* wo = nullptr;
        uint8_t* wgu = nullptr;
        uint8_t* wd = nullptr;
        // tile-major copies of the quantized projections for the batched GEMM
        uint8_t *wqkv_t = nullptr, *wo_t = nullptr, *wgu_t = nullptr, *wd_t = nullptr;
        float* bqkv = nullptr;
        float* an = nullptr;
        float* fn = nullptr;
        uint32_t dt_attn = 0xFFFFFFFFu, dt_mlp = 0xFFFFFFFFu;
        uint32_t have = 0;  // bit per tensor
        bool has_bias = false;
    };
    std::vector<Layer> layers;
    uint8_t* embed = nullptr;
    uint32_t dt_embed = 0xFFFFFFFFu;
    uint8_t* head = nullptr;
    uint32_t dt_head = 0xFFFFFFFFu;
    uint8_t* head_t = nullptr;  // tile-major copy of the LM head (or the tied embedding)
    float* onorm = nullptr;
    std::vector<void*> allocs;

    // KV pool and pages
    uint8_t* kpool = nullptr;
    uint8_t* vpool = nullptr;
    size_t layer_kv_bytes = 0;
    KvPages pages;                    // sequences, their pages, the free list (host only)
    int32_t scratch_page = 0;         // one page past the pool's num_pages: written and read by pad rows only
    int row_pad = 16;                 // steps of more than 8 rows are padded to a multiple of this (graphs on)
    bool fuse_rope = true;            // one-row steps: RoPE/append fused into the QKV matvec
    bool fuse_swiglu = true;          // steps over 256 rows: SiLU-gate in the gate/up GEMM's epilogue
    bool batch_mv = true;             // steps of 2-8 rows: projections on the multi-vector matvec
    int32_t default_seq = -1;
    int last_logit_rows = 0;          // logit rows the last step left in `logits`
    bool keep_logits = true;          // false: greedy-only steps take the head's argmax without writing logits
    int qbs = 0;                      // quant block size of every quantized tensor (0: none bound yet, then 32)
    bool last_logits_kept = true;     // the last step's logits are in `logits` (not a greedy-only step)
    qraf_engine_stats stats{};        // host-side time of qraf_engine_step
    // Repetition penalty on the device (qraf_engine_set_repetition_penalty):
    // a slot of V occurrence counts per penalised sequence, bumped by the
    // embedding for every token the sequence is fed, read by the argmax
    uint32_t* pen_counts = nullptr;   // [2 max_batch slots][V], allocated on first use (a pipelined scheduler
                                      // admits a request while one whose last token is in flight still holds its slot)
    std::vector<int32_t> pen_slot;    // sequence id -> slot, -1 for none
    std::vector<float> pen_value;     // sequence id -> penalty
    std::vector<int32_t> pen_free;    // free slots
    int pen_live = 0;                 // sequences with a slot
    uint8_t* samp = nullptr;          // sampling staging: recent tokens, counts, uniforms, tokens
    size_t samp_cap = 0;
    void* sort_ws = nullptr;          // sampling sort storage (large top_k, flat whole-vocabulary rows)
    size_t sort_cap = 0;

    // activations (max_batch rows)
    float *h = nullptr, *xn = nullptr, *qkv = nullptr, *q = nullptr, *att = nullptr, *gu = nullptr, *act = nullptr,
          *logits = nullptr, *xhead = nullptr, *rope = nullptr;
    uint16_t *xh = nullptr, *xl = nullptr;
    uint16_t *ah = nullptr, *al = nullptr;  // SwiGLU activation planes [max_batch][F] (fused gate/up epilogue)
    uint32_t* amax = nullptr;
    int32_t* d_in = nullptr;  // tokens | positions | ctx | logit rows | token sources | penalty slots | penalties |
                              // page table rows
    // Pinned staging, one slot per step in flight: a step's inputs are written
    // into slot `slot` while the previous step (the other slot) may still be
    // queued; its tokens come back into h_amax of the same slot.
    int32_t* h_in[2] = {nullptr, nullptr};
    uint32_t* h_amax[2] = {nullptr, nullptr};
    hipEvent_t done_ev[2] = {nullptr, nullptr};  // recorded after a step's last copy
    int slot = 0;
    struct Pending {
        int slot = 0, n_tok = 0;
    };
    Pending pending[2];  // issued, not yet collected steps, oldest first
    int n_pending = 0;
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    void* gemm_ws = nullptr;  // split-K partial tiles of the batched projections
    size_t gemm_ws_bytes = 0;
    float* am_val = nullptr;  // argmax chunk winners [max_batch][32]
    int* am_idx = nullptr;
    uint64_t* am_keys = nullptr;  // the fused head's per-workgroup argmax keys
    size_t am_keys_bytes = 0;
    void* part_ws = nullptr;  // [S][rows][N] partials the fused batched layer sums downstream
    size_t part_ws_bytes = 0;
    bool fused = false;  // every layer has tile-major copies: batched steps run the fused pipeline
    size_t in_words = 0;

    // Captured steps.  A step's launch sequence depends only on its row count,
    // its logit-row count, whether the head runs, the attention grid's context
    // bound and the kernel tuning; everything else (tokens, positions, page
    // tables) reaches the device through the pinned staging copy the graph
    // itself performs.  Replaying it saves the host ~300 kernel launches per
    // decode step.
    struct StepGraph {
        int n = 0, n_logit_rows = 0, ctx = 0;
        int head = 0;  // 0: no head, 1: logits (and argmax), 2: argmax only
        uint32_t gen = 0;
        hipGraphExec_t exec = nullptr;
        uint64_t used = 0;
    };
    std::vector<StepGraph> graphs;
    // shapes seen once: a shape is captured the second time it comes (a
    // chunked-prefill schedule produces many one-off row counts, whose
    // capture would cost more than their eager launch)
    std::vector<StepGraph> seen;
    bool use_graphs = true;
    uint64_t graph_clock = 0;
    void drop_graphs() {
        for (auto& g : graphs) hipGraphExecDestroy(g.exec);
        graphs.clear();
        seen.clear();
    }
};

constexpr size_t MAX_STEP_GRAPHS = 48;

static int ealloc(qraf_engine* e, void** p, size_t bytes) {
    hipError_t r = hipMalloc(p, bytes ? bytes : 16);
    if (r == hipErrorOutOfMemory)
        return set_error(QRAF_HIP_ERR_NOMEM, "engine: out of device memory (%zu bytes)", bytes);
    QH_CHECK_HIP(r);
    e->allocs.push_back(*p);
    return QRAF_HIP_OK;
}

static size_t dt_row_bytes(uint32_t dt, uint32_t cols, int bs) {
    if (dt == DT_F32) return (size_t)cols * 4;
    if (dt == DT_F16) return (size_t)cols * 2;
    return q_row_bytes(dt, bs, cols);
}

enum {
    T_Q = 1, T_K = 2, T_V = 4, T_O = 8, T_G = 16, T_U = 32, T_D = 64, T_AN = 128, T_FN = 256,
    T_ALL = 511
};

// parse "model.layers.<l>.<rest>"
static bool layer_name(const char* name, int* l, const char** rest) {
    const char* pre = "model.layers.";
    if (strncmp(name, pre, strlen(pre)) != 0) return false;
    const char* p = name + strlen(pre);
    char* end = nullptr;
    long v = strtol(p, &end, 10);
    if (end == p || *end != '.') return false;
    *l = (int)v;
    *rest = end + 1;
    return true;
}

// host dequantisation of a norm vector (load_tensor_f32, transformer.cpp:34-39)
static int host_to_f32(uint32_t dt, const void* data, uint64_t bytes, uint32_t n, std::vector<float>& out) {
    out.assign(n, 0.f);
    if (dt == DT_F32) {
        QH_REQUIRE(bytes >= (uint64_t)n * 4, QRAF_HIP_ERR_INVALID, "tensor too small");
        memcpy(out.data(), data, (size_t)n * 4);
        return QRAF_HIP_OK;
    }
    return set_error(QRAF_HIP_ERR_DTYPE, "norm weights must be F32 (got dtype %u)", dt);
}

extern "C" {

int qraf_engine_create(const qraf_model_config* cfg, const qraf_engine_options* opt, qraf_engine** out) {
    clear_error();
    QH_REQUIRE(cfg && out, QRAF_HIP_ERR_INVALID, "engine: null argument");
    *out = nullptr;
    const qraf_model_config& c = *cfg;
    QH_REQUIRE(c.vocab_size && c.hidden_size && c.num_layers && c.num_heads && c.intermediate_size,
               QRAF_HIP_ERR_INVALID, "engine: empty dimension in the model config");
    const uint32_t kvh = c.num_kv_heads ? c.num_kv_heads : c.num_heads;  // types.h:123
    QH_REQUIRE(c.hidden_size % c.num_heads == 0 && c.num_heads % kvh == 0, QRAF_HIP_ERR_INVALID,
               "engine: heads do not divide hidden size / kv heads");
    const int hd = (int)(c.hidden_size / c.num_heads);  // types.h:122
    QH_REQUIRE(hd == 16 || hd == 32 || hd == 64 || hd == 128, QRAF_HIP_ERR_INVALID,
               "engine: head_dim %d (16, 32, 64 or 128 supported)", hd);
    QH_REQUIRE(c.hidden_size % 32 == 0 && c.intermediate_size % 32 == 0, QRAF_HIP_ERR_INVALID,
               "engine: hidden and intermediate sizes must be multiples of 32");
    qraf_engine_options o = opt ? *opt : qraf_engine_options{};
    if (!o.kv_dtype) o.kv_dtype = DT_F32;
    if (o.kv_dtype != DT_F32 && o.kv_dtype != DT_F16 && o.kv_dtype != DT_I8)
        return set_error(QRAF_HIP_ERR_DTYPE, "engine: KV dtype %u", o.kv_dtype);
    if (!o.page_size) o.page_size = 16;
    QH_REQUIRE(o.kv_dtype != DT_I8 || ((hd == 64 || hd == 128) && c.num_heads / kvh <= 16 && o.page_size % 4 == 0),
               QRAF_HIP_ERR_INVALID, "engine: int8 KV pages need head_dim 64/128, group <= 16, page_size %% 4 == 0");
    if (!o.max_batch) o.max_batch = 1;
    QH_REQUIRE(o.max_batch <= 1024, QRAF_HIP_ERR_INVALID, "engine: max_batch %u > 1024", o.max_batch);
    QH_REQUIRE(o.page_size <= 256 && (256 % o.page_size) == 0, QRAF_HIP_ERR_INVALID,
               "engine: page_size must divide 256");

    qraf_engine* e = new qraf_engine();
    e->c = c;
    e->c.num_kv_heads = kvh;
    e->hd = hd;
    e->qd = (int)c.num_heads * hd;
    e->kvd = (int)kvh * hd;
    e->qkvd = e->qd + 2 * e->kvd;
    e->capacity = (int)std::min(c.max_seq_len ? c.max_seq_len : 2048u, 8192u);  // transformer.cpp:425-428
    e->max_pages = (e->capacity + (int)o.page_size - 1) / (int)o.page_size;
    if (!o.num_pages) o.num_pages = o.max_batch * (uint32_t)e->max_pages;
    e->o = o;
    e->layers.resize(c.num_layers);
    auto fail = [&](int rc) {
        for (void* p : e->allocs) hipFree(p);
        for (int k = 0; k < 2; k++) {
            if (e->h_in[k]) hipHostFree(e->h_in[k]);
            if (e->h_amax[k]) hipHostFree(e->h_amax[k]);
            if (e->done_ev[k]) hipEventDestroy(e->done_ev[k]);
        }
        if (e->stream) hipStreamDestroy(e->stream);
        delete e;
        return rc;
    };
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess)
        return fail(set_error(QRAF_HIP_ERR_HIP, "engine: stream creation failed"));
    const int B = (int)o.max_batch, D = (int)c.hidden_size, F = (int)c.intermediate_size, V = (int)c.vocab_size;
    // a (page, KV head) block: page_size positions x head_dim elements, and
    // for int8 a f32 scale per position after them
    const size_t kv_block = o.kv_dtype == DT_I8 ? (size_t)o.page_size * (hd + 4)
                                                : (size_t)o.page_size * hd * (o.kv_dtype == DT_F16 ? 2 : 4);
    e->layer_kv_bytes = (size_t)(o.num_pages + 1) * kvh * kv_block;  // + the scratch page
    e->scratch_page = (int32_t)o.num_pages;
    int rc = QRAF_HIP_OK;
#define A(ptr, bytes)                                           \
    if ((rc = ealloc(e, (void**)&(ptr), (bytes))) != QRAF_HIP_OK) \
        return fail(rc);
    A(e->kpool, e->layer_kv_bytes * c.num_layers);
    A(e->vpool, e->layer_kv_bytes * c.num_layers);
    A(e->h, (size_t)B * D * 4);
    A(e->xn, (size_t)B * D * 4);
    A(e->xhead, (size_t)B * D * 4);
    A(e->qkv, (size_t)B * e->qkvd * 4);
    A(e->q, (size_t)B * e->qd * 4);
    A(e->att, (size_t)B * e->qd * 4);
    A(e->gu, (size_t)B * 2 * F * 4);
    A(e->act, (size_t)B * F * 4);
    A(e->logits, (size_t)B * V * 4);
    const size_t kmax = std::max({(size_t)D, (size_t)F, (size_t)e->qd});
    A(e->xh, (size_t)B * kmax * 2 + 64);
    A(e->xl, (size_t)B * kmax * 2 + 64);
    A(e->ah, (size_t)B * F * 2 + 64);
    A(e->al, (size_t)B * F * 2 + 64);
    A(e->amax, (size_t)B * 4);
    A(e->am_val, (size_t)B * ARGMAX_CHUNKS * 4);
    A(e->am_idx, (size_t)B * ARGMAX_CHUNKS * 4);
    e->am_keys_bytes = qgemm_argmax_keys_bytes((int)V, (int)B);
    A(e->am_keys, e->am_keys_bytes);
    e->in_words = (size_t)B * (7 + e->max_pages);
    A(e->d_in, e->in_words * 4);
    e->attn_ws_bytes = attn_workspace_bytes(B, (int)c.num_heads, (int)kvh, hd, e->capacity);
    A(e->attn_ws, e->attn_ws_bytes);
    A(e->rope, (size_t)e->capacity * hd * 4);
    {
        const int shapes[5][2] = {{e->qkvd, D}, {D, e->qd}, {2 * F, D}, {D, F}, {V, D}};
        for (uint32_t dt : {DT_Q8_0, DT_Q4_0})
            for (auto& sh : shapes)
                for (int m = 2; m <= B; m++)
                    e->gemm_ws_bytes = std::max({e->gemm_ws_bytes, qgemm_workspace_bytes(dt, sh[0], sh[1], m),
                                                  qgemm_workspace_bytes(dt, sh[0], sh[1], m, true)});
    }
    if (e->gemm_ws_bytes) A(e->gemm_ws, e->gemm_ws_bytes);
    {
        const int shapes[4][2] = {{e->qkvd, D}, {D, e->qd}, {2 * F, D}, {D, F}};
        for (uint32_t dt : {DT_Q8_0, DT_Q4_0})
            for (auto& sh : shapes)
                for (int m = 2; m <= B; m++)
                    e->part_ws_bytes = std::max(e->part_ws_bytes, qgemm_partials_bytes(dt, sh[0], sh[1], m, true));
    }
    if (e->part_ws_bytes) A(e->part_ws, e->part_ws_bytes);
#undef A
    if (hipMemset(e->attn_ws, 0, e->attn_ws_bytes) != hipSuccess)
        return fail(set_error(QRAF_HIP_ERR_HIP, "engine: workspace set-up failed"));
    for (int k = 0; k < 2; k++)
        if (hipHostMalloc((void**)&e->h_in[k], e->in_words * 4, hipHostMallocDefault) != hipSuccess ||
            hipHostMalloc((void**)&e->h_amax[k], (size_t)B * 4, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&e->done_ev[k], hipEventDisableTiming) != hipSuccess)
            return fail(set_error(QRAF_HIP_ERR_HIP, "engine: staging set-up failed"));
    // RoPE table from the host libm (RopeCache::init, ops.cpp:179-193)
    {
        std::vector<float> tab((size_t)e->capacity * hd);
        qraf_hip_rope_table_host(e->capacity, hd, c.rope_theta, tab.data());
        if (hipMemcpy(e->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return fail(set_error(QRAF_HIP_ERR_HIP, "engine: rope table upload failed"));
    }
    {
        const int rc = e->pages.init((int)o.num_pages, (int)o.page_size, e->capacity);
        if (rc != QRAF_HIP_OK) return fail(rc);
    }
    *out = e;
    return QRAF_HIP_OK;
}

int qraf_engine_destroy(qraf_engine* e) {
    if (!e) return QRAF_HIP_OK;
    hipStreamSynchronize(e->stream);
    e->drop_graphs();
    for (void* p : e->allocs) hipFree(p);
    for (int k = 0; k < 2; k++) {
        if (e->h_in[k]) hipHostFree(e->h_in[k]);
        if (e->h_amax[k]) hipHostFree(e->h_amax[k]);
        if (e->done_ev[k]) hipEventDestroy(e->done_ev[k]);
    }
    hipStreamDestroy(e->stream);
    delete e;
    return QRAF_HIP_OK;
}

// Bind one tensor by its reference name (transformer.cpp:96-126, :310-400).
int qraf_engine_set_tensor(qraf_engine* e, const char* name, uint32_t dtype, uint32_t block_size, const uint32_t* shape,
                           uint32_t ndim, const void* data, uint64_t bytes) {
    clear_error();
    QH_REQUIRE(e && name && data && shape && ndim >= 1, QRAF_HIP_ERR_INVALID, "set_tensor: null argument");
    QH_REQUIRE(!e->finalized, QRAF_HIP_ERR_STATE, "set_tensor: engine already finalized");
    QH_REQUIRE(dtype == DT_F32 || dtype == DT_F16 || dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE,
               "set_tensor %s: unsupported dtype %u", name, dtype);
    const qraf_model_config& c = e->c;
    const uint32_t D = c.hidden_size, F = c.intermediate_size;
    // One quant block size per model (the reference's QrafModel keeps one
    // scheme per dtype, quant.h): 32, or 4 / 8 / 16 dividing every matrix
    // width, so that a row holds whole blocks; the model's first quantized
    // tensor binds it.  Block sizes other than 32 run every projection on the
    // matvec (the batched GEMM's tiles are 32 wide).
    const int bs = block_size ? (int)block_size : 32;
    if (dtype == DT_Q8_0 || dtype == DT_Q4_0) {
        QH_REQUIRE(bs == 4 || bs == 8 || bs == 16 || bs == 32, QRAF_HIP_ERR_DTYPE,
                   "set_tensor %s: quant block size %d (4, 8, 16 or 32 supported)", name, bs);
        QH_REQUIRE(D % bs == 0 && F % bs == 0 && e->qd % bs == 0, QRAF_HIP_ERR_DTYPE,
                   "set_tensor %s: quant block size %d does not divide the model's widths", name, bs);
        QH_REQUIRE(!e->qbs || e->qbs == bs, QRAF_HIP_ERR_DTYPE,
                   "set_tensor %s: quant block size %d differs from the model's %d", name, bs, e->qbs);
        e->qbs = bs;
    }
    const uint32_t rows = shape[0], cols = ndim > 1 ? shape[1] : 1;
    auto need = [&](uint32_t r, uint32_t cc) -> int {
        QH_REQUIRE(rows == r && (ndim == 1 ? cc == 1 : cols == cc), QRAF_HIP_ERR_INVALID,
                   "set_tensor %s: shape [%u, %u], expected [%u, %u]", name, rows, cols, r, cc);
        QH_REQUIRE(bytes >= (uint64_t)r * dt_row_bytes(dtype, cc, bs), QRAF_HIP_ERR_INVALID,
                   "set_tensor %s: %llu bytes, expected %zu", name, (unsigned long long)bytes,
                   (size_t)r * dt_row_bytes(dtype, cc, bs));
        return QRAF_HIP_OK;
    };
    auto upload = [&](void* dst, const void* src, size_t n) -> int {
        QH_CHECK_HIP(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
        return QRAF_HIP_OK;
    };
    auto ensure = [&](uint8_t** p, size_t n) -> int {
        if (!*p) QH_TRY(ealloc(e, (void**)p, n));
        return QRAF_HIP_OK;
    };

    if (!strcmp(name, "model.embed_tokens.weight")) {
        QH_TRY(need(c.vocab_size, D));
        const size_t n = (size_t)c.vocab_size * dt_row_bytes(dtype, D, bs);
        QH_REQUIRE(!e->embed || e->dt_embed == dtype, QRAF_HIP_ERR_STATE, "embedding dtype changed");
        QH_TRY(ensure(&e->embed, n));
        e->dt_embed = dtype;
        return upload(e->embed, data, n);
    }
    if (!strcmp(name, "lm_head.weight")) {
        QH_TRY(need(c.vocab_size, D));
        const size_t n = (size_t)c.vocab_size * dt_row_bytes(dtype, D, bs);
        QH_REQUIRE(!e->head || e->dt_head == dtype, QRAF_HIP_ERR_STATE, "lm_head dtype changed");
        QH_TRY(ensure(&e->head, n));
        e->dt_head = dtype;
        return upload(e->head, data, n);
    }
    if (!strcmp(name, "model.norm.weight")) {
        QH_TRY(need(D, 1));
        std::vector<float> f;
        QH_TRY(host_to_f32(dtype, data, bytes, D, f));
        QH_TRY(ensure((uint8_t**)&e->onorm, (size_t)D * 4));
        return upload(e->onorm, f.data(), (size_t)D * 4);
    }
    int l;
    const char* rest;
    if (!layer_name(name, &l, &rest) || l < 0 || l >= (int)c.num_layers)
        return QRAF_HIP_OK;  // tensors the LLaMA path does not read are ignored, as by the reference
    qraf_engine::Layer& L = e->layers[l];
    const uint32_t qd = e->qd, kvd = e->kvd;
    struct {
        const char* n;
        int bit;
        uint32_t r, cc;
        int group;  // 0 attention matrix, 1 mlp matrix, 2 bias, 3 norm
        uint32_t off;  // row offset (matrices) / element offset (biases)
    } tab[] = {
        {"self_attn.q_proj.weight", T_Q, qd, D, 0, 0},         {"self_attn.k_proj.weight", T_K, kvd, D, 0, qd},
        {"self_attn.v_proj.weight", T_V, kvd, D, 0, qd + kvd}, {"self_attn.o_proj.weight", T_O, D, qd, 0, 0},
        {"mlp.gate_proj.weight", T_G, F, D, 1, 0},             {"mlp.up_proj.weight", T_U, F, D, 1, 1},
        {"mlp.down_proj.weight", T_D, D, F, 1, 0},             {"self_attn.q_proj.bias", 0, qd, 1, 2, 0},
        {"self_attn.k_proj.bias", 0, kvd, 1, 2, qd},           {"self_attn.v_proj.bias", 0, kvd, 1, 2, qd + kvd},
        {"input_layernorm.weight", T_AN, D, 1, 3, 0},          {"post_attention_layernorm.weight", T_FN, D, 1, 3, 1},
    };
    for (auto& t : tab) {
        if (strcmp(rest, t.n)) continue;
        if (t.group == 2) {  // biases: F32 only, others silently dropped (transformer.cpp:45-50)
            if (dtype != DT_F32) return QRAF_HIP_OK;
            QH_REQUIRE(rows == t.r && bytes >= (uint64_t)t.r * 4, QRAF_HIP_ERR_INVALID, "set_tensor %s: bad shape", name);
            if (!L.bqkv) {
                QH_TRY(ensure((uint8_t**)&L.bqkv, (size_t)e->qkvd * 4));
                QH_CHECK_HIP(hipMemset(L.bqkv, 0, (size_t)e->qkvd * 4));
            }
            L.has_bias = true;
            return upload(L.bqkv + t.off, data, (size_t)t.r * 4);
        }
        if (t.group == 3) {
            QH_TRY(need(t.r, 1));
            std::vector<float> f;
            QH_TRY(host_to_f32(dtype, data, bytes, D, f));
            float** dst = t.off ? &L.fn : &L.an;
            QH_TRY(ensure((uint8_t**)dst, (size_t)D * 4));
            L.have |= t.bit;
            return upload(*dst, f.data(), (size_t)D * 4);
        }
        QH_TRY(need(t.r, t.cc));
        QH_REQUIRE(dtype != DT_F16, QRAF_HIP_ERR_DTYPE, "set_tensor %s: F16 projection weights are not supported", name);
        // one dtype per group (AttentionWeights / MLPWeights carry a single dtype)
        uint32_t& gdt = t.group == 0 ? L.dt_attn : L.dt_mlp;
        QH_REQUIRE(gdt == 0xFFFFFFFFu || gdt == dtype, QRAF_HIP_ERR_DTYPE,
                   "set_tensor %s: dtype %u differs from the other matrices of its group (%u)", name, dtype, gdt);
        const size_t rb = dt_row_bytes(dtype, t.cc, bs);
        const size_t n = (size_t)t.r * rb;
        if (t.bit == T_Q || t.bit == T_K || t.bit == T_V) {
            if (L.wqkv && gdt != dtype) return set_error(QRAF_HIP_ERR_STATE, "dtype changed");
            QH_TRY(ensure(&L.wqkv, (size_t)e->qkvd * rb));
            gdt = dtype;
            L.have |= t.bit;
            return upload(L.wqkv + (size_t)t.off * rb, data, n);
        }
        if (t.bit == T_O) {
            QH_TRY(ensure(&L.wo, n));
            gdt = dtype;
            L.have |= t.bit;
            return upload(L.wo, data, n);
        }
        if (t.bit == T_D) {
            QH_TRY(ensure(&L.wd, n));
            gdt = dtype;
            L.have |= t.bit;
            return upload(L.wd, data, n);
        }
        // gate / up: interleave rows (row 2i = gate_i, 2i+1 = up_i)
        QH_TRY(ensure(&L.wgu, 2 * n));
        gdt = dtype;
        L.have |= t.bit;
        QH_CHECK_HIP(hipMemcpy2D(L.wgu + (size_t)t.off * rb, 2 * rb, data, rb, rb, t.r, hipMemcpyHostToDevice));
        return QRAF_HIP_OK;
    }
    return QRAF_HIP_OK;  // unknown per-layer tensor: not read by the LLaMA path
}

// Synthetic weights generated on the device with the repository's generator
// (same names, seed and per-tensor streams as the test oracle's model).
int qraf_engine_generate_weights(qraf_engine* e, uint32_t wdtype, uint32_t embed_dtype, uint32_t head_dtype,
                                 int32_t tied, int32_t qkv_bias, uint64_t seed) {
    clear_error();
    QH_REQUIRE(e && !e->finalized, QRAF_HIP_ERR_STATE, "generate_weights: engine finalized or null");
    auto ok_dt = [](uint32_t d) { return d == DT_F32 || d == DT_Q8_0 || d == DT_Q4_0; };
    QH_REQUIRE(ok_dt(wdtype) && ok_dt(embed_dtype) && (tied || ok_dt(head_dtype)), QRAF_HIP_ERR_DTYPE,
               "generate_weights: unsupported dtype");
    const qraf_model_config& c = e->c;
    const uint32_t D = c.hidden_size, F = c.intermediate_size;
    hipStream_t s = e->stream;
    auto gen = [&](const std::string& nm, uint8_t* dst, uint32_t dt, size_t count) -> int {
        return launch_gen_weights(dst, dt, count, seed, qraf_hip_name_hash(nm.c_str()), 0.02f, s);
    };
    auto fill1 = [&](float* p, size_t n) -> int {
        hipLaunchKernelGGL(fill_kernel, dim3(64), dim3(256), 0, s, p, 1.0f, n);
        QH_CHECK_HIP(hipGetLastError());
        return QRAF_HIP_OK;
    };
    QH_REQUIRE(!e->qbs || e->qbs == 32, QRAF_HIP_ERR_DTYPE, "generate_weights: tensors of block size %d bound", e->qbs);
    e->qbs = 32;  // the device generator quantizes in blocks of 32
    e->dt_embed = embed_dtype;
    QH_TRY(ealloc(e, (void**)&e->embed, (size_t)c.vocab_size * dt_row_bytes(embed_dtype, D, 32)));
    QH_TRY(gen("model.embed_tokens.weight", e->embed, embed_dtype, (size_t)c.vocab_size * D));
    const size_t rbD = dt_row_bytes(wdtype, D, 32), rbF = dt_row_bytes(wdtype, F, 32),
                 rbQ = dt_row_bytes(wdtype, e->qd, 32);
    uint8_t* tmp = nullptr;
    QH_TRY(ealloc(e, (void**)&tmp, std::max((size_t)F * rbD, (size_t)e->qd * 4)));
    for (uint32_t l = 0; l < c.num_layers; l++) {
        qraf_engine::Layer& L = e->layers[l];
        const std::string pre = "model.layers." + std::to_string(l) + ".";
        L.dt_attn = L.dt_mlp = wdtype;
        QH_TRY(ealloc(e, (void**)&L.wqkv, (size_t)e->qkvd * rbD));
        QH_TRY(gen(pre + "self_attn.q_proj.weight", L.wqkv, wdtype, (size_t)e->qd * D));
        QH_TRY(gen(pre + "self_attn.k_proj.weight", L.wqkv + (size_t)e->qd * rbD, wdtype, (size_t)e->kvd * D));
        QH_TRY(gen(pre + "self_attn.v_proj.weight", L.wqkv + (size_t)(e->qd + e->kvd) * rbD, wdtype,
                   (size_t)e->kvd * D));
        QH_TRY(ealloc(e, (void**)&L.wo, (size_t)D * rbQ));
        QH_TRY(gen(pre + "self_attn.o_proj.weight", L.wo, wdtype, (size_t)D * e->qd));
        if (qkv_bias) {
            QH_TRY(ealloc(e, (void**)&L.bqkv, (size_t)e->qkvd * 4));
            QH_TRY(gen(pre + "self_attn.q_proj.bias", (uint8_t*)L.bqkv, DT_F32, e->qd));
            QH_TRY(gen(pre + "self_attn.k_proj.bias", (uint8_t*)(L.bqkv + e->qd), DT_F32, e->kvd));
            QH_TRY(gen(pre + "self_attn.v_proj.bias", (uint8_t*)(L.bqkv + e->qd + e->kvd), DT_F32, e->kvd));
            L.has_bias = true;
        }
        QH_TRY(ealloc(e, (void**)&L.wgu, (size_t)2 * F * rbD));
        QH_TRY(gen(pre + "mlp.gate_proj.weight", tmp, wdtype, (size_t)F * D));
        QH_CHECK_HIP(hipMemcpy2DAsync(L.wgu, 2 * rbD, tmp, rbD, rbD, F, hipMemcpyDeviceToDevice, s));
        QH_TRY(gen(pre + "mlp.up_proj.weight", tmp, wdtype, (size_t)F * D));
        QH_CHECK_HIP(hipMemcpy2DAsync(L.wgu + rbD, 2 * rbD, tmp, rbD, rbD, F, hipMemcpyDeviceToDevice, s));
        QH_TRY(ealloc(e, (void**)&L.wd, (size_t)D * rbF));
        QH_TRY(gen(pre + "mlp.down_proj.weight", L.wd, wdtype, (size_t)D * F));
        QH_TRY(ealloc(e, (void**)&L.an, (size_t)D * 4));
        QH_TRY(ealloc(e, (void**)&L.fn, (size_t)D * 4));
        QH_TRY(fill1(L.an, D));
        QH_TRY(fill1(L.fn, D));
        L.have = T_ALL;
    }
    QH_TRY(ealloc(e, (void**)&e->onorm, (size_t)D * 4));
    QH_TRY(fill1(e->onorm, D));
    if (!tied) {
        e->dt_head = head_dtype;
        QH_TRY(ealloc(e, (void**)&e->head, (size_t)c.vocab_size * dt_row_bytes(head_dtype, D, 32)));
        QH_TRY(gen("lm_head.weight", e->head, head_dtype, (size_t)c.vocab_size * D));
    }
    QH_CHECK_HIP(hipStreamSynchronize(s));
    return QRAF_HIP_OK;
}

int qraf_engine_finalize(qraf_engine* e) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "finalize: null engine");
    QH_REQUIRE(e->embed, QRAF_HIP_ERR_STATE, "finalize: model.embed_tokens.weight missing");
    QH_REQUIRE(e->onorm, QRAF_HIP_ERR_STATE, "finalize: model.norm.weight missing");
    for (size_t l = 0; l < e->layers.size(); l++)
        QH_REQUIRE(e->layers[l].have == T_ALL, QRAF_HIP_ERR_STATE, "finalize: layer %zu incomplete (mask %x)", l,
                   e->layers[l].have);
    // Batched steps run the matrix-core GEMM on tile-major copies of the
    // quantized weights (same bytes, reordered so wavefront loads are contiguous).
    if (e->o.max_batch > 1 && !e->finalized) {
        const qraf_model_config& c = e->c;
        const int D = (int)c.hidden_size, F = (int)c.intermediate_size;
        auto tile = [&](const uint8_t* w, uint32_t dt, int N, int K, uint8_t** out) -> int {
            if ((dt != DT_Q8_0 && dt != DT_Q4_0) || K % 32 || (e->qbs && e->qbs != 32)) return QRAF_HIP_OK;
            QH_TRY(ealloc(e, (void**)out, tiled_weight_bytes(dt, N, K)));
            return launch_repack_tiles(w, dt, N, K, *out, e->stream);
        };
        for (auto& L : e->layers) {
            QH_TRY(tile(L.wqkv, L.dt_attn, e->qkvd, D, &L.wqkv_t));
            QH_TRY(tile(L.wo, L.dt_attn, D, e->qd, &L.wo_t));
            QH_TRY(tile(L.wgu, L.dt_mlp, 2 * F, D, &L.wgu_t));
            QH_TRY(tile(L.wd, L.dt_mlp, D, F, &L.wd_t));
        }
        QH_TRY(tile(e->head ? e->head : e->embed, e->head ? e->dt_head : e->dt_embed, (int)c.vocab_size, D, &e->head_t));
        QH_CHECK_HIP(hipStreamSynchronize(e->stream));
        e->fused = e->part_ws != nullptr;
        for (auto& L : e->layers) e->fused = e->fused && L.wqkv_t && L.wo_t && L.wgu_t && L.wd_t;
    }
    e->finalized = true;
    return QRAF_HIP_OK;
}

int qraf_engine_seq_create(qraf_engine* e, int32_t* id) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "seq_create: null engine");
    return e->pages.seq_create(id);
}

int qraf_engine_seq_release(qraf_engine* e, int32_t id) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "seq_release: null engine");
    QH_TRY(e->pages.seq_release(id));
    if (id < (int32_t)e->pen_slot.size() && e->pen_slot[id] >= 0) {  // its penalty slot back to the free list
        e->pen_free.push_back(e->pen_slot[id]);
        e->pen_slot[id] = -1;
        e->pen_live -= 1;
    }
    return QRAF_HIP_OK;
}

int qraf_engine_set_repetition_penalty(qraf_engine* e, int32_t id, float penalty) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "set_repetition_penalty: null engine");
    QH_REQUIRE(e->pages.live(id), QRAF_HIP_ERR_INVALID, "set_repetition_penalty: unknown sequence %d", id);
    QH_REQUIRE(std::isfinite(penalty) && penalty > 0.f, QRAF_HIP_ERR_INVALID, "set_repetition_penalty: penalty %g",
               (double)penalty);
    QH_REQUIRE(e->c.vocab_size % 4 == 0, QRAF_HIP_ERR_INVALID,
               "set_repetition_penalty: the device argmax needs a vocabulary that is a multiple of 4 (%u)",
               e->c.vocab_size);
    int32_t len = 0;
    QH_TRY(e->pages.seq_length(id, &len));
    QH_REQUIRE(len == 0, QRAF_HIP_ERR_STATE,
               "set_repetition_penalty: sequence %d already holds %d positions (set it before its first step)", id, len);
    if ((int32_t)e->pen_slot.size() <= id) {
        e->pen_slot.resize((size_t)id + 1, -1);
        e->pen_value.resize((size_t)id + 1, 1.f);
    }
    if (penalty == 1.0f) {  // sampler.cpp:39: no penalty; the slot, if any, goes back
        if (e->pen_slot[id] >= 0) {
            e->pen_free.push_back(e->pen_slot[id]);
            e->pen_slot[id] = -1;
            e->pen_live -= 1;
        }
        return QRAF_HIP_OK;
    }
    if (!e->pen_counts) {  // first use: 2 max_batch slots of V counts; captured steps hold the old (absent) counts
        const size_t bytes = (size_t)2 * e->o.max_batch * e->c.vocab_size * 4;
        void* p = nullptr;
        const hipError_t err = hipMalloc(&p, bytes);
        QH_REQUIRE(err == hipSuccess, QRAF_HIP_ERR_NOMEM, "set_repetition_penalty: %zu bytes of counts", bytes);
        e->allocs.push_back(p);
        e->pen_counts = (uint32_t*)p;
        for (int k = 2 * (int)e->o.max_batch - 1; k >= 0; k--) e->pen_free.push_back(k);
        QH_CHECK_HIP(hipStreamSynchronize(e->stream));  // steps in flight finish before their graphs go
        e->drop_graphs();
    }
    if (e->pen_slot[id] < 0) {
        QH_REQUIRE(!e->pen_free.empty(), QRAF_HIP_ERR_NOMEM,
                   "set_repetition_penalty: all %u penalty slots in use", 2 * e->o.max_batch);
        e->pen_slot[id] = e->pen_free.back();
        e->pen_free.pop_back();
        e->pen_live += 1;
        // stream-ordered after every step issued so far, before the next
        QH_CHECK_HIP(hipMemsetAsync(e->pen_counts + (size_t)e->pen_slot[id] * e->c.vocab_size, 0,
                                    (size_t)e->c.vocab_size * 4, e->stream));
    }
    e->pen_value[id] = penalty;
    return QRAF_HIP_OK;
}

int qraf_engine_seq_length(qraf_engine* e, int32_t id, int32_t* len) {
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "seq_length: null engine");
    return e->pages.seq_length(id, len);
}

int qraf_engine_free_pages(qraf_engine* e, int32_t* n) {
    QH_REQUIRE(e && n, QRAF_HIP_ERR_INVALID, "free_pages: null argument");
    *n = (int32_t)e->pages.free_pages();
    return QRAF_HIP_OK;
}

static double now_us() {
    return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// Validates one step and issues it on the engine's stream: its inputs into
// staging slot e->slot, the staging copy, the captured (or eager) launches,
// the logits copy (logits != null) and the greedy tokens' copy into the
// slot's h_amax (tok_out), then the slot's event.  The step joins e->pending.
static int step_issue(qraf_engine* e, int32_t n, const int32_t* seq_ids, const uint32_t* tokens,
                      const int32_t* token_src, const int32_t* positions, const uint8_t* want_logits, float* logits,
                      bool tok_out) {
    const double t_enter = now_us();
    QH_REQUIRE(e && seq_ids && tokens && positions, QRAF_HIP_ERR_INVALID, "step: null argument");
    QH_REQUIRE(e->finalized, QRAF_HIP_ERR_STATE, "step: engine not finalized");
    QH_REQUIRE(e->n_pending < 2, QRAF_HIP_ERR_STATE, "step: two steps in flight; collect one first");
    QH_REQUIRE(n > 0 && n <= (int32_t)e->o.max_batch, QRAF_HIP_ERR_INVALID, "step: %d rows (max_batch %u)", n,
               e->o.max_batch);
    const qraf_model_config& c = e->c;
    const int ps = (int)e->o.page_size, MP = e->max_pages;
    for (int i = 0; i < n; i++) {
        const int32_t from = token_src ? token_src[i] : -1;
        QH_REQUIRE(from < e->last_logit_rows, QRAF_HIP_ERR_INVALID,
                   "step: row %d takes the token of logit row %d of the previous step, which left %d", i, from,
                   e->last_logit_rows);
        QH_REQUIRE(from >= 0 || tokens[i] < c.vocab_size, QRAF_HIP_ERR_INVALID, "Token %u >= vocab %u", tokens[i],
                   c.vocab_size);
    }
    // With step graphs, a step of more than 8 rows runs padded to a multiple
    // of row_pad rows (at most max_batch), and its logit rows likewise, so
    // that steps of nearby sizes share one graph: a pad row is token 0 at
    // position 0 of the scratch page (context 1), which only pad rows write
    // and read, and it wants no logits; a pad logit row repeats the last real
    // one (whose logits are computed twice).  Every kernel's result for a row
    // depends on that row alone.
    const int n_real = n;
    const int n_pad = e->use_graphs && e->row_pad > 1 && n > 8
                          ? std::min((n + e->row_pad - 1) / e->row_pad * e->row_pad, (int)e->o.max_batch)
                          : n;
    int n_logit_rows = 0;
    int32_t* tok = e->h_in[e->slot];
    int32_t* pos = tok + n_pad;
    int32_t* ctx = pos + n_pad;
    int32_t* lrows = ctx + n_pad;
    int32_t* src = lrows + n_pad;
    int32_t* pslot = src + n_pad;
    float* ppen = (float*)(pslot + n_pad);
    int32_t* ptab = (int32_t*)(ppen + n_pad);
    // the rows' sequences and positions checked, their new pages taken from
    // the pool and their page-table rows written (nothing changes on failure);
    // step_ctx, the longest context of this step, sizes the attention grid
    // (and skips the merge)
    int step_ctx = 1;
    QH_TRY(e->pages.plan_step(n, seq_ids, positions, ptab, &step_ctx));
    e->last_logit_rows = 0;  // set again once this step's launches are issued
    for (int i = 0; i < n; i++) {
        src[i] = token_src ? token_src[i] : -1;
        tok[i] = src[i] >= 0 ? 0 : (int32_t)tokens[i];
        pos[i] = positions[i];
        ctx[i] = positions[i] + 1;
        const int32_t sq = seq_ids[i];
        const bool pen = sq < (int32_t)e->pen_slot.size() && e->pen_slot[sq] >= 0;
        pslot[i] = pen ? e->pen_slot[sq] : -1;
        ppen[i] = pen ? e->pen_value[sq] : 1.f;
        if (!want_logits || want_logits[i]) lrows[n_logit_rows++] = i;
    }
    for (int i = n; i < n_pad; i++) {
        tok[i] = 0;
        pos[i] = 0;
        ctx[i] = 1;
        src[i] = -1;
        pslot[i] = -1;
        ppen[i] = 1.f;
        for (int j = 0; j < MP; j++) ptab[(size_t)i * MP + j] = j == 0 ? e->scratch_page : 0;
    }
    const int n_logit_real = n_logit_rows;
    if (n_pad != n && n_logit_rows > 0) {
        const int nl = std::min((n_logit_rows + e->row_pad - 1) / e->row_pad * e->row_pad, n_pad);
        for (int i = n_logit_rows; i < nl; i++) lrows[i] = lrows[n_logit_real - 1];
        n_logit_rows = nl;
    }
    n = n_pad;
    hipStream_t s = e->stream;
    const size_t words = (size_t)n * (7 + MP);
    const bool head = n_logit_rows > 0 && (logits || tok_out);
    // greedy-only step (no logits wanted, none kept): the head's argmax fused into its GEMM where it runs one
    const bool argmax_only = head && !logits && tok_out && !e->keep_logits && e->pen_live == 0;
    const int head_mode = head ? (argmax_only ? 2 : 1) : 0;
    const int32_t* d_tok = e->d_in;
    const int32_t* d_pos = d_tok + n;
    const int32_t* d_ctx = d_pos + n;
    const int32_t* d_lrows = d_ctx + n;
    const int32_t* d_src = d_lrows + n;
    const int32_t* d_pslot = d_src + n;
    const float* d_ppen = (const float*)(d_pslot + n);
    const int32_t* d_ptab = (const int32_t*)(d_ppen + n);

    const int D = (int)c.hidden_size, F = (int)c.intermediate_size, V = (int)c.vocab_size;
    const int H = (int)c.num_heads, Hkv = (int)c.num_kv_heads, hd = e->hd;
    const float scale = 1.0f / sqrtf((float)hd);  // attention.cpp:122

    // 2-8 rows: the multi-vector matvec where it covers the shape and beats the GEMM
    const int qbs = e->qbs ? e->qbs : 32;  // the model's quant block size
    auto use_bmv = [&](uint32_t dt, int N, int K, int rows) {
        return rows >= 2 && rows <= MV_BATCH_SMALL && e->batch_mv && dt != DT_F32 && qbs == 32 &&
               matvec_batch_ok(dt, K, rows) &&
               (long long)rows * N * K <= MV_BATCH_WORK;
    };
    // y[n][N] = x[n][K] * W^T (+ add): matvec at batch 1, else the matrix-core GEMM
    // Wt: the tile-major copy (batched steps); K not a multiple of 32: one matvec per row
    // prep (optional): x is formed from its source first (norm or SiLU-gate):
    // inside the matvec at batch 1, else by a kernel writing prep->xbuf
    // rope (one row only): the QKV epilogue fused into the matvec when its
    // one-shot form runs; *fused says whether it did
    auto proj = [&](const uint8_t* W, const uint8_t* Wt, uint32_t dt, int N, int K, const float* x, int rows, float* y,
                    const float* add, const MvPrep* prep = nullptr, const MvRope* rope = nullptr,
                    bool* fused = nullptr) -> int {
        if (fused) *fused = false;
        if (use_bmv(dt, N, K, rows))
            return launch_matvec_q_batch(W, dt, N, K, x, prep && prep->op == XP_SILU_GATE ? 2 * K : K, rows, y, N, s,
                                         add, prep);
        if (prep && (dt == DT_F32 || rows != 1)) {
            if (prep->op == XP_NORM)
                hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, s, x, prep->w, K, prep->eps,
                                   prep->xbuf, nullptr);
            else
                hipLaunchKernelGGL(silu_gate_kernel, dim3(std::min((rows * K + 255) / 256, 4096)), dim3(256), 0, s, x,
                                   K, rows, prep->xbuf);
            QH_CHECK_HIP(hipGetLastError());
            x = prep->xbuf;
            prep = nullptr;
        }
        if (dt == DT_F32) {
            for (int r = 0; r < rows; r++)
                QH_TRY(launch_matvec_f32((const float*)W, x + (size_t)r * K, y + (size_t)r * N, N, K, s,
                                         add ? add + (size_t)r * N : nullptr));
            return QRAF_HIP_OK;
        }
        if (rows == 1 && rope) return launch_matvec_q(W, dt, qbs, N, K, x, y, s, add, prep, rope, fused);
        if (rows == 1 || !Wt) {
            for (int r = 0; r < rows; r++)
                QH_TRY(launch_matvec_q(W, dt, qbs, N, K, x + (size_t)r * K, y + (size_t)r * N, s,
                                       add ? add + (size_t)r * N : nullptr, prep));
            return QRAF_HIP_OK;
        }
        QH_TRY(launch_split_bf16(x, e->xh, e->xl, rows, K, 0, nullptr, s));
        return launch_qgemm(Wt, dt, 32, N, K, e->xh, e->xl, rows, y, add, e->gemm_ws, e->gemm_ws_bytes, s, true);
    };

    // The step's launches, stream-ordered: embedding, layers, head and argmax.
    // ctx_grid >= every row's context sizes the attention grid.
    auto enqueue = [&](int ctx_grid) -> int {
        hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, s, e->embed, e->dt_embed, qbs, D, d_tok, d_src, e->amax,
                           e->h, d_pslot, e->pen_counts, V);
        QH_CHECK_HIP(hipGetLastError());
        // steps of 2-8 rows whose QKV and O projections go to the multi-vector
        // matvec take the per-projection loop below (gate/up and down each
        // take it or the GEMM)
        bool small_mv = n >= 2 && n <= MV_BATCH_SMALL && e->batch_mv;
        for (uint32_t l = 0; l < c.num_layers && small_mv; l++) {
            const qraf_engine::Layer& L = e->layers[l];
            small_mv = use_bmv(L.dt_attn, e->qkvd, D, n) && use_bmv(L.dt_attn, D, e->qd, n);
        }
        const bool gemm_layers = n > 1 && e->fused && !small_mv;
        if (gemm_layers) {
            // Batched layer on the matrix cores, 9 launches (8 with the SwiGLU
            // epilogue): each projection writes split-K partials that the next
            // kernel sums (with the bias, residual, norm or SiLU-gate it applies
            // anyway), and every kernel that feeds a projection writes its input
            // as the hi (bf16) and lo (fp16) planes directly.
            QH_TRY(launch_residual_norm_split(nullptr, 0, 0, e->h, e->layers[0].an, D, c.rms_norm_eps, e->xh, e->xl, n, s));
            for (uint32_t l = 0; l < c.num_layers; l++) {
                qraf_engine::Layer& L = e->layers[l];
                uint8_t* kc = e->kpool + (size_t)l * e->layer_kv_bytes;
                uint8_t* vc = e->vpool + (size_t)l * e->layer_kv_bytes;
                float* P = (float*)e->part_ws;
                int S = 0;
                QH_TRY(launch_qgemm(L.wqkv_t, L.dt_attn, 32, e->qkvd, D, e->xh, e->xl, n, e->qkv, nullptr, P,
                                    e->part_ws_bytes, s, true, &S));
                QH_TRY(launch_rope_append(P, L.has_bias ? L.bqkv : nullptr, n, H, Hkv, hd, d_pos, e->rope, e->q, kc, vc,
                                          e->o.kv_dtype, d_ptab, MP, ps, s, S, (size_t)n * e->qkvd));
                QH_TRY(launch_attention(e->q, kc, vc, e->o.kv_dtype, d_ptab, MP, d_ctx, n, H, Hkv, hd, ps, scale,
                                        ctx_grid, nullptr, e->attn_ws, e->attn_ws_bytes, s, e->xh, e->xl));
                QH_TRY(launch_qgemm(L.wo_t, L.dt_attn, 32, D, e->qd, e->xh, e->xl, n, e->qkv, nullptr, P, e->part_ws_bytes,
                                    s, true, &S));
                QH_TRY(launch_residual_norm_split(P, S, (size_t)n * D, e->h, L.fn, D, c.rms_norm_eps, e->xh, e->xl, n, s));
                if (e->fuse_swiglu && n > 256) {
                    // gate/up unsplit with the SiLU-gate in its epilogue, writing
                    // the down GEMM's planes (its own buffers: xh/xl are its input).
                    // Above 256 rows only: MI355X, Qwen2.5-3B shapes, a decode step
                    // at 384 / 512 rows 10.80 -> 9.80 / 12.03 -> 11.62 ms, at 48-256
                    // rows about 1% slower than split-K partials and a SiLU launch
                    QH_TRY(launch_qgemm_silu(L.wgu_t, L.dt_mlp, 2 * F, D, e->xh, e->xl, n, e->ah, e->al, s));
                    QH_TRY(launch_qgemm(L.wd_t, L.dt_mlp, 32, D, F, e->ah, e->al, n, e->qkv, nullptr, P, e->part_ws_bytes,
                                        s, true, &S));
                } else {
                    QH_TRY(launch_qgemm(L.wgu_t, L.dt_mlp, 32, 2 * F, D, e->xh, e->xl, n, e->qkv, nullptr, P,
                                        e->part_ws_bytes, s, true, &S));
                    QH_TRY(launch_split_bf16(P, e->xh, e->xl, n, F, 1, nullptr, s, S, (size_t)n * 2 * F));
                    QH_TRY(launch_qgemm(L.wd_t, L.dt_mlp, 32, D, F, e->xh, e->xl, n, e->qkv, nullptr, P, e->part_ws_bytes,
                                        s, true, &S));
                }
                const float* wn = l + 1 < c.num_layers ? e->layers[l + 1].an : nullptr;  // last layer: residual only
                QH_TRY(launch_residual_norm_split(P, S, (size_t)n * D, e->h, wn, D, c.rms_norm_eps, e->xh, e->xl, n, s));
            }
        }
        for (uint32_t l = 0; l < c.num_layers && !gemm_layers; l++) {
            qraf_engine::Layer& L = e->layers[l];
            uint8_t* kc = e->kpool + (size_t)l * e->layer_kv_bytes;
            uint8_t* vc = e->vpool + (size_t)l * e->layer_kv_bytes;
            const MvPrep attn_norm{XP_NORM, L.an, c.rms_norm_eps, e->xn};  // transformer.cpp:586
            // one row: bias, RoPE and the K/V store fused into the QKV matvec where its one-shot form runs
            MvRope rope;
            rope.bias = L.has_bias ? L.bqkv : nullptr;
            rope.pos = d_pos;
            rope.rope = e->rope;
            rope.q_out = e->q;
            rope.kc = kc;
            rope.vc = vc;
            rope.page_table = d_ptab;
            rope.H = H;
            rope.Hkv = Hkv;
            rope.hd = hd;
            rope.page_size = ps;
            rope.kv_dtype = e->o.kv_dtype;
            bool fused = false;
            QH_TRY(proj(L.wqkv, L.wqkv_t, L.dt_attn, e->qkvd, D, e->h, n, e->qkv, nullptr, &attn_norm,
                        e->fuse_rope && e->o.kv_dtype != DT_I8 ? &rope : nullptr, &fused));
            if (!fused)
                QH_TRY(launch_rope_append(e->qkv, L.has_bias ? L.bqkv : nullptr, n, H, Hkv, hd, d_pos, e->rope, e->q,
                                          kc, vc, e->o.kv_dtype, d_ptab, MP, ps, s));
            QH_TRY(launch_attention(e->q, kc, vc, e->o.kv_dtype, d_ptab, MP, d_ctx, n, H, Hkv, hd, ps, scale, ctx_grid,
                                    e->att, e->attn_ws, e->attn_ws_bytes, s));
            QH_TRY(proj(L.wo, L.wo_t, L.dt_attn, D, e->qd, e->att, n, e->h, e->h));  // + residual (transformer.cpp:593)
            const MvPrep ffn_norm{XP_NORM, L.fn, c.rms_norm_eps, e->xn};  // transformer.cpp:595
            QH_TRY(proj(L.wgu, L.wgu_t, L.dt_mlp, 2 * F, D, e->h, n, e->gu, nullptr, &ffn_norm));
            if (n == 1 || !L.wd_t || use_bmv(L.dt_mlp, D, F, n)) {
                const MvPrep gate{XP_SILU_GATE, nullptr, 0.f, e->act};  // attention.cpp:172-183
                QH_TRY(proj(L.wd, L.wd_t, L.dt_mlp, D, F, e->gu, n, e->h, e->h, &gate));  // + residual (transformer.cpp:601)
            } else {
                QH_TRY(launch_split_bf16(e->gu, e->xh, e->xl, n, F, 1, nullptr, s));  // SiLU-gate fused into the split
                QH_TRY(launch_qgemm(L.wd_t, L.dt_mlp, 32, D, F, e->xh, e->xl, n, e->h, e->h, e->gemm_ws, e->gemm_ws_bytes, s,
                                    true));
            }
        }
        QH_CHECK_HIP(hipGetLastError());
        if (head) {
            // final norm of the rows that want logits (transformer.cpp:605), then the head
            const uint8_t* W = e->head ? e->head : e->embed;  // tied head reads the embedding (transformer.cpp:392-400)
            const uint32_t dt = e->head ? e->dt_head : e->dt_embed;
            if (n == 1 && dt != DT_F32) {
                const MvPrep out_norm{XP_NORM, e->onorm, c.rms_norm_eps, e->xhead};
                QH_TRY(proj(W, e->head_t, dt, V, D, e->h, 1, e->logits, nullptr, &out_norm));
            } else {
                hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(n_logit_rows), dim3(256), 0, s, e->h, e->onorm, D,
                                   c.rms_norm_eps, e->xhead, d_lrows);
                if (argmax_only && dt != DT_F32 && e->head_t && !use_bmv(dt, V, D, n_logit_rows) &&
                    qgemm_argmax_fits(dt, V, D, n_logit_rows, e->am_keys_bytes)) {
                    // the GEMM proj would run, with Sampler::argmax in its epilogue
                    QH_TRY(launch_split_bf16(e->xhead, e->xh, e->xl, n_logit_rows, D, 0, nullptr, s));
                    bool done = false;
                    QH_TRY(launch_qgemm_argmax(e->head_t, dt, V, D, e->xh, e->xl, n_logit_rows, e->am_keys,
                                               e->am_keys_bytes, e->amax, s, &done));
                    QH_REQUIRE(done, QRAF_HIP_ERR_STATE, "engine: fused head not launched");
                    return QRAF_HIP_OK;
                }
                QH_TRY(proj(W, e->head_t, dt, V, D, e->xhead, n_logit_rows, e->logits, nullptr));
            }
            if (V % 4 == 0) {  // one pass per row (logits rows are 16-byte aligned then)
                hipLaunchKernelGGL(argmax_rows_kernel, dim3(n_logit_rows), dim3(1024), 0, s, e->logits, V, e->amax,
                                   d_lrows, d_pslot, d_ppen, e->pen_counts);
            } else {
                hipLaunchKernelGGL(argmax_chunk_kernel, dim3(ARGMAX_CHUNKS, n_logit_rows), dim3(256), 0, s, e->logits, V,
                                   e->am_val, e->am_idx);
                hipLaunchKernelGGL(argmax_final_kernel, dim3(n_logit_rows), dim3(64), 0, s, e->am_val, e->am_idx, V, e->amax);
            }
            QH_CHECK_HIP(hipGetLastError());
        }
        return QRAF_HIP_OK;
    };

    // the staging copy stays outside the captured launches: its source is the
    // slot's pinned buffer, which alternates between steps
    QH_CHECK_HIP(hipMemcpyAsync(e->d_in, e->h_in[e->slot], words * 4, hipMemcpyHostToDevice, s));
    if (e->use_graphs) {
        // context bound rounded up to a power of two (>= one attention chunk) so
        // that a decode reuses one graph for many steps
        int ctx_grid = 256;
        while (ctx_grid < step_ctx) ctx_grid *= 2;
        ctx_grid = std::min(ctx_grid, e->capacity);
        const uint32_t gen = tuning_generation();
        qraf_engine::StepGraph* g = nullptr;
        for (auto& sg : e->graphs)
            if (sg.n == n && sg.n_logit_rows == n_logit_rows && sg.ctx == ctx_grid && sg.head == head_mode && sg.gen == gen)
                g = &sg;
        bool second = false;
        if (!g) {
            for (auto it = e->seen.begin(); it != e->seen.end(); ++it)
                if (it->n == n && it->n_logit_rows == n_logit_rows && it->ctx == ctx_grid && it->head == head_mode &&
                    it->gen == gen) {
                    second = true;
                    e->seen.erase(it);
                    break;
                }
            if (!second) {
                qraf_engine::StepGraph sg;
                sg.n = n;
                sg.n_logit_rows = n_logit_rows;
                sg.ctx = ctx_grid;
                sg.head = head_mode;
                sg.gen = gen;
                if (e->seen.size() >= 4 * MAX_STEP_GRAPHS) e->seen.erase(e->seen.begin());
                e->seen.push_back(sg);
            }
        }
        if (!g && !second) {
            QH_TRY(enqueue(ctx_grid));  // first sighting: eager
            e->stats.eager_steps += 1;
        } else if (!g) {
            hipGraph_t graph = nullptr;
            e->stats.graph_captures += 1;
            QH_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue(ctx_grid);
            const hipError_t ec = hipStreamEndCapture(s, &graph);
            if (rc != QRAF_HIP_OK) {
                if (graph) hipGraphDestroy(graph);
                return rc;
            }
            QH_CHECK_HIP(ec);
            hipGraphExec_t exec = nullptr;
            const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            hipGraphDestroy(graph);
            QH_CHECK_HIP(ei);
            if (e->graphs.size() >= MAX_STEP_GRAPHS) {  // evict the least recently used
                auto lru = std::min_element(e->graphs.begin(), e->graphs.end(),
                                            [](const qraf_engine::StepGraph& a, const qraf_engine::StepGraph& b) {
                                                return a.used < b.used;
                                            });
                hipGraphExecDestroy(lru->exec);
                e->graphs.erase(lru);
            }
            qraf_engine::StepGraph sg;
            sg.n = n;
            sg.n_logit_rows = n_logit_rows;
            sg.ctx = ctx_grid;
            sg.head = head_mode;
            sg.gen = gen;
            sg.exec = exec;
            e->graphs.push_back(sg);
            g = &e->graphs.back();
        }
        if (g) {
            g->used = ++e->graph_clock;
            QH_CHECK_HIP(hipGraphLaunch(g->exec, s));
            e->stats.graph_launches += 1;
        }
    } else {
        QH_TRY(enqueue(step_ctx));
        e->stats.eager_steps += 1;
    }
    e->last_logit_rows = head ? n_logit_real : 0;
    e->last_logits_kept = !argmax_only;
    if (head && logits)
        QH_CHECK_HIP(hipMemcpyAsync(logits, e->logits, (size_t)n_logit_real * V * 4, hipMemcpyDeviceToHost, s));
    // tokens come back through pinned staging: an async copy into pageable
    // memory would block the host until the whole step has run
    const int slot = e->slot;
    const bool toks = head && tok_out;
    if (toks) QH_CHECK_HIP(hipMemcpyAsync(e->h_amax[slot], e->amax, (size_t)n_logit_real * 4, hipMemcpyDeviceToHost, s));
    QH_CHECK_HIP(hipEventRecord(e->done_ev[slot], s));
    e->pending[e->n_pending].slot = slot;
    e->pending[e->n_pending].n_tok = toks ? n_logit_real : 0;
    e->n_pending += 1;
    e->slot ^= 1;
    e->stats.steps += 1;
    e->stats.rows += (uint64_t)n_real;
    e->stats.pad_rows += (uint64_t)(n - n_real);
    e->stats.host_us += now_us() - t_enter;
    return QRAF_HIP_OK;
}

int qraf_engine_step(qraf_engine* e, int32_t n, const int32_t* seq_ids, const uint32_t* tokens,
                     const int32_t* positions, const uint8_t* want_logits, float* logits, uint32_t* next_tokens) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "step: null engine");
    QH_REQUIRE(e->n_pending == 0, QRAF_HIP_ERR_STATE, "step: %d asynchronous steps not collected", e->n_pending);
    QH_TRY(step_issue(e, n, seq_ids, tokens, nullptr, positions, want_logits, logits, next_tokens != nullptr));
    const qraf_engine::Pending p = e->pending[0];
    e->n_pending = 0;
    const double t0 = now_us();
    QH_CHECK_HIP(hipStreamSynchronize(e->stream));  // also completes a logits copy into pageable memory
    e->stats.wait_us += now_us() - t0;
    if (next_tokens && p.n_tok) memcpy(next_tokens, e->h_amax[p.slot], (size_t)p.n_tok * 4);
    return QRAF_HIP_OK;
}

// One step issued without waiting for it: row i's token is tokens[i], or,
// where token_src[i] >= 0, the greedy token of logit row token_src[i] of the
// step issued just before (taken on the device).  At most two steps are in
// flight; qraf_engine_step_collect returns them in order.
int qraf_engine_step_async(qraf_engine* e, int32_t n, const int32_t* seq_ids, const uint32_t* tokens,
                           const int32_t* token_src, const int32_t* positions, const uint8_t* want_logits) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "step_async: null engine");
    return step_issue(e, n, seq_ids, tokens, token_src, positions, want_logits, nullptr, true);
}

int qraf_engine_step_collect(qraf_engine* e, uint32_t* next_tokens, int32_t* n_tokens) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "step_collect: null engine");
    QH_REQUIRE(e->n_pending > 0, QRAF_HIP_ERR_STATE, "step_collect: no step in flight");
    const qraf_engine::Pending p = e->pending[0];
    e->pending[0] = e->pending[1];
    e->n_pending -= 1;
    const double t0 = now_us();
    QH_CHECK_HIP(hipEventSynchronize(e->done_ev[p.slot]));
    e->stats.wait_us += now_us() - t0;
    if (next_tokens && p.n_tok) memcpy(next_tokens, e->h_amax[p.slot], (size_t)p.n_tok * 4);
    if (n_tokens) *n_tokens = p.n_tok;
    return QRAF_HIP_OK;
}

// The logit rows the last step left in HBM (rows row0 .. row0+rows-1 of them) -> host.
int qraf_engine_read_logits(qraf_engine* e, int32_t row0, int32_t rows, float* out) {
    clear_error();
    QH_REQUIRE(e && out && rows > 0 && row0 >= 0, QRAF_HIP_ERR_INVALID, "read_logits: bad arguments");
    QH_REQUIRE(row0 + rows <= e->last_logit_rows, QRAF_HIP_ERR_STATE,
               "read_logits: rows %d..%d, the last step left %d logit rows", row0, row0 + rows - 1, e->last_logit_rows);
    QH_REQUIRE(e->last_logits_kept, QRAF_HIP_ERR_STATE,
               "read_logits: the last step was greedy-only and kept no logits (qraf_engine_set_keep_logits)");
    const size_t V = e->c.vocab_size;
    QH_CHECK_HIP(hipMemcpyAsync(out, e->logits + (size_t)row0 * V, (size_t)rows * V * 4, hipMemcpyDeviceToHost,
                                e->stream));
    QH_CHECK_HIP(hipStreamSynchronize(e->stream));
    return QRAF_HIP_OK;
}

int qraf_engine_set_fusion(qraf_engine* e, int32_t flags) {
    clear_error();
    QH_REQUIRE(e && (flags & ~7) == 0, QRAF_HIP_ERR_INVALID, "set_fusion: flags %d", flags);
    QH_CHECK_HIP(hipStreamSynchronize(e->stream));  // no captured step still in flight
    e->fuse_rope = (flags & 1) != 0;
    e->fuse_swiglu = (flags & 2) != 0;
    e->batch_mv = (flags & 4) != 0;
    e->drop_graphs();  // captured steps hold the other form
    return QRAF_HIP_OK;
}

int qraf_engine_set_row_padding(qraf_engine* e, int32_t rows) {
    clear_error();
    QH_REQUIRE(e && rows >= 1 && rows <= 256, QRAF_HIP_ERR_INVALID, "set_row_padding: rows %d outside 1..256", rows);
    e->row_pad = rows;
    return QRAF_HIP_OK;
}

int qraf_engine_get_stats(qraf_engine* e, qraf_engine_stats* out, int32_t reset) {
    clear_error();
    QH_REQUIRE(e && out, QRAF_HIP_ERR_INVALID, "get_stats: null argument");
    *out = e->stats;
    if (reset) e->stats = qraf_engine_stats{};
    return QRAF_HIP_OK;
}

// Sampler::apply_repetition_penalty + Sampler::sample on the last step's
// logit rows (sampler.cpp:37-128), where they lie in HBM.
int qraf_engine_sample(qraf_engine* e, int32_t row0, int32_t rows, const qraf_sampling_params* p,
                       const uint32_t* recent, const int32_t* counts, int32_t stride, const float* uniforms,
                       uint32_t* tokens) {
    clear_error();
    QH_REQUIRE(e && p && tokens && rows > 0 && row0 >= 0, QRAF_HIP_ERR_INVALID, "sample: bad arguments");
    QH_REQUIRE(row0 + rows <= e->last_logit_rows, QRAF_HIP_ERR_STATE,
               "sample: rows %d..%d, the last step left %d logit rows", row0, row0 + rows - 1, e->last_logit_rows);
    QH_REQUIRE(e->last_logits_kept, QRAF_HIP_ERR_STATE,
               "sample: the last step was greedy-only and kept no logits (qraf_engine_set_keep_logits)");
    const bool greedy = !(p->temperature > 0.f);
    const bool pen = p->repetition_penalty != 1.0f && recent;
    QH_REQUIRE(!pen || (counts && stride > 0), QRAF_HIP_ERR_INVALID, "sample: recent tokens need counts");
    QH_REQUIRE(greedy || uniforms, QRAF_HIP_ERR_INVALID, "sample: temperature %g needs uniforms", p->temperature);
    const size_t rb = ((size_t)rows * 4 + 255) / 256 * 256;
    const size_t rec = pen ? ((size_t)rows * stride * 4 + 255) / 256 * 256 : 0;
    const size_t need = 3 * rb + rec;  // tokens, uniforms, counts, recent
    if (need > e->samp_cap) {
        const size_t cap = std::max(need, (size_t)1 << 20);
        QH_TRY(ealloc(e, (void**)&e->samp, cap));  // held until the engine is destroyed
        e->samp_cap = cap;
    }
    const size_t sort_need = sample_sort_bytes(rows, (int)e->c.vocab_size, *p);
    if (sort_need > e->sort_cap) {
        QH_TRY(ealloc(e, &e->sort_ws, sort_need));  // held until the engine is destroyed
        e->sort_cap = sort_need;
    }
    hipStream_t s = e->stream;
    uint32_t* d_tok = (uint32_t*)e->samp;
    float* d_uni = (float*)(e->samp + rb);
    int32_t* d_cnt = (int32_t*)(e->samp + 2 * rb);
    uint32_t* d_rec = (uint32_t*)(e->samp + 3 * rb);
    if (!greedy) QH_CHECK_HIP(hipMemcpyAsync(d_uni, uniforms, (size_t)rows * 4, hipMemcpyHostToDevice, s));
    if (pen) {
        QH_CHECK_HIP(hipMemcpyAsync(d_cnt, counts, (size_t)rows * 4, hipMemcpyHostToDevice, s));
        QH_CHECK_HIP(hipMemcpyAsync(d_rec, recent, (size_t)rows * stride * 4, hipMemcpyHostToDevice, s));
    }
    QH_TRY(launch_sample(e->logits + (size_t)row0 * e->c.vocab_size, rows, (int)e->c.vocab_size, *p,
                         pen ? d_rec : nullptr, pen ? d_cnt : nullptr, stride, greedy ? nullptr : d_uni, d_tok,
                         e->sort_ws, e->sort_cap, s));
    QH_CHECK_HIP(hipMemcpyAsync(tokens, d_tok, (size_t)rows * 4, hipMemcpyDeviceToHost, s));
    QH_CHECK_HIP(hipStreamSynchronize(s));
    return QRAF_HIP_OK;
}

// Greedy-only steps without logits (keep = 0) or with them (1, the default).
int qraf_engine_set_keep_logits(qraf_engine* e, int32_t keep) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "set_keep_logits: null engine");
    e->keep_logits = keep != 0;
    return QRAF_HIP_OK;
}

// Graph capture and replay of steps (on by default); off: every step launches eagerly.
int qraf_engine_set_graphs(qraf_engine* e, int32_t on) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "set_graphs: null engine");
    QH_CHECK_HIP(hipStreamSynchronize(e->stream));
    e->use_graphs = on != 0;
    if (!e->use_graphs) e->drop_graphs();
    return QRAF_HIP_OK;
}

// Transformer::forward(token, pos) on the engine's default sequence.
int qraf_engine_forward(qraf_engine* e, uint32_t token, int32_t pos, float* logits) {
    clear_error();
    QH_REQUIRE(e && logits, QRAF_HIP_ERR_INVALID, "forward: null argument");
    if (e->default_seq < 0) QH_TRY(qraf_engine_seq_create(e, &e->default_seq));
    return qraf_engine_step(e, 1, &e->default_seq, &token, &pos, nullptr, logits, nullptr);
}

// Transformer::reset(): the default sequence forgets its cache.
int qraf_engine_reset(qraf_engine* e) {
    clear_error();
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "reset: null engine");
    if (e->default_seq >= 0) {
        QH_TRY(qraf_engine_seq_release(e, e->default_seq));
        e->default_seq = -1;
    }
    return QRAF_HIP_OK;
}

}  // extern "C"
