// attention.hip -- ragged decode attention over a block-paged KV cache.
//
// Replaces the per-head score / softmax / weighted-sum loops of
// attention_forward (reference attention.cpp:122-150) and the KVCache store
// (attention.cpp:39-44, :119), for a batch of sequences that each add one
// token.  KV layout in HBM, per layer:
//     K, V : [num_pages][Hkv][page_size][head_dim]   (f32 or f16)
// and a page table per sequence maps logical page j (positions
// j*page_size .. +page_size-1) to a physical page.
//
// Work decomposition: the context of every sequence is cut into chunks of
// CH = 256 positions; one workgroup handles one (sequence, chunk) item for
// one KV head and all H/Hkv query heads that share it (GQA).  Items are
// numbered by an exclusive prefix sum of ceil(ctx_s / CH) over the ragged
// batch, which every workgroup recomputes in LDS from the device-resident
// context lengths, so the packing follows whatever lengths are on the device
// when the kernel runs (no host round trip).  Sequences with several chunks
// write (max, sum, unnormalised output) partials; the last chunk to finish
// (an atomic counter per sequence and KV head) merges them in chunk order.
//
// Scores: thread = position; q is read from LDS (broadcast), K rows with
// 16-byte loads.  Output: thread = (head subset, dimension), V rows read
// coalesced, probabilities broadcast from LDS.  fp32 arithmetic throughout.
#include <math.h>

#include "common.h"

namespace qraf_hip {

constexpr int ACH = 256;  // positions per chunk = threads per workgroup

template <typename KT>
__device__ __forceinline__ float kv_load(const KT* p) {
    return (float)*p;
}

// load 8 consecutive K/V values starting at p (16- or 32-byte aligned)
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void load8(const _Float16* p, float (&v)[8]) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const h8 a = *(const h8*)p;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)a[i];
}

struct AttnArgs {
    const float* q;            // [n][H][HD]
    const void* kc;            // layer K pages
    const void* vc;            // layer V pages
    const int32_t* page_table; // [n][max_pages]
    const int32_t* ctx;        // [n] positions attended (pos + 1)
    float* out;                // [n][H][HD]
    float* part_o;             // [items][H][HD]   (multi-chunk partials)
    float* part_ml;            // [items][H][2]
    uint32_t* counters;        // [n][Hkv]          zero on entry, zero on exit
    int n, H, Hkv, page_size, max_pages, max_ctx;
    float scale;
};

template <typename KT, int HD, int G>
__global__ __launch_bounds__(ACH) void attn_decode_kernel(AttnArgs a) {
    static_assert(HD % 8 == 0, "head_dim must be a multiple of 8");
    constexpr int NOUT = G * HD;                 // outputs of this workgroup
    constexpr int HPT = (NOUT + ACH - 1) / ACH;  // outputs per thread in the PV phase
    __shared__ int s_pref[1025];
    __shared__ float s_q[G][HD];
    __shared__ float s_p[G][ACH];
    __shared__ float s_red[G][4];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.y;
    const int n = a.n;

    // ---- item -> (sequence, chunk): exclusive prefix sum of chunk counts
    // (block scan: 4 entries per thread, wave scan, then across the 4 waves)
    {
        int c[4], run = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = tid * 4 + j;
            c[j] = i < n ? (min(a.ctx[i], a.max_ctx) + ACH - 1) / ACH : 0;
            run += c[j];
        }
        int incl = run;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (lane >= o) incl += v;
        }
        __shared__ int s_wtot[4];
        if (lane == 63) s_wtot[wave] = incl;
        __syncthreads();
        int off = incl - run;
        for (int w = 0; w < wave; w++) off += s_wtot[w];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = tid * 4 + j;
            off += c[j];
            if (i < n) s_pref[i + 1] = off;
        }
        if (tid == 0) s_pref[0] = 0;
        __syncthreads();
    }
    const int item = blockIdx.x;
    if (item >= s_pref[n]) return;
    int lo = 0, hi = n - 1;  // largest s with s_pref[s] <= item
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_pref[mid] <= item) lo = mid;
        else hi = mid - 1;
    }
    const int s = lo, chunk = item - s_pref[s], nchunks = s_pref[s + 1] - s_pref[s];
    const int ctx = min(a.ctx[s], a.max_ctx);
    const int t0 = chunk * ACH;

    // ---- q of the G heads sharing this KV head
    for (int i = tid; i < G * HD; i += ACH) s_q[i / HD][i % HD] = a.q[((size_t)s * a.H + kvh * G) * HD + i];
    __syncthreads();

    // ---- scores: thread = position t0 + tid
    const KT* kc = (const KT*)a.kc;
    const KT* vc = (const KT*)a.vc;
    const int t = t0 + tid;
    float sc[G];
#pragma unroll
    for (int h = 0; h < G; h++) sc[h] = 0.f;
    if (t < ctx) {
        const int page = a.page_table[(size_t)s * a.max_pages + t / a.page_size];
        const KT* kr = kc + (((size_t)page * a.Hkv + kvh) * a.page_size + t % a.page_size) * HD;
        for (int d = 0; d < HD; d += 8) {
            float kv[8];
            load8(kr + d, kv);
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float4 qa = *(const float4*)&s_q[h][d], qb = *(const float4*)&s_q[h][d + 4];
                sc[h] = __builtin_fmaf(qa.x, kv[0], sc[h]);
                sc[h] = __builtin_fmaf(qa.y, kv[1], sc[h]);
                sc[h] = __builtin_fmaf(qa.z, kv[2], sc[h]);
                sc[h] = __builtin_fmaf(qa.w, kv[3], sc[h]);
                sc[h] = __builtin_fmaf(qb.x, kv[4], sc[h]);
                sc[h] = __builtin_fmaf(qb.y, kv[5], sc[h]);
                sc[h] = __builtin_fmaf(qb.z, kv[6], sc[h]);
                sc[h] = __builtin_fmaf(qb.w, kv[7], sc[h]);
            }
        }
#pragma unroll
        for (int h = 0; h < G; h++) sc[h] *= a.scale;  // attention.cpp:134: dot * scale
    } else {
#pragma unroll
        for (int h = 0; h < G; h++) sc[h] = -INFINITY;
    }

    // ---- chunk softmax statistics per head
    float m[G], l[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        float v = sc[h];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
        if (lane == 0) s_red[h][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; h++) m[h] = fmaxf(fmaxf(s_red[h][0], s_red[h][1]), fmaxf(s_red[h][2], s_red[h][3]));
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; h++) {
        const float p = (t < ctx) ? __expf(sc[h] - m[h]) : 0.f;
        s_p[h][tid] = p;
        float v = p;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0) s_red[h][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; h++) l[h] = (s_red[h][0] + s_red[h][1]) + (s_red[h][2] + s_red[h][3]);

    // ---- weighted sum of V: thread handles outputs o = tid + 256*j (head
    // o / HD, dimension o % HD); for head_dim >= 64 a wave's 64 outputs share
    // one head, so the probabilities are LDS broadcasts and V reads coalesce.
    float o[HPT];
#pragma unroll
    for (int j = 0; j < HPT; j++) o[j] = 0.f;
    const int tend = min(ACH, ctx - t0);
    int cur_lp = -1;
    const KT* vpage = nullptr;
    for (int tt = 0; tt < tend; tt++) {
        const int tp = t0 + tt;
        const int lp = tp / a.page_size;
        if (lp != cur_lp) {
            cur_lp = lp;
            const int page = a.page_table[(size_t)s * a.max_pages + lp];
            vpage = vc + ((size_t)page * a.Hkv + kvh) * a.page_size * HD;
        }
        const KT* vrow = vpage + (size_t)(tp % a.page_size) * HD;
#pragma unroll
        for (int j = 0; j < HPT; j++) {
            const int oi = tid + ACH * j;
            if (oi < NOUT) o[j] = __builtin_fmaf(s_p[oi / HD][tt], kv_load(vrow + oi % HD), o[j]);
        }
    }

    if (nchunks == 1) {
#pragma unroll
        for (int j = 0; j < HPT; j++) {
            const int oi = tid + ACH * j;
            if (oi < NOUT) a.out[((size_t)s * a.H + kvh * G) * HD + oi] = o[j] / l[oi / HD];
        }
        return;
    }

    // ---- multi-chunk: publish partials, last chunk merges in chunk order
#pragma unroll
    for (int j = 0; j < HPT; j++) {
        const int oi = tid + ACH * j;
        if (oi < NOUT) a.part_o[((size_t)item * a.H + kvh * G) * HD + oi] = o[j];
    }
    if (tid < G) {
        a.part_ml[((size_t)item * a.H + kvh * G + tid) * 2 + 0] = m[tid];
        a.part_ml[((size_t)item * a.H + kvh * G + tid) * 2 + 1] = l[tid];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.counters[(size_t)s * a.Hkv + kvh], 1u);
        s_last = (prev == (uint32_t)nchunks - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const int base = s_pref[s];
#pragma unroll
    for (int j = 0; j < HPT; j++) {
        const int oi = tid + ACH * j;
        if (oi >= NOUT) continue;
        const size_t hidx = (size_t)kvh * G + oi / HD;
        float M = -INFINITY;
        for (int c = 0; c < nchunks; c++) M = fmaxf(M, a.part_ml[((size_t)(base + c) * a.H + hidx) * 2]);
        float L = 0.f, O = 0.f;
        for (int c = 0; c < nchunks; c++) {
            const size_t it = (size_t)(base + c) * a.H + hidx;
            const float w = __expf(a.part_ml[it * 2] - M);
            L = __builtin_fmaf(a.part_ml[it * 2 + 1], w, L);
            O = __builtin_fmaf(a.part_o[it * HD + oi % HD], w, O);
        }
        a.out[((size_t)s * a.H + hidx) * HD + oi % HD] = O / L;
    }
    if (tid == 0) a.counters[(size_t)s * a.Hkv + kvh] = 0u;  // ready for the next launch
}

template <typename KT>
static int launch_attn_t(const AttnArgs& a, int hd, int G, int grid_x, hipStream_t st) {
    dim3 grid(grid_x, a.Hkv);
#define QH_ATTN(HDv, Gv)                                                                   \
    if (hd == HDv && G == Gv) {                                                            \
        hipLaunchKernelGGL((attn_decode_kernel<KT, HDv, Gv>), grid, dim3(ACH), 0, st, a); \
        QH_CHECK_HIP(hipGetLastError());                                                   \
        return QRAF_HIP_OK;                                                                \
    }
    QH_ATTN(128, 1) QH_ATTN(128, 2) QH_ATTN(128, 3) QH_ATTN(128, 4) QH_ATTN(128, 6) QH_ATTN(128, 8)
    QH_ATTN(128, 12) QH_ATTN(128, 16) QH_ATTN(64, 1) QH_ATTN(64, 2) QH_ATTN(64, 3) QH_ATTN(64, 4) QH_ATTN(64, 6)
    QH_ATTN(64, 8) QH_ATTN(64, 12) QH_ATTN(64, 16) QH_ATTN(32, 1) QH_ATTN(32, 2) QH_ATTN(32, 4) QH_ATTN(32, 8)
    QH_ATTN(16, 1) QH_ATTN(16, 2) QH_ATTN(16, 4) QH_ATTN(16, 8)
#undef QH_ATTN
    return set_error(QRAF_HIP_ERR_INVALID, "attention: unsupported head_dim %d / group %d", hd, G);
}

size_t attn_workspace_bytes(int n, int H, int Hkv, int hd, int max_ctx) {
    const size_t items = (size_t)n * ((max_ctx + ACH - 1) / ACH);
    return items * H * hd * 4 + items * H * 2 * 4 + (size_t)n * Hkv * 4 + 256;
}

int launch_attention(const float* q, const void* kc, const void* vc, uint32_t kv_dtype, const int32_t* page_table,
                     int max_pages, const int32_t* ctx, int n, int H, int Hkv, int hd, int page_size, float scale,
                     int max_ctx, float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    QH_REQUIRE(q && kc && vc && page_table && ctx && out && ws, QRAF_HIP_ERR_INVALID, "attention: null pointer");
    QH_REQUIRE(n > 0 && n <= 1024, QRAF_HIP_ERR_INVALID, "attention: batch %d outside 1..1024", n);
    QH_REQUIRE(Hkv > 0 && H % Hkv == 0, QRAF_HIP_ERR_INVALID, "attention: %d heads not a multiple of %d kv heads", H, Hkv);
    QH_REQUIRE(page_size > 0 && max_pages > 0 && max_ctx > 0 && max_ctx <= max_pages * page_size, QRAF_HIP_ERR_INVALID,
               "attention: bad page geometry");
    QH_REQUIRE(kv_dtype == DT_F32 || kv_dtype == DT_F16, QRAF_HIP_ERR_DTYPE, "attention: KV dtype %u", kv_dtype);
    QH_REQUIRE(ws_bytes >= attn_workspace_bytes(n, H, Hkv, hd, max_ctx), QRAF_HIP_ERR_INVALID,
               "attention: workspace too small");
    const int items = n * ((max_ctx + ACH - 1) / ACH);
    AttnArgs a;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.page_table = page_table;
    a.ctx = ctx;
    a.out = out;
    uint8_t* w = (uint8_t*)ws;
    a.counters = (uint32_t*)w;  // zeroed by the caller once; kernels leave them zero
    w += ((size_t)n * Hkv * 4 + 255) / 256 * 256;
    a.part_ml = (float*)w;
    w += (size_t)items * H * 2 * 4;
    a.part_o = (float*)w;
    a.n = n;
    a.H = H;
    a.Hkv = Hkv;
    a.page_size = page_size;
    a.max_pages = max_pages;
    a.max_ctx = max_ctx;
    a.scale = scale;
    const int G = H / Hkv;
    if (kv_dtype == DT_F32) return launch_attn_t<float>(a, hd, G, items, st);
    return launch_attn_t<_Float16>(a, hd, G, items, st);
}

// ----------------------------------------------------------------------------
// Per-token post-processing of the fused QKV projection (attention.cpp:100-119):
// bias add (F32 biases only, transformer.cpp:45-50), interleaved-pair RoPE on
// every q and k head (ops.cpp:158-177), and the store of k, v at the token's
// position into the paged cache.  One workgroup per sequence.
// ----------------------------------------------------------------------------
template <typename KT>
__global__ void rope_append_kernel(const float* __restrict__ qkv, const float* __restrict__ bias, int H, int Hkv,
                                   int hd, const int32_t* __restrict__ pos, const float* __restrict__ rope,
                                   float* __restrict__ q_out, KT* __restrict__ kc, KT* __restrict__ vc,
                                   const int32_t* __restrict__ page_table, int max_pages, int page_size) {
    const int s = blockIdx.x;
    const int qd = H * hd, kvd = Hkv * hd, row = qd + 2 * kvd;
    const float* src = qkv + (size_t)s * row;
    const int p = pos[s];
    const int page = page_table[(size_t)s * max_pages + p / page_size], off = p % page_size;
    const float* cs = rope + (size_t)p * hd;  // (cos, sin) of pair i/2 at [i], [i+1]
    // pairs (i, i+1) of q heads, then k heads: rotate; v: copy.  Products are
    // rounded separately (no FMA contraction), as the reference's scalar code.
    for (int e = threadIdx.x; e < (qd + kvd) / 2 + kvd; e += blockDim.x) {
        if (e < (qd + kvd) / 2) {
            const int i0 = 2 * e;  // element index in [0, qd + kvd)
            const int i = i0 % hd;   // even index inside the head
            float a = src[i0], b = src[i0 + 1];
            if (bias) {
                a = __fadd_rn(a, bias[i0]);
                b = __fadd_rn(b, bias[i0 + 1]);
            }
            const float c = cs[i], sn = cs[i + 1];
            const float ra = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, sn));
            const float rb = __fadd_rn(__fmul_rn(a, sn), __fmul_rn(b, c));
            if (i0 < qd) {
                q_out[(size_t)s * qd + i0] = ra;
                q_out[(size_t)s * qd + i0 + 1] = rb;
            } else {
                const int kh = (i0 - qd) / hd;
                KT* dst = kc + (((size_t)page * Hkv + kh) * page_size + off) * hd + i;
                dst[0] = (KT)ra;
                dst[1] = (KT)rb;
            }
        } else {
            const int j = e - (qd + kvd) / 2;  // v element
            float v = src[qd + kvd + j];
            if (bias) v = __fadd_rn(v, bias[qd + kvd + j]);
            const int vh = j / hd;
            vc[(((size_t)page * Hkv + vh) * page_size + off) * hd + j % hd] = (KT)v;
        }
    }
}

int launch_rope_append(const float* qkv, const float* bias, int n, int H, int Hkv, int hd, const int32_t* pos,
                       const float* rope, float* q_out, void* kc, void* vc, uint32_t kv_dtype,
                       const int32_t* page_table, int max_pages, int page_size, hipStream_t st) {
    QH_REQUIRE(qkv && pos && rope && q_out && kc && vc && page_table && n > 0 && hd % 2 == 0, QRAF_HIP_ERR_INVALID,
               "rope_append: bad arguments");
    if (kv_dtype == DT_F32)
        hipLaunchKernelGGL(rope_append_kernel<float>, dim3(n), dim3(256), 0, st, qkv, bias, H, Hkv, hd, pos, rope,
                           q_out, (float*)kc, (float*)vc, page_table, max_pages, page_size);
    else if (kv_dtype == DT_F16)
        hipLaunchKernelGGL(rope_append_kernel<_Float16>, dim3(n), dim3(256), 0, st, qkv, bias, H, Hkv, hd, pos, rope,
                           q_out, (_Float16*)kc, (_Float16*)vc, page_table, max_pages, page_size);
    else
        return set_error(QRAF_HIP_ERR_DTYPE, "rope_append: KV dtype %u", kv_dtype);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip

extern "C" {

uint64_t qraf_hip_attention_workspace_bytes(int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                            int32_t max_ctx) {
    return qraf_hip::attn_workspace_bytes(n_seqs, n_heads, n_kv_heads, head_dim, max_ctx);
}

int qraf_hip_paged_attention_dev(const float* q, const void* k_cache, const void* v_cache, uint32_t kv_dtype,
                                 const int32_t* page_table, int32_t max_pages_per_seq, const int32_t* ctx_lens,
                                 int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                 int32_t page_size, float scale, int32_t max_ctx, float* out, void* workspace,
                                 uint64_t workspace_bytes, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_attention(q, k_cache, v_cache, kv_dtype, page_table, max_pages_per_seq, ctx_lens, n_seqs,
                                      n_heads, n_kv_heads, head_dim, page_size, scale, max_ctx, out, workspace,
                                      workspace_bytes, qraf_hip::as_stream(stream));
}

// RopeCache::init (ops.cpp:179-193) on the host, with the host libm the
// reference uses: entry [pos][i], [pos][i+1] = cos, sin(pos / theta^(i/hd))
// for even i, so the device rotation reads the reference's exact values.
int qraf_hip_rope_table_host(int32_t max_pos, int32_t head_dim, float rope_theta, float* table) {
    qraf_hip::clear_error();
    QH_REQUIRE(max_pos > 0 && head_dim > 0 && head_dim % 2 == 0 && table, QRAF_HIP_ERR_INVALID,
               "rope table: bad arguments");
    for (int i = 0; i < head_dim; i += 2) {
        const float freq = 1.0f / powf(rope_theta, (float)i / (float)head_dim);  // ops.cpp:160
        for (int p = 0; p < max_pos; p++) {
            const float val = (float)p * freq;
            table[(size_t)p * head_dim + i] = cosf(val);
            table[(size_t)p * head_dim + i + 1] = sinf(val);
        }
    }
    return QRAF_HIP_OK;
}

int qraf_hip_rope_append_dev(const float* qkv, const float* bias, int32_t n_seqs, int32_t n_heads,
                             int32_t n_kv_heads, int32_t head_dim, const int32_t* positions, const float* rope_table,
                             float* q_out, void* k_cache, void* v_cache, uint32_t kv_dtype, const int32_t* page_table,
                             int32_t max_pages_per_seq, int32_t page_size, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_rope_append(qkv, bias, n_seqs, n_heads, n_kv_heads, head_dim, positions, rope_table, q_out,
                                        k_cache, v_cache, kv_dtype, page_table, max_pages_per_seq, page_size,
                                        qraf_hip::as_stream(stream));
}

}  // extern "C"
