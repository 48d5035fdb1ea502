// attention.hip -- ragged decode attention over a block-paged KV cache.
//
// Replaces the per-head score / softmax / weighted-sum loops of
// attention_forward (reference attention.cpp:122-150) and the KVCache store
// (attention.cpp:39-44, :119), for a batch of sequences that each add one
// token.  KV layout in HBM, per layer (a page holds page_size positions):
//     K     : [num_pages][Hkv][page_size][head_dim]   (f32 or f16)
//     V f32 : [num_pages][Hkv][page_size][head_dim]
//     V f16 : [num_pages][Hkv][head_dim][page_size]   (dimension-major in a page)
//     int8  : [num_pages][Hkv] blocks of page_size * (head_dim + 4) bytes,
//             K block = int8 [page_size][head_dim] then f32 scale [page_size]
//             V block = int8 [head_dim][page_size] then f32 scale [page_size]
// and a page table per sequence maps logical page j (positions
// j*page_size .. +page_size-1) to a physical page.  fp16 V is stored
// dimension-major so that the matrix-core kernel's V operand (consecutive
// positions of one dimension) is a contiguous load.
//
// Work decomposition, chunk grid: the context of every sequence is cut into
// chunks of CH = 256 positions; one workgroup handles one (sequence, chunk)
// item for one KV head and all H/Hkv query heads that share it (GQA).  The
// grid has ceil(max_ctx / CH) items per sequence (item = s * that + chunk);
// a workgroup whose chunk starts at or past its sequence's device-resident
// context length exits at once, so the lengths can change on the device
// between launches with no host round trip.  Sequences with several chunks
// write (max, sum, unnormalised output) partials, which attn_merge_kernel (a
// second launch, one wave per sequence and query head) combines in chunk
// order.  Balanced split (the default for the matrix-core kernels, described
// at attn_split_kernel): the batch's 64-position tiles are divided into
// equal shares, one per resident workgroup, computed on the device from the
// same device-resident lengths; a sequence split across shares is merged in
// share order.
//
// int8 pages hold the scheme of QuantizedKVCache (kv_cache_quant.h:61-128):
// per (position, KV head) scale = absmax / 127 and q = clamp(round(x / scale),
// +-127); a score is (sum_d q_k[d] * query[d]) * k_scale * 1/sqrt(hd) and a
// value element q_v[d] * v_scale.
//
// The matrix-core kernels, attn_mfma_kernel (chunk grid) and
// attn_split_kernel (balanced split), take f32, fp16 or int8 pages, head_dim
// 64 or 128, up to 16 query heads per KV head and a power-of-two page_size
// (pages addressed by shifts).  fp16 and int8 pages run q.K^T and P.V on
// v_mfma_f32_16x16x32_f16: K and V enter as stored (fp16, or int8 widened to
// fp16, both exact), q and the probabilities as fp16 hi + lo pairs (q scaled
// per head by a power of two so hi + lo carries 22 bits of it), products
// accumulate in fp32.  int8 scales are applied in fp32: a K scale to each
// position's score, a V scale folded into that position's probability
// before the P.V product.  f32 pages run on v_mfma_f32_16x16x4_f32 with
// every operand in fp32 as it is.  attn_decode_kernel (the other shapes, and
// f32 / fp16 pages on request) is plain fp32 VALU code on the chunk grid:
// scores with thread = position, output with thread = (head, dimension).
#include <math.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

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
    float* out;                // [n][H][HD] f32, or (out_hi != null) the bf16 split planes below
    uint16_t* out_hi;          // [n][H][HD] hi plane of qraf_hip_split_bf16_dev form
    uint16_t* out_lo;          // [n][H][HD] lo plane
    float* part_o;             // [items][H][HD]   (multi-chunk partials)
    float* part_ml;            // [items][H][2]
    uint32_t* counters;        // [n][Hkv]          (reserved)
    int32_t* pref;             // [n + 1] tile prefix of the split kernel, for its merge
    int n, H, Hkv, page_size, max_pages, max_ctx;
    float scale;
    int gx;                    // split kernel: workgroups per KV head
    int ps_log2;               // matrix-core kernels: page_size = 1 << ps_log2
};

// final output element: f32, or split into the two planes a GEMM consumes
__device__ __forceinline__ void attn_store(const AttnArgs& a, size_t i, float v) {
    if (a.out_hi) split_bf16(v, &a.out_hi[i], &a.out_lo[i]);
    else a.out[i] = v;
}

// Item -> (sequence, chunk): item = s * chunks_per_seq + chunk.  Returns
// false when the chunk starts at or past the sequence's context.
__device__ __forceinline__ bool attn_item(const AttnArgs& a, int& s, int& chunk, int& nchunks, int& ctx) {
    const int per = (a.max_ctx + ACH - 1) / ACH;
    s = blockIdx.x / per;
    chunk = blockIdx.x - s * per;
    ctx = min(a.ctx[s], a.max_ctx);
    nchunks = (ctx + ACH - 1) / ACH;
    return chunk < nchunks;
}

template <typename KT, int HD, int G>
__global__ __launch_bounds__(ACH) void attn_decode_kernel(AttnArgs a) {
    static_assert(HD % 8 == 0, "head_dim must be a multiple of 8");
    constexpr int NOUT = G * HD;                 // outputs of this workgroup
    constexpr int HPT = (NOUT + ACH - 1) / ACH;  // outputs per thread at the end
    constexpr int NG = ACH / HD;                 // position groups of the PV phase
    constexpr int PVU = 16;                      // V loads in flight per thread in the PV phase
    constexpr int PADP = PVU * NG;               // past-the-end slots its unrolled loop may touch
    static_assert(PADP <= ACH, "padding is written by the first PADP threads");
    constexpr int QPT = (G * HD + ACH - 1) / ACH;  // q elements per thread
    __shared__ __align__(16) float s_qf[QPT * ACH];  // q of the G heads, [G][HD], padded to whole rounds
    float (*s_q)[HD] = (float (*)[HD])s_qf;
    __shared__ float s_p[G][ACH + PADP];         // probabilities (zero past the end); then PV partials
    __shared__ uint32_t s_voff[ACH + PADP];      // element offset of each position's V row in the layer pages
    __shared__ float s_red[G][4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.y;
    const int item = blockIdx.x;
    // Requested together, before any of them is used: the context length, q
    // of the G heads, and the page id of this thread's position (its table
    // index clamped into the table; used only for positions inside the
    // context).  Then the K row of the position, and after one barrier the
    // first round of V loads of the PV phase, both in flight while the scores
    // and the softmax are formed.
    const int per = (a.max_ctx + ACH - 1) / ACH;
    const int s = item / per, chunk = item - s * per;
    const int t0 = chunk * ACH;
    const int t = t0 + tid;
    // (q's loads are in flight with the page id's: the K row is requested
    // after one round trip.)
    const int ctx_raw = a.ctx[s];
    const int page_t = a.page_table[(size_t)s * a.max_pages + min(t, a.max_ctx - 1) / a.page_size];
    float qv[QPT];
#pragma unroll
    for (int k = 0; k < QPT; k++) qv[k] = a.q[((size_t)s * a.H + kvh * G) * HD + min(tid + ACH * k, G * HD - 1)];
    const int ctx = min(ctx_raw, a.max_ctx);
    const int nchunks = (ctx + ACH - 1) / ACH;

    const KT* kc = (const KT*)a.kc;
    const KT* vc = (const KT*)a.vc;
    // every thread's V row offset from its page id (positions past the
    // context are given position t0's below), so the page id is waited for
    // once, before the branch, in parallel with the context length
    {
        const uint32_t row = ((uint32_t)page_t * a.Hkv + kvh) * a.page_size;
        s_voff[tid] = sizeof(KT) == 4 ? (row + t % a.page_size) * HD : row * HD + t % a.page_size;
    }
#pragma unroll
    for (int k = 0; k < QPT; k++) s_qf[tid + ACH * k] = qv[k];  // unconditional: the loads stay ahead of the branch
    float kv[HD];
    if (t < ctx) {
        const KT* kr = kc + (((size_t)page_t * a.Hkv + kvh) * a.page_size + t % a.page_size) * HD;
#pragma unroll
        for (int d = 0; d < HD; d += 8) {
            float k8[8];
            load8(kr + d, k8);
#pragma unroll
            for (int i = 0; i < 8; i++) kv[d + i] = k8[i];
        }
    }
    __syncthreads();
    if (chunk >= nchunks) return;  // the whole workgroup (no position of its chunk was loaded)
    // V row offsets of positions past the end (and of the padding the PV
    // loop may touch): position t0's row, which exists; its probability is 0
    if (t >= ctx) s_voff[tid] = s_voff[0];
    if (tid < PADP) s_voff[ACH + tid] = s_voff[0];
    __syncthreads();

    const int dd = tid % HD, grp = tid / HD;
    const int tend = min(ACH, ctx - t0);
    const KT* vd = vc + (sizeof(KT) == 4 ? (size_t)dd : (size_t)dd * a.page_size);
    float vpre[PVU];  // the PV loop's first round, requested before the scores
#pragma unroll
    for (int u = 0; u < PVU; u++) vpre[u] = kv_load(vd + s_voff[grp + NG * u]);

    // ---- scores: thread = position t0 + tid
    float sc[G];
#pragma unroll
    for (int h = 0; h < G; h++) sc[h] = 0.f;
    if (t < ctx) {
#pragma unroll
        for (int d = 0; d < HD; d += 8) {
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float4 qa = *(const float4*)&s_q[h][d], qb = *(const float4*)&s_q[h][d + 4];
                sc[h] = __builtin_fmaf(qa.x, kv[d + 0], sc[h]);
                sc[h] = __builtin_fmaf(qa.y, kv[d + 1], sc[h]);
                sc[h] = __builtin_fmaf(qa.z, kv[d + 2], sc[h]);
                sc[h] = __builtin_fmaf(qa.w, kv[d + 3], sc[h]);
                sc[h] = __builtin_fmaf(qb.x, kv[d + 4], sc[h]);
                sc[h] = __builtin_fmaf(qb.y, kv[d + 5], sc[h]);
                sc[h] = __builtin_fmaf(qb.z, kv[d + 6], sc[h]);
                sc[h] = __builtin_fmaf(qb.w, kv[d + 7], sc[h]);
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
        if (tid < PADP) s_p[h][ACH + tid] = 0.f;
        float v = p;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0) s_red[h][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; h++) l[h] = (s_red[h][0] + s_red[h][1]) + (s_red[h][2] + s_red[h][3]);

    // ---- weighted sum of V.  Thread (dimension d = tid % HD, group g = tid /
    // HD) sums positions g, g + NG, ... of the chunk for all G heads at once
    // (each V element is loaded once for the heads that share it), with PVU
    // independent loads in flight; the NG group sums are then added in group
    // order.  For f32 pages and head_dim >= 64 a wave reads one V row.
    float acc[G];
#pragma unroll
    for (int h = 0; h < G; h++) acc[h] = 0.f;
#pragma unroll
    for (int u = 0; u < PVU; u++)  // the first round (grp < tend always: tend >= 1, grp < NG <= PVU * NG)
#pragma unroll
        for (int h = 0; h < G; h++) acc[h] = __builtin_fmaf(s_p[h][grp + NG * u], vpre[u], acc[h]);
    for (int tt = grp + NG * PVU; tt < tend; tt += NG * PVU) {
        float v[PVU];
#pragma unroll
        for (int u = 0; u < PVU; u++) v[u] = kv_load(vd + s_voff[tt + NG * u]);
#pragma unroll
        for (int u = 0; u < PVU; u++)
#pragma unroll
            for (int h = 0; h < G; h++) acc[h] = __builtin_fmaf(s_p[h][tt + NG * u], v[u], acc[h]);
    }
    __syncthreads();  // every probability read: s_p now holds the group partials [NG][G][HD]
    float* s_acc = &s_p[0][0];
#pragma unroll
    for (int h = 0; h < G; h++) s_acc[(grp * G + h) * HD + dd] = acc[h];
    __syncthreads();
    float o[HPT];
#pragma unroll
    for (int j = 0; j < HPT; j++) {
        const int oi = tid + ACH * j;
        float sum = 0.f;
        if (oi < NOUT) {
            const int h = oi / HD, d = oi % HD;
#pragma unroll
            for (int g = 0; g < NG; g++) sum += s_acc[(g * G + h) * HD + d];
        }
        o[j] = sum;
    }

    if (nchunks == 1) {
#pragma unroll
        for (int j = 0; j < HPT; j++) {
            const int oi = tid + ACH * j;
            if (oi < NOUT) attn_store(a, ((size_t)s * a.H + kvh * G) * HD + oi, o[j] / l[oi / HD]);
        }
        return;
    }

    // ---- multi-chunk: publish (max, sum, unnormalised output) for attn_merge_kernel
#pragma unroll
    for (int j = 0; j < HPT; j++) {
        const int oi = tid + ACH * j;
        if (oi < NOUT) a.part_o[((size_t)item * a.H + kvh * G) * HD + oi] = o[j];
    }
    if (tid < G) {
        a.part_ml[((size_t)item * a.H + kvh * G + tid) * 2 + 0] = m[tid];
        a.part_ml[((size_t)item * a.H + kvh * G + tid) * 2 + 1] = l[tid];
    }
}

// ---------------------------------------------------------------------------
// Matrix-core decode attention for fp16 pages (see the file comment).  One
// workgroup = one (sequence, ACH-position chunk, KV head); wave w takes the
// chunk's positions 64w .. 64w+63 as four 16-position tiles.
//
// q.K^T, per tile: A = K (lane: position l%16, 8 dimensions), B = q^T (lane:
// head l%16, the same 8 dimensions), D[position][head]; heads >= G are zero
// columns.  P.V, per 32 positions: A = P (lane: head l%16, 8 positions),
// B = V (lane: dimension l%16, the same 8 positions, contiguous in a
// dimension-major page), D[head][dimension].  Lane (l%16, s = l/16) holds
// positions 4s..4s+3 of every score tile, so its P operand for tiles 2b, 2b+1
// is positions {4s..4s+3} and {16+4s..16+4s+3}, and its V operand is the same
// two 4-position runs.  Positions at or past ctx get score -inf (p = 0) and
// their V values are zeroed, so page contents past ctx never matter.
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4a __attribute__((ext_vector_type(4)));

// page types of the matrix-core kernels
enum : int { KV_F16 = 0, KV_I8 = 1, KV_F32 = 2 };

// f32 pages (KV_F32) run q.K^T and P.V on v_mfma_f32_16x16x4_f32: K, V, q
// and the probabilities enter as they are (fp32 products, fp32 sums), so no
// split or range scaling is involved.  The tile decomposition is the fp16
// one, with k = 4 per instruction:
//   q.K^T k-step 4c+e: lane (l%16, s = l/16) gives K[position l%16][dim
//     16c + 4s + e] and q[head l%16][same dim]; a lane's K operands of one
//     tile are HD/16 float4 loads (the 4 lane groups read 64 contiguous
//     bytes of each row per load);
//   P.V k-step (tile t, r): lane gives P[head l%16][position 16t + 4s + r]
//     (its own score register sc[t][r]) and V[that position][dim
//     dvf(l%16, d)] for output tile d, dvf(j, d) = 4j + 64(d/4) + d%4, so a
//     lane's V operands of one position are HD/64 float4 loads (16 lanes
//     read 256 contiguous bytes of the row).
// Output tile d, register r of lane (j, s) is O[head 4s + r][dvf(j, d)].
__device__ __forceinline__ constexpr int dvf(int j, int d) { return 4 * j + 64 * (d >> 2) + (d & 3); }

// Start of the (page pg, KV head kvh) block of a K or V pool whose blocks are
// block_bytes long.  Loads add 32-bit byte offsets inside the block (a block
// is at most page_size * (head_dim + 4) * 4 bytes): with a wave-uniform page
// id the base lives in scalar registers and each load needs no 64-bit
// address arithmetic per lane.
__device__ __forceinline__ const char* page_block(const void* pool, int pg, int Hkv, int kvh, size_t block_bytes) {
    return (const char*)pool + ((size_t)pg * Hkv + kvh) * block_bytes;
}
// A page id read from the table: UPG (page_size >= 16) makes it wave-uniform.
// Each id a lane reads is that of a 16-aligned group of 16 positions (K rows
// pw + 16t + l16) or of 4-position runs inside one (V runs pw + 16t + 4s), each
// clamped into the context; with pages of 16 or more positions the whole
// group lies in one page, so every lane of the wave reads the same id.
template <bool UPG>
__device__ __forceinline__ int page_id(const int32_t* ptab, int idx) {
    const int v = ptab[idx];
    return UPG ? __builtin_amdgcn_readfirstlane(v) : v;
}

// K operands of one f32 score tile: position pc of page pg, the lane group's dims
template <int HD>
__device__ __forceinline__ void kload_f32(const AttnArgs& a, int pg, int kvh, int row, int seg,
                                          float4 (&kb)[HD / 16]) {
    const char* kp = page_block(a.kc, pg, a.Hkv, kvh, (size_t)a.page_size * HD * 4);
    const uint32_t o = (uint32_t)(row * HD + 4 * seg) * 4u;
#pragma unroll
    for (int c = 0; c < HD / 16; c++) kb[c] = *(const float4*)(kp + (o + 64u * c));
}

// V operands of one f32 P.V tile: 4 positions (rows r0 .. of page pg, each
// clamped by the caller) x the lane's HD/16 dims
template <int HD>
__device__ __forceinline__ void vload_f32(const AttnArgs& a, int pg, int kvh, const int (&rows)[4], int l16,
                                          float4 (&vb)[4][HD / 64]) {
    const char* vp = page_block(a.vc, pg, a.Hkv, kvh, (size_t)a.page_size * HD * 4);
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int i = 0; i < HD / 64; i++)
            vb[r][i] = *(const float4*)(vp + (uint32_t)(rows[r] * HD + 4 * l16 + 64 * i) * 4u);
}

// one f32 score tile: sc += K . q^T over all HD dims (q from LDS, row stride HD + 4)
template <int HD>
__device__ __forceinline__ void score_f32(const float* s_qrow, int seg, const float4 (&kb)[HD / 16], f32x4a& sc) {
#pragma unroll
    for (int c = 0; c < HD / 16; c++) {
        const float4 qf = *(const float4*)(s_qrow + 16 * c + 4 * seg);
        sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kb[c].x, qf.x, sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kb[c].y, qf.y, sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kb[c].z, qf.z, sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kb[c].w, qf.w, sc, 0, 0, 0);
    }
}

// one f32 P.V tile: o[d] += P[., 16t + 4s + r] V[16t + 4s + r, dvf(., d)], r = 0..3
template <int HD>
__device__ __forceinline__ void pv_f32(const f32x4a& p, const float4 (&vb)[4][HD / 64], f32x4a (&o)[HD / 16]) {
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int d = 0; d < HD / 16; d++) {
            const float4 v = vb[r][d >> 2];
            const float x = (d & 3) == 0 ? v.x : (d & 3) == 1 ? v.y : (d & 3) == 2 ? v.z : v.w;
            o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], x, o[d], 0, 0, 0);
        }
}

// f32 page rows of a lane's V operands for tile t of the 64 positions from
// pw: positions pw + 16t + 4s + r, each clamped to ctx - 1.  The 4-position
// group starts at a = min(pw + 16t + 4s, vlast), vlast = (ctx - 1) & ~3, so
// every clamped row lies in a's page (page_size % 4 == 0).
__device__ __forceinline__ void vrows_f32(int pw, int t, int seg, int ctx, int vlast, int psm, int (&rows)[4]) {
    const int pa = min(pw + 16 * t + 4 * seg, vlast);
#pragma unroll
    for (int r = 0; r < 4; r++) rows[r] = min(pa + r, ctx - 1) & psm;
}

// zero the fp16 lanes of a 4-position run (2 dwords) at or past ctx
__device__ __forceinline__ uint2 mask_run(uint2 v, int pos0, int ctx) {
    const int k = ctx - pos0;  // valid positions in the run (selects, no branches)
    const uint32_t mx = k >= 2 ? 0xFFFFFFFFu : (k == 1 ? 0xFFFFu : 0u);
    const uint32_t my = k >= 4 ? 0xFFFFFFFFu : (k == 3 ? 0xFFFFu : 0u);
    return make_uint2(v.x & mx, v.y & my);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// 4 int8 (one dword, byte i = element i) -> 4 fp16, exactly: the biased byte
// u = q + 128 goes under the exponent of 1024 (fp16 bits 0x6400 | u encode
// 1024 + u, spacing 1 in [1024, 2048)), then 1152 = 1024 + 128 is subtracted
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // 0x64,u1,0x64,u0
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // 0x64,u3,0x64,u2
    const f16x2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const f16x2 a = __builtin_bit_cast(f16x2, lo) - off, b = __builtin_bit_cast(f16x2, hi) - off;
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}
__device__ __forceinline__ f16x8 i8x8_to_f16x8(uint32_t w0, uint32_t w1) {
    const uint2 a = i8x4_to_f16x4(w0), b = i8x4_to_f16x4(w1);
    return __builtin_bit_cast(f16x8, make_uint4(a.x, a.y, b.x, b.y));
}

// 4 workgroups per CU (at most 128 VGPRs): the K and V loads of one wave
// already cover its own latency, more resident workgroups cover the
// prologue and epilogue of the others
template <int HD, int KV, bool UPG>
__global__ __launch_bounds__(ACH, 4) void attn_mfma_kernel(AttnArgs a, int G) {
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    constexpr bool I8 = KV == KV_I8, F32 = KV == KV_F32;
    constexpr int KK = HD / 32;  // MFMA k-steps per score tile
    // q.K^T k-step kk, lane group s = l/16 covers 8 dimensions starting at
    // kdim(kk, s).  fp16: 8*(4kk+s), so the 4 groups of one step read 64
    // consecutive bytes of a K row; int8: 8*(KK*s+kk), so each lane reads
    // its 8*KK bytes of the row at once (one or two 16-byte loads)
    auto kdim = [](int kk, int sg) { return I8 ? 8 * (KK * sg + kk) : 8 * (4 * kk + sg); };
    constexpr int DT = HD / 16;  // 16-dimension output tiles
    typedef typename std::conditional<I8, uint32_t, uint2>::type VRun;  // one 4-position V run
    constexpr int QS = HD + 8;   // q plane row stride (fp16): 16-byte reads of 16 rows hit distinct banks
    // q: fp16 hi/lo planes [2][16][QS], or (f32 pages) f32 rows [16][HD + 4]
    __shared__ __align__(16) float s_qbuf[16 * QS];
    _Float16(*s_q)[16][QS] = (_Float16(*)[16][QS])s_qbuf;
    float(*s_qf)[HD + 4] = (float(*)[HD + 4])s_qbuf;
    __shared__ float s_qs[16];
    __shared__ float s_m[4][16], s_l[4][16];
    __shared__ __align__(16) float s_kvs[2][4][64];  // int8: K, V scale of position pw + lane, per wave
    extern __shared__ __align__(16) float s_odyn[];  // [4][G][HD]: the waves' partial outputs
    float(*s_o)[HD] = (float(*)[HD])s_odyn;  // s_o[wave * G + head][dim]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, seg = lane >> 4;
    const int kvh = blockIdx.y;
    const int item = blockIdx.x;
    int s, chunk, nchunks;
    int ctx;
    if (!attn_item(a, s, chunk, nchunks, ctx)) return;
    const int ps = a.page_size, psl = a.ps_log2, psm = ps - 1;  // page_size is a power of two here
    const int32_t* ptab = a.page_table + (size_t)s * a.max_pages;
    const int pw = chunk * ACH + 64 * wave;  // first position of this wave
    const bool active = pw < ctx;            // wave-uniform

    // Every global read that does not depend on another is requested before
    // the first wait: q of the G heads with the page ids; for int8 pages then
    // (page ids known) the K rows, V runs and scales before q is staged, so
    // the staging and its barrier overlap those loads.
    constexpr int PER = HD / 64;
    float qv[4][PER];  // q of head wave + 4j, dimensions lane + 64i
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int h = wave + 4 * j;
#pragma unroll
        for (int i = 0; i < PER; i++)
            qv[j][i] = h < G ? a.q[((size_t)s * a.H + kvh * G + h) * HD + lane + 64 * i] : 0.f;
    }

    // ---- page ids of every K row and V run this lane reads (clamped into
    // the context, so every read is inside the page table)
    int kpg[4], vpg[4];
#pragma unroll
    for (int t = 0; t < 4; t++) kpg[t] = page_id<UPG>(ptab, min(pw + 16 * t + l16, ctx - 1) >> psl);
    const int vlast = (ctx - 1) & ~3;
#pragma unroll
    for (int j = 0; j < 4; j++) vpg[j] = page_id<UPG>(ptab, min(pw + 16 * j + 4 * seg, vlast) >> psl);
    // int8: lane l loads the K and V scales of position pw + l (clamped like
    // its K row, whose page is kpg[l / 16]) and stores them to LDS before the
    // staging barrier; a score's or probability's lane reads its 4-position
    // run back as a float4.  (Not by shuffle: the compiler may move a shuffle
    // whose result feeds a select into the branch of the select, where a
    // source lane outside the branch reads as 0.)
    const size_t blk = (size_t)ps * (HD + 4);  // int8 bytes of one (page, KV head) block
    float ks_own = 0.f, vs_own = 0.f;
    if (I8 && active) {
        const int pg = seg == 0 ? kpg[0] : seg == 1 ? kpg[1] : seg == 2 ? kpg[2] : kpg[3];
        const size_t b = ((size_t)pg * a.Hkv + kvh) * blk + (size_t)ps * HD + 4 * (min(pw + lane, ctx - 1) & psm);
        ks_own = *(const float*)((const int8_t*)a.kc + b);
        vs_own = *(const float*)((const int8_t*)a.vc + b);
    }

    // ---- K rows of the wave's 4 score tiles: lane row pw + 16t + l16
    // (clamped: past-ctx scores are masked later), the lane's 8*KK dimensions
    const _Float16* kc = (const _Float16*)a.kc;
    const _Float16* vc = (const _Float16*)a.vc;
    typedef typename std::conditional<I8, uint4[KK / 2], f16x8[KK]>::type KRow;
    KRow kreg[4];
    auto kload = [&]() {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int pc = min(pw + 16 * t + l16, ctx - 1);
            if constexpr (I8) {
                const char* kb = page_block(a.kc, kpg[t], a.Hkv, kvh, blk);
                const uint32_t o = (uint32_t)((pc & psm) * HD + 8 * KK * seg);
#pragma unroll
                for (int i = 0; i < KK / 2; i++) kreg[t][i] = *(const uint4*)(kb + (o + 16u * i));
            } else {
                const char* kb = page_block(kc, kpg[t], a.Hkv, kvh, (size_t)ps * HD * 2);
                const uint32_t o = (uint32_t)((pc & psm) * HD + 8 * seg) * 2u;
#pragma unroll
                for (int kk = 0; kk < KK; kk++) kreg[t][kk] = *(const f16x8*)(kb + (o + 64u * kk));
            }
        }
    };
    // int8 rows (half the registers) are requested here; fp16 ones after the
    // staging barrier (holding them across it would spill)
    if (I8 && active) kload();

    // ---- V of the wave's 64 positions: int8 runs are requested here, with
    // the K rows; fp16 ones (twice the registers) after the score tiles,
    // still before the softmax.  Per lane and 32-position step b: two
    // 4-position runs (b*32 + 4seg and +16) per 16-dimension tile, clamped
    // into the context (fp16 values past it are masked; int8 ones are finite
    // and meet a zero probability), 4-aligned so a run never leaves a page.
    VRun va0[DT], vb0[DT], va1[DT], vb1[DT];
    auto vload = [&](int b, VRun (&ra)[DT], VRun (&rb)[DT]) {
        const int pac = min(pw + 32 * b + 4 * seg, vlast), pbc = min(pw + 32 * b + 16 + 4 * seg, vlast);
        if constexpr (I8) {
            const char* va = page_block(a.vc, vpg[2 * b], a.Hkv, kvh, blk);
            const char* vb = page_block(a.vc, vpg[2 * b + 1], a.Hkv, kvh, blk);
#pragma unroll
            for (int d = 0; d < DT; d++) {
                const int dim = 16 * d + l16;
                ra[d] = *(const uint32_t*)(va + (uint32_t)((pac & psm) + dim * ps));
                rb[d] = *(const uint32_t*)(vb + (uint32_t)((pbc & psm) + dim * ps));
            }
        } else {
            const char* va = page_block(vc, vpg[2 * b], a.Hkv, kvh, (size_t)HD * ps * 2);
            const char* vb = page_block(vc, vpg[2 * b + 1], a.Hkv, kvh, (size_t)HD * ps * 2);
#pragma unroll
            for (int d = 0; d < DT; d++) {
                const int dim = 16 * d + l16;
                ra[d] = *(const uint2*)(va + (uint32_t)((pac & psm) + dim * ps) * 2u);
                rb[d] = *(const uint2*)(vb + (uint32_t)((pbc & psm) + dim * ps) * 2u);
            }
        }
    };
    if (I8 && active) {
        vload(0, va0, vb0);
        vload(1, va1, vb1);
    }

    if (I8) {
        s_kvs[0][wave][lane] = ks_own;
        s_kvs[1][wave][lane] = vs_own;
    }

    // ---- q of the G heads: f32 rows for f32 pages; otherwise fp16 hi + lo,
    // scaled per head by 2^e so that max|q| lands in [2^14, 2^15): hi + lo
    // then carries 22 bits of every element that matters at fp32 precision
    if constexpr (F32) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int h = wave + 4 * j;
#pragma unroll
            for (int i = 0; i < PER; i++) s_qf[h][lane + 64 * i] = qv[j][i];
            if (lane == 0) s_qs[h] = a.scale;  // attention.cpp:134: dot * scale
        }
    } else {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int h = wave + 4 * j;
        float* v = qv[j];
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < PER; i++) mx = fmaxf(mx, fabsf(v[i]));
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        float sigma = 1.f;
        if (mx > 0.f && mx <= 3.0e38f) {
            int e;
            frexpf(mx, &e);
            sigma = ldexpf(1.f, min(15 - e, 120));
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const float x = v[i] * sigma;
            const _Float16 hi = (_Float16)x;
            s_q[0][h][lane + 64 * i] = hi;
            s_q[1][h][lane + 64 * i] = (_Float16)(x - (float)hi);
        }
        if (lane == 0) s_qs[h] = a.scale / sigma;  // attention.cpp:134: dot * scale
    }
    }
    __syncthreads();

    // ---- scores of 4 tiles: sc[t][r] = position pw + 16t + 4seg + r, head l16
    f32x4a sc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) sc[t] = f32x4a{0.f, 0.f, 0.f, 0.f};
    // f32 pages: K of two score tiles in flight, then V of the first two P.V
    // tiles requested behind the last score tiles (their K registers free)
    float4 vf0[4][HD / 64], vf1[4][HD / 64];
    if constexpr (F32) {
        if (active) {
            float4 k0[HD / 16], k1[HD / 16];
            auto krow = [&](int t) { return min(pw + 16 * t + l16, ctx - 1) & psm; };
            kload_f32<HD>(a, kpg[0], kvh, krow(0), seg, k0);
            kload_f32<HD>(a, kpg[1], kvh, krow(1), seg, k1);
            score_f32<HD>(s_qf[l16], seg, k0, sc[0]);
            kload_f32<HD>(a, kpg[2], kvh, krow(2), seg, k0);
            score_f32<HD>(s_qf[l16], seg, k1, sc[1]);
            kload_f32<HD>(a, kpg[3], kvh, krow(3), seg, k1);
            score_f32<HD>(s_qf[l16], seg, k0, sc[2]);
            int rows[4];
            vrows_f32(pw, 0, seg, ctx, vlast, psm, rows);
            vload_f32<HD>(a, vpg[0], kvh, rows, l16, vf0);
            score_f32<HD>(s_qf[l16], seg, k1, sc[3]);
            vrows_f32(pw, 1, seg, ctx, vlast, psm, rows);
            vload_f32<HD>(a, vpg[1], kvh, rows, l16, vf1);
        }
    } else if (active) {  // k-step outer: one step's q fragments live at a time
        if (!I8) kload();
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            const f16x8 qh = *(const f16x8*)&s_q[0][l16][kdim(kk, seg)];
            const f16x8 ql = *(const f16x8*)&s_q[1][l16][kdim(kk, seg)];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                f16x8 kf;
                if constexpr (I8) {
                    const uint4 w = kreg[t][kk / 2];
                    kf = (kk & 1) ? i8x8_to_f16x8(w.z, w.w) : i8x8_to_f16x8(w.x, w.y);
                } else {
                    kf = kreg[t][kk];
                }
                sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh, sc[t], 0, 0, 0);
                sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql, sc[t], 0, 0, 0);
            }
        }
    }

    if (!I8 && !F32 && active) {  // fp16: after the score tiles (their K registers are free again)
        vload(0, va0, vb0);
        vload(1, va1, vb1);
    }

    // ---- softmax statistics over the workgroup's positions, per head l16
    const float qs = s_qs[l16];
    float mloc = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const float4 ks4 = I8 ? *(const float4*)&s_kvs[0][wave][16 * t + 4 * seg] : float4{};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool ok = active && pw + 16 * t + 4 * seg + r < ctx;
            const float ks = r == 0 ? ks4.x : r == 1 ? ks4.y : r == 2 ? ks4.z : ks4.w;
            if constexpr (I8) sc[t][r] = ok ? (sc[t][r] * ks) * qs : -INFINITY;  // kv_cache_quant.h:127
            else sc[t][r] = ok ? sc[t][r] * qs : -INFINITY;
            mloc = fmaxf(mloc, sc[t][r]);
        }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    if (seg == 0) s_m[wave][l16] = mloc;
    __syncthreads();
    const float m = fmaxf(fmaxf(s_m[0][l16], s_m[1][l16]), fmaxf(s_m[2][l16], s_m[3][l16]));
    float lsum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = sc[t][r] == -INFINITY ? 0.f : __expf(sc[t][r] - m);
            sc[t][r] = p;
            lsum += p;
        }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (seg == 0) s_l[wave][l16] = lsum;

    // ---- int8: fold each position's V scale into its probability, times a
    // power of two 2^-e per wave that brings the wave's largest V scale into
    // [1/2, 1), so the fp16 hi + lo split of p * scale neither overflows nor
    // loses bits to fp16 underflow; the output is multiplied back by 2^e
    float ounit = 1.f;
    if constexpr (I8) {
        // lane l holds position pw + l's scale: the wave maximum over valid positions
        float vm = active && pw + lane < ctx ? fmaxf(0.f, vs_own) : 0.f;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) vm = fmaxf(vm, __shfl_xor(vm, o));
        float cw = 1.f;
        if (vm > 0.f && vm <= 3.0e38f) {
            int e;
            frexpf(vm, &e);
            e = max(-120, min(e, 120));
            cw = ldexpf(1.f, -e);
            ounit = ldexpf(1.f, e);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float4 vs4 = *(const float4*)&s_kvs[1][wave][16 * t + 4 * seg];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const bool ok = active && pw + 16 * t + 4 * seg + r < ctx;
                const float vs = r == 0 ? vs4.x : r == 1 ? vs4.y : r == 2 ? vs4.z : vs4.w;
                sc[t][r] = ok ? sc[t][r] * (vs * cw) : 0.f;
            }
        }
    }

    // ---- P.V over the wave's 64 positions (two 32-position MFMA steps)
    f32x4a o[DT];
#pragma unroll
    for (int d = 0; d < DT; d++) o[d] = f32x4a{0.f, 0.f, 0.f, 0.f};
    if constexpr (F32) {
        if (active) {
            int rows[4];
            pv_f32<HD>(sc[0], vf0, o);
            vrows_f32(pw, 2, seg, ctx, vlast, psm, rows);
            vload_f32<HD>(a, vpg[2], kvh, rows, l16, vf0);
            pv_f32<HD>(sc[1], vf1, o);
            vrows_f32(pw, 3, seg, ctx, vlast, psm, rows);
            vload_f32<HD>(a, vpg[3], kvh, rows, l16, vf1);
            pv_f32<HD>(sc[2], vf0, o);
            pv_f32<HD>(sc[3], vf1, o);
        }
    } else if (active) {
        auto pv = [&](int b, const VRun (&ra)[DT], const VRun (&rb)[DT]) {
            f16x8 ph, pl;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float p = sc[2 * b + (i >> 2)][i & 3];
                const _Float16 h = (_Float16)p;
                ph[i] = h;
                pl[i] = (_Float16)(p - (float)h);
            }
            const int pa = pw + 32 * b + 4 * seg, pb = pa + 16;
#pragma unroll
            for (int d = 0; d < DT; d++) {
                f16x8 vf;
                if constexpr (I8) {
                    vf = i8x8_to_f16x8(ra[d], rb[d]);
                } else {
                    const uint2 xa = mask_run(ra[d], pa, ctx), xb = mask_run(rb[d], pb, ctx);
                    vf = __builtin_bit_cast(f16x8, make_uint4(xa.x, xa.y, xb.x, xb.y));
                }
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vf, o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vf, o[d], 0, 0, 0);
            }
        };
        pv(0, va0, vb0);
        pv(1, va1, vb1);
    }

    // ---- combine the 4 waves: o[d][r] = O[head 4seg+r][dim 16d+l16]
    // (f32 pages: dim dvf(l16, d), four consecutive dims per float4)
    if constexpr (F32) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int h = 4 * seg + r;
            if (h < G)
#pragma unroll
                for (int i = 0; i < DT / 4; i++)
                    *(float4*)&s_o[wave * G + h][dvf(l16, 4 * i)] =
                        float4{o[4 * i][r], o[4 * i + 1][r], o[4 * i + 2][r], o[4 * i + 3][r]};
        }
    } else {
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int h = 4 * seg + r;
            if (h < G) s_o[wave * G + h][16 * d + l16] = o[d][r] * ounit;
        }
    }
    __syncthreads();
    const size_t hbase = (size_t)s * a.H + kvh * G;
    if (nchunks == 1) {
        for (int i = tid; i < G * HD; i += ACH) {
            const int h = i / HD, dd = i % HD;
            const float O = (s_o[h][dd] + s_o[G + h][dd]) + (s_o[2 * G + h][dd] + s_o[3 * G + h][dd]);
            const float L = (s_l[0][h] + s_l[1][h]) + (s_l[2][h] + s_l[3][h]);
            attn_store(a, (hbase + h) * HD + dd, O / L);
        }
        return;
    }
    // ---- multi-chunk: publish (max, sum, unnormalised output) for attn_merge_kernel
    const size_t ibase = (size_t)item * a.H + kvh * G;
    for (int i = tid; i < G * HD; i += ACH) {
        const int h = i / HD, dd = i % HD;
        a.part_o[(ibase + h) * HD + dd] = (s_o[h][dd] + s_o[G + h][dd]) + (s_o[2 * G + h][dd] + s_o[3 * G + h][dd]);
    }
    if (tid < G) {
        a.part_ml[(ibase + tid) * 2 + 0] = fmaxf(fmaxf(s_m[0][tid], s_m[1][tid]), fmaxf(s_m[2][tid], s_m[3][tid]));
        a.part_ml[(ibase + tid) * 2 + 1] = (s_l[0][tid] + s_l[1][tid]) + (s_l[2][tid] + s_l[3][tid]);
    }
}

// ---------------------------------------------------------------------------
// Balanced split of the whole batch (the default for fp16 and int8 pages).
// The batch's contexts are cut into 64-position tiles; tiles of sequence s
// are numbered pref[s] .. pref[s+1]-1 (pref = exclusive prefix of the tile
// counts, computed by every workgroup from the device-resident context
// lengths).  Workgroup w of the gx per KV head takes tiles
// [w*T/g, (w+1)*T/g), T = pref[n], g = min(gx, T): equal non-empty shares
// of the batch, all resident at once, whatever the lengths.  A share spans one or more
// sequences; for each sequence segment in it, the 4 waves take its tiles in
// turn (wave v: tiles a+v, a+v+4, ...), each keeping an online softmax
// (running max and sum per head, output rows in LDS rescaled per tile), and
// the 4 wave states are combined at the segment's end.  A segment that is
// the whole sequence writes the output; otherwise it writes a partial
// (max, sum, output) to slot w + s (unique: along the staircase of
// (workgroup, sequence) pairs w + s increases), and attn_merge_kernel<HD,
// true> combines sequence s's slots in workgroup order, i.e. position order.
// Per tile the matrix-core arithmetic is the chunk kernel's above.
// ---------------------------------------------------------------------------
constexpr int SPLIT_MAXN = 1024;   // sequences per launch (the batch bound)
// resident workgroups aimed at: 256 CUs x 4 (head_dim 64) or 3 (head_dim
// 128, whose 148-168 registers per lane leave room for 3)
constexpr int split_slots(int hd) { return 256 * (hd == 128 ? 3 : 4); }

template <int HD, int KV, bool UPG>
__global__ __launch_bounds__(ACH, HD == 128 ? 3 : 4) void attn_split_kernel(AttnArgs a, int G) {
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    constexpr bool I8 = KV == KV_I8, F32 = KV == KV_F32;
    constexpr int KK = HD / 32, DT = HD / 16, QS = HD + 8, PER = HD / 64;
    auto kdim = [](int kk, int sg) { return I8 ? 8 * (KK * sg + kk) : 8 * (4 * kk + sg); };
    typedef typename std::conditional<I8, uint32_t, uint2>::type VRun;
    typedef typename std::conditional<I8, uint4[KK / 2], f16x8[KK]>::type KRow;
    __shared__ __align__(16) float s_qbuf[16 * QS];  // as in attn_mfma_kernel
    _Float16(*s_q)[16][QS] = (_Float16(*)[16][QS])s_qbuf;
    float(*s_qf)[HD + 4] = (float(*)[HD + 4])s_qbuf;
    __shared__ float s_qs[16];
    __shared__ float s_m[4][16], s_l[4][16], s_alpha[4][16];
    __shared__ __align__(16) float s_kvs[2][4][64];
    __shared__ int s_pref[SPLIT_MAXN + 1];
    __shared__ int s_tsum[64];
    extern __shared__ __align__(16) float s_odyn[];
    float(*s_o)[HD] = (float(*)[HD])s_odyn;  // s_o[wave * G + head][dim]: running outputs

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // lane indices are re-derived per tile (see the tile loop)
    int lane = tid & 63, l16 = lane & 15, seg = lane >> 4;
    const int kvh = blockIdx.y, w = blockIdx.x, n = a.n, ps = a.page_size, psl = a.ps_log2, psm = ps - 1;

    // ---- tile counts and their exclusive prefix (n <= 1024): wave 0 lane l
    // sums entries 16l .. 16l+15, then adds the sums of lanes 0 .. l-1 (64
    // broadcast LDS reads) and writes its entries' prefixes.  Workgroup
    // barriers between the phases: a value one lane writes to LDS and another
    // reads needs one (without it the compiler may forward a lane's own
    // earlier store to its load).
    for (int i = tid; i < n; i += ACH) s_pref[i] = (min(a.ctx[i], a.max_ctx) + 63) >> 6;
    __syncthreads();
    int loc[16];
    if (wave == 0) {
        int sum = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int idx = 16 * lane + k;
            loc[k] = idx < n ? s_pref[idx] : 0;
            sum += loc[k];
        }
        s_tsum[lane] = sum;
    }
    __syncthreads();
    if (wave == 0) {
        int run = 0, total = 0;
#pragma unroll 16
        for (int i = 0; i < 64; i++) {
            const int v = s_tsum[i];
            run += i < lane ? v : 0;
            total += v;
        }
        if (lane == 0) s_pref[n] = total;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int idx = 16 * lane + k;
            if (idx < n) s_pref[idx] = run;
            run += loc[k];
        }
    }
    __syncthreads();
    if (w == 0 && kvh == 0)
        for (int i = tid; i <= n; i += ACH) a.pref[i] = s_pref[i];
    // g = min(workgroups, tiles) shares, each non-empty (floor((w+1)T/g) -
    // floor(wT/g) >= 1 for g <= T); workgroups past g have no share
    const int T = s_pref[n];
    const int g = min((int)gridDim.x, T);
    if (w >= g) return;
    const int t0 = (int)(((long long)w * T) / g), t1 = (int)(((long long)(w + 1) * T) / g);
    // first sequence of the share: the last s with pref[s] <= t0
    int s = 0;
    {
        int lo = 0, hi = n - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_pref[mid] <= t0) lo = mid;
            else hi = mid - 1;
        }
        s = __builtin_amdgcn_readfirstlane(lo);
    }

    for (; s < n; s++) {
        const int p0 = s_pref[s], p1 = s_pref[s + 1];
        if (p0 >= t1) break;
        const int ja = max(t0, p0) - p0, jb = min(t1, p1) - p0;  // the segment: tiles [ja, jb) of s
        const bool whole = ja == 0 && jb == p1 - p0;
        const int ctx = min(a.ctx[s], a.max_ctx);
        const int32_t* ptab = a.page_table + (size_t)s * a.max_pages;
        const int vlast = (ctx - 1) & ~3;
        const size_t blk = (size_t)ps * (HD + 4);
        const _Float16* kc = (const _Float16*)a.kc;
        const _Float16* vc = (const _Float16*)a.vc;

        // ---- per-tile loads (tile j: positions 64j .. 64j+63 of s)
        // page ids: kpg/vpg of the tile being loaded; int8 also keeps the
        // ids of the tile after it (kpg2/vpg2), requested a tile earlier
        int kpg[4], vpg[4], kpg2[4], vpg2[4];
        auto ids_to = [&](int j, int (&kp)[4], int (&vp)[4]) {
            const int pw = 64 * j;
#pragma unroll
            for (int t = 0; t < 4; t++) kp[t] = page_id<UPG>(ptab, min(pw + 16 * t + l16, ctx - 1) >> psl);
#pragma unroll
            for (int t = 0; t < 4; t++) vp[t] = page_id<UPG>(ptab, min(pw + 16 * t + 4 * seg, vlast) >> psl);
        };
        auto ids = [&](int j) { ids_to(j, kpg, vpg); };
        KRow kreg[4];
        auto kload = [&](int j) {
            const int pw = 64 * j;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int pc = min(pw + 16 * t + l16, ctx - 1);
                if constexpr (I8) {
                    const char* kb = page_block(a.kc, kpg[t], a.Hkv, kvh, blk);
                    const uint32_t o = (uint32_t)((pc & psm) * HD + 8 * KK * seg);
#pragma unroll
                    for (int i = 0; i < KK / 2; i++) kreg[t][i] = *(const uint4*)(kb + (o + 16u * i));
                } else {
                    const char* kb = page_block(kc, kpg[t], a.Hkv, kvh, (size_t)ps * HD * 2);
                    const uint32_t o = (uint32_t)((pc & psm) * HD + 8 * seg) * 2u;
#pragma unroll
                    for (int kk = 0; kk < KK; kk++) kreg[t][kk] = *(const f16x8*)(kb + (o + 64u * kk));
                }
            }
        };
        VRun va0[DT], vb0[DT], va1[DT], vb1[DT];
        auto vload = [&](int j, int b, VRun (&ra)[DT], VRun (&rb)[DT]) {
            const int pw = 64 * j;
            const int pac = min(pw + 32 * b + 4 * seg, vlast), pbc = min(pw + 32 * b + 16 + 4 * seg, vlast);
            if constexpr (I8) {
                const char* va = page_block(a.vc, vpg[2 * b], a.Hkv, kvh, blk);
                const char* vb = page_block(a.vc, vpg[2 * b + 1], a.Hkv, kvh, blk);
#pragma unroll
                for (int d = 0; d < DT; d++) {
                    const int off = (16 * d + l16) * ps;
                    ra[d] = *(const uint32_t*)(va + (uint32_t)((pac & psm) + off));
                    rb[d] = *(const uint32_t*)(vb + (uint32_t)((pbc & psm) + off));
                }
            } else {
                const char* va = page_block(vc, vpg[2 * b], a.Hkv, kvh, (size_t)HD * ps * 2);
                const char* vb = page_block(vc, vpg[2 * b + 1], a.Hkv, kvh, (size_t)HD * ps * 2);
#pragma unroll
                for (int d = 0; d < DT; d++) {
                    const int off = (16 * d + l16) * ps;
                    ra[d] = *(const uint2*)(va + (uint32_t)((pac & psm) + off) * 2u);
                    rb[d] = *(const uint2*)(vb + (uint32_t)((pbc & psm) + off) * 2u);
                }
            }
        };
        // int8 scales of position 64j + lane (page kpg[lane / 16]), stored to
        // LDS at the top of the tile's iteration and read back per 4-position run
        float ks_own = 0.f, vs_own = 0.f;
        auto sload = [&](int j) {
            const int pg = seg == 0 ? kpg[0] : seg == 1 ? kpg[1] : seg == 2 ? kpg[2] : kpg[3];
            const size_t b = ((size_t)pg * a.Hkv + kvh) * blk + (ps * HD + 4 * (min(64 * j + lane, ctx - 1) & psm));
            ks_own = *(const float*)((const int8_t*)a.kc + b);
            vs_own = *(const float*)((const int8_t*)a.vc + b);
        };

        // ---- q of the G heads (requested first), the wave's first tile's
        // page ids (and int8 K rows and V runs), then q staged as in the
        // chunk kernel
        float qv[4][PER];
#pragma unroll
        for (int jh = 0; jh < 4; jh++) {
            const int h = wave + 4 * jh;
#pragma unroll
            for (int i = 0; i < PER; i++)
                qv[jh][i] = h < G ? a.q[((size_t)s * a.H + kvh * G + h) * HD + lane + 64 * i] : 0.f;
        }
        int j = ja + wave;
        if (j < jb) {
            ids(j);
            if (I8) {
                sload(j);
                kload(j);
                vload(j, 0, va0, vb0);
                vload(j, 1, va1, vb1);
                if (j + 4 < jb) ids_to(j + 4, kpg2, vpg2);
            }
        }
        if constexpr (F32) {
#pragma unroll
            for (int jh = 0; jh < 4; jh++) {
                const int h = wave + 4 * jh;
#pragma unroll
                for (int i = 0; i < PER; i++) s_qf[h][lane + 64 * i] = qv[jh][i];
                if (lane == 0) s_qs[h] = a.scale;  // attention.cpp:134: dot * scale
            }
        } else {
#pragma unroll
        for (int jh = 0; jh < 4; jh++) {
            const int h = wave + 4 * jh;
            float mx = 0.f;
#pragma unroll
            for (int i = 0; i < PER; i++) mx = fmaxf(mx, fabsf(qv[jh][i]));
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            float sigma = 1.f;
            if (mx > 0.f && mx <= 3.0e38f) {
                int e;
                frexpf(mx, &e);
                sigma = ldexpf(1.f, min(15 - e, 120));
            }
#pragma unroll
            for (int i = 0; i < PER; i++) {
                const float x = qv[jh][i] * sigma;
                const _Float16 hi = (_Float16)x;
                s_q[0][h][lane + 64 * i] = hi;
                s_q[1][h][lane + 64 * i] = (_Float16)(x - (float)hi);
            }
            if (lane == 0) s_qs[h] = a.scale / sigma;  // attention.cpp:134: dot * scale
        }
        }
        __syncthreads();
        const float qs = s_qs[l16];

        // ---- the wave's tiles, online softmax per head (lane: head l16)
        float m_run = -INFINITY, l_run = 0.f;
        bool first = true;
        for (; j < jb; j += 4) {
            // opaque to the compiler: every lane-derived address below is
            // recomputed per tile instead of being hoisted out of the loops
            // and held (spilled) across them
            asm volatile("" : "+v"(lane));
            l16 = lane & 15;
            seg = lane >> 4;
            const int pw = 64 * j;
            if (I8) {
                s_kvs[0][wave][lane] = ks_own;
                s_kvs[1][wave][lane] = vs_own;
            }
            if (!I8 && !F32) kload(j);
            f32x4a sc[4];
#pragma unroll
            for (int t = 0; t < 4; t++) sc[t] = f32x4a{0.f, 0.f, 0.f, 0.f};
            // f32 pages: the chunk kernel's pipeline (K of two score tiles in
            // flight, V of the first two P.V tiles behind the last score tiles)
            float4 vf0[4][HD / 64], vf1[4][HD / 64];
            if constexpr (F32) {
                float4 k0[HD / 16], k1[HD / 16];
                auto krow = [&](int t) { return min(pw + 16 * t + l16, ctx - 1) & psm; };
                kload_f32<HD>(a, kpg[0], kvh, krow(0), seg, k0);
                kload_f32<HD>(a, kpg[1], kvh, krow(1), seg, k1);
                score_f32<HD>(s_qf[l16], seg, k0, sc[0]);
                kload_f32<HD>(a, kpg[2], kvh, krow(2), seg, k0);
                score_f32<HD>(s_qf[l16], seg, k1, sc[1]);
                kload_f32<HD>(a, kpg[3], kvh, krow(3), seg, k1);
                score_f32<HD>(s_qf[l16], seg, k0, sc[2]);
                int rows[4];
                vrows_f32(pw, 0, seg, ctx, vlast, psm, rows);
                vload_f32<HD>(a, vpg[0], kvh, rows, l16, vf0);
                score_f32<HD>(s_qf[l16], seg, k1, sc[3]);
                vrows_f32(pw, 1, seg, ctx, vlast, psm, rows);
                vload_f32<HD>(a, vpg[1], kvh, rows, l16, vf1);
            } else
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const f16x8 qh = *(const f16x8*)&s_q[0][l16][kdim(kk, seg)];
                const f16x8 ql = *(const f16x8*)&s_q[1][l16][kdim(kk, seg)];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    f16x8 kf;
                    if constexpr (I8) {
                        const uint4 wv = kreg[t][kk / 2];
                        kf = (kk & 1) ? i8x8_to_f16x8(wv.z, wv.w) : i8x8_to_f16x8(wv.x, wv.y);
                    } else {
                        kf = kreg[t][kk];
                    }
                    sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh, sc[t], 0, 0, 0);
                    sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql, sc[t], 0, 0, 0);
                }
            }
            if (!I8 && !F32) {  // fp16: V after the score tiles (K's registers are free again)
                vload(j, 0, va0, vb0);
                vload(j, 1, va1, vb1);
            }
            // scores (int8: times each position's K scale), tile max per head
            float mt = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float4 ks4 = I8 ? *(const float4*)&s_kvs[0][wave][16 * t + 4 * seg] : float4{};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const bool ok = pw + 16 * t + 4 * seg + r < ctx;
                    const float ks = r == 0 ? ks4.x : r == 1 ? ks4.y : r == 2 ? ks4.z : ks4.w;
                    if constexpr (I8) sc[t][r] = ok ? (sc[t][r] * ks) * qs : -INFINITY;  // kv_cache_quant.h:127
                    else sc[t][r] = ok ? sc[t][r] * qs : -INFINITY;
                    mt = fmaxf(mt, sc[t][r]);
                }
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float m_new = fmaxf(m_run, mt);  // finite: a tile holds a position < ctx
            const float alpha = first ? 0.f : __expf(m_run - m_new);
            float lsum = 0.f;
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float p = sc[t][r] == -INFINITY ? 0.f : __expf(sc[t][r] - m_new);
                    sc[t][r] = p;
                    lsum += p;
                }
            lsum += __shfl_xor(lsum, 16);
            lsum += __shfl_xor(lsum, 32);
            l_run = l_run * alpha + lsum;
            m_run = m_new;
            if (seg == 0) s_alpha[wave][l16] = alpha;

            // int8: fold each position's V scale (times a per-tile power of
            // two 2^-e) into its probability; the tile's output is scaled by 2^e
            float ounit = 1.f;
            if constexpr (I8) {
                float vm = pw + lane < ctx ? fmaxf(0.f, s_kvs[1][wave][lane]) : 0.f;
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) vm = fmaxf(vm, __shfl_xor(vm, o));
                float cw = 1.f;
                if (vm > 0.f && vm <= 3.0e38f) {
                    int e;
                    frexpf(vm, &e);
                    e = max(-120, min(e, 120));
                    cw = ldexpf(1.f, -e);
                    ounit = ldexpf(1.f, e);
                }
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float4 vs4 = *(const float4*)&s_kvs[1][wave][16 * t + 4 * seg];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const bool ok = pw + 16 * t + 4 * seg + r < ctx;
                        const float vs = r == 0 ? vs4.x : r == 1 ? vs4.y : r == 2 ? vs4.z : vs4.w;
                        sc[t][r] = ok ? sc[t][r] * (vs * cw) : 0.f;
                    }
                }
            }

            // ---- P.V of the tile (two 32-position MFMA steps)
            f32x4a o[DT];
#pragma unroll
            for (int d = 0; d < DT; d++) o[d] = f32x4a{0.f, 0.f, 0.f, 0.f};
            auto pv = [&](int b, const VRun (&ra)[DT], const VRun (&rb)[DT]) {
                f16x8 ph, pl;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float p = sc[2 * b + (i >> 2)][i & 3];
                    const _Float16 h = (_Float16)p;
                    ph[i] = h;
                    pl[i] = (_Float16)(p - (float)h);
                }
                const int pa = pw + 32 * b + 4 * seg, pb = pa + 16;
#pragma unroll
                for (int d = 0; d < DT; d++) {
                    f16x8 vf;
                    if constexpr (I8) {
                        vf = i8x8_to_f16x8(ra[d], rb[d]);
                    } else {
                        const uint2 xa = mask_run(ra[d], pa, ctx), xb = mask_run(rb[d], pb, ctx);
                        vf = __builtin_bit_cast(f16x8, make_uint4(xa.x, xa.y, xb.x, xb.y));
                    }
                    o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vf, o[d], 0, 0, 0);
                    o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vf, o[d], 0, 0, 0);
                }
            };
            if constexpr (F32) {
                int rows[4];
                pv_f32<HD>(sc[0], vf0, o);
                vrows_f32(pw, 2, seg, ctx, vlast, psm, rows);
                vload_f32<HD>(a, vpg[2], kvh, rows, l16, vf0);
                pv_f32<HD>(sc[1], vf1, o);
                vrows_f32(pw, 3, seg, ctx, vlast, psm, rows);
                vload_f32<HD>(a, vpg[3], kvh, rows, l16, vf1);
                pv_f32<HD>(sc[2], vf0, o);
                pv_f32<HD>(sc[3], vf1, o);
            } else {
                pv(0, va0, vb0);
                pv(1, va1, vb1);
            }

            // the next tile's loads in flight while this tile's output is
            // folded into the wave's rows.  int8: its ids arrived during this
            // tile, so its scales, rows and runs are requested at once, and
            // the ids of the tile after it are requested; fp16: its ids (its
            // rows are requested at its top: holding them here would spill)
            if (j + 4 < jb) {
                if (I8) {
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        kpg[t] = kpg2[t];
                        vpg[t] = vpg2[t];
                    }
                    sload(j + 4);
                    kload(j + 4);
                    vload(j + 4, 0, va0, vb0);
                    vload(j + 4, 1, va1, vb1);
                    if (j + 8 < jb) ids_to(j + 8, kpg2, vpg2);
                } else {
                    ids(j + 4);
                }
            }
            // o[d][r] = O[head 4seg+r][dim 16d+l16]: row = row * alpha(head) + o * 2^e
            // (f32 pages: dim dvf(l16, d), four consecutive dims per float4)
            if constexpr (F32) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int h = 4 * seg + r;
                    if (h < G) {
                        const float al = s_alpha[wave][h];
#pragma unroll
                        for (int i = 0; i < DT / 4; i++) {
                            float4* row = (float4*)&s_o[wave * G + h][dvf(l16, 4 * i)];
                            const float4 x{o[4 * i][r], o[4 * i + 1][r], o[4 * i + 2][r], o[4 * i + 3][r]};
                            if (first) {
                                *row = x;
                            } else {
                                const float4 y = *row;
                                *row = float4{__builtin_fmaf(y.x, al, x.x), __builtin_fmaf(y.y, al, x.y),
                                              __builtin_fmaf(y.z, al, x.z), __builtin_fmaf(y.w, al, x.w)};
                            }
                        }
                    }
                }
            } else
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int h = 4 * seg + r;
                if (h < G) {
                    const float al = s_alpha[wave][h];
#pragma unroll
                    for (int d = 0; d < DT; d++) {
                        float* row = &s_o[wave * G + h][16 * d + l16];
                        *row = first ? o[d][r] * ounit : __builtin_fmaf(*row, al, o[d][r] * ounit);
                    }
                }
            }
            first = false;
        }

        // ---- combine the 4 waves' states of the segment
        if (seg == 0) {
            s_m[wave][l16] = m_run;  // -inf for a wave without tiles (its rows are not read)
            s_l[wave][l16] = l_run;
        }
        __syncthreads();
        const size_t hbase = (size_t)s * a.H + kvh * G;
        const size_t sbase = ((size_t)w + s) * a.H + kvh * G;  // partial slot w + s
        for (int i = tid; i < G * HD; i += ACH) {
            const int h = i / HD, dd = i % HD;
            const float M = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
            float O = 0.f, L = 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float mv = s_m[v][h];
                const float e = mv == -INFINITY ? 0.f : __expf(mv - M);
                O = mv == -INFINITY ? O : __builtin_fmaf(s_o[v * G + h][dd], e, O);
                L = __builtin_fmaf(s_l[v][h], e, L);
            }
            if (whole) attn_store(a, (hbase + h) * HD + dd, O / L);
            else a.part_o[(sbase + h) * HD + dd] = O;
        }
        if (!whole && tid < G) {
            const int h = tid;
            const float M = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
            float L = 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) L = __builtin_fmaf(s_l[v][h], s_m[v][h] == -INFINITY ? 0.f : __expf(s_m[v][h] - M), L);
            a.part_ml[(sbase + h) * 2 + 0] = M;
            a.part_ml[(sbase + h) * 2 + 1] = L;
        }
        __syncthreads();  // s_q, s_o, s_m are reused by the next segment
    }
}

// Sequences of several chunks: one wave per (sequence, query head) merges
// the chunk partials (a separate launch: no device-scope fence or atomic,
// which on a multi-XCD part would write back and invalidate L2 for every
// workgroup).  Lane c holds chunk c's (m, l) (64 chunks per round), the
// weights exp(m_c - M) reach every lane by shuffle, and lane d accumulates
// output dimensions d, d+64, ... over the chunks in chunk order.
// SPLIT: the partials of attn_split_kernel, sequence s's in slots w + s for
// the workgroups w whose tile range meets its tiles [pref[s], pref[s+1])
// (tile t lies in workgroup ((t+1)*g - 1) / T, g = min(gx, T): every one of
// them has a share, so every slot in the range is written).
template <int HD, bool SPLIT>
__global__ __launch_bounds__(64) void attn_merge_kernel(AttnArgs a) {
    constexpr int HPL = HD >= 64 ? HD / 64 : 1;  // dimensions per lane
    const int s = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int dl = min(lane, HD - 1);            // lanes past a head_dim < 64 redo the last dimension, unstored
    int nch;
    size_t base;                                 // partial row of the sequence's first chunk or slot
    if (SPLIT) {
        const long long T = a.pref[a.n], P0 = a.pref[s], P1 = a.pref[s + 1];
        if (T <= 0 || P1 <= P0) return;
        const long long g = std::min<long long>(a.gx, T);
        const int wf = (int)(((P0 + 1) * g - 1) / T), wl = (int)((P1 * g - 1) / T);
        nch = wl - wf + 1;
        base = ((size_t)wf + s) * a.H + h;
    } else {
        nch = (min(a.ctx[s], a.max_ctx) + ACH - 1) / ACH;
        base = (size_t)s * ((a.max_ctx + ACH - 1) / ACH) * a.H + h;
    }
    if (nch <= 1) return;
    float M = -INFINITY;
    for (int c = lane; c < nch; c += 64) M = fmaxf(M, a.part_ml[(base + (size_t)c * a.H) * 2]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    float L = 0.f, O[HPL];
#pragma unroll
    for (int k = 0; k < HPL; k++) O[k] = 0.f;
    for (int c0 = 0; c0 < nch; c0 += 64) {
        const int c = c0 + lane;
        float w = 0.f, lw = 0.f;
        if (c < nch) {
            const size_t it = base + (size_t)c * a.H;
            w = __expf(a.part_ml[it * 2] - M);
            lw = a.part_ml[it * 2 + 1] * w;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) lw += __shfl_xor(lw, o);
        L += lw;
        const int cn = min(64, nch - c0);
        const float* po = a.part_o + (base + (size_t)c0 * a.H) * HD + dl;
        for (int j0 = 0; j0 < cn; j0 += 8) {  // 8 chunks' loads in flight (clamped into the valid ones)
            float v[8][HPL];
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int k = 0; k < HPL; k++) v[u][k] = po[(size_t)min(j0 + u, cn - 1) * a.H * HD + 64 * k];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float wj = __shfl(w, j0 + u);
#pragma unroll
                for (int k = 0; k < HPL; k++) O[k] = j0 + u < cn ? __builtin_fmaf(v[u][k], wj, O[k]) : O[k];
            }
        }
    }
    if (lane < HD) {
#pragma unroll
        for (int k = 0; k < HPL; k++) attn_store(a, ((size_t)s * a.H + h) * HD + lane + 64 * k, O[k] / L);
    }
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

// split kernel: workgroups per KV head (at most one 64-position tile each)
static int split_gx(int n, int Hkv, int hd, int max_ctx) {
    return (int)std::min<long long>(std::max(1, split_slots(hd) / Hkv), (long long)n * ((max_ctx + 63) / 64));
}

// partial slots: chunk items of the chunk grid, or gx + n of the split
static size_t attn_slots(int n, int Hkv, int hd, int max_ctx) {
    return std::max<size_t>((size_t)n * ((max_ctx + ACH - 1) / ACH), (size_t)split_gx(n, Hkv, hd, max_ctx) + n);
}

size_t attn_workspace_bytes(int n, int H, int Hkv, int hd, int max_ctx) {
    const size_t slots = attn_slots(n, Hkv, hd, max_ctx);
    return ((size_t)n * Hkv * 4 + 255) / 256 * 256 + ((size_t)(n + 1) * 4 + 255) / 256 * 256 + slots * H * 2 * 4 +
           slots * H * hd * 4;
}

// 0: automatic (the balanced split when the chunk grid would need more than
// one round of resident workgroups, 4 per CU x 256 CUs, at the host-known
// bound n x ceil(max_ctx / 256); below that the chunk grid, whose per-chunk
// workgroups carry no share bookkeeping), 1: chunk grid, 2: balanced split,
// 3: the plain fp32 VALU kernel for f32 and fp16 pages (int8 pages: automatic)
static int g_attn_form = 0;

int launch_attention(const float* q, const void* kc, const void* vc, uint32_t kv_dtype, const int32_t* page_table,
                     int max_pages, const int32_t* ctx, int n, int H, int Hkv, int hd, int page_size, float scale,
                     int max_ctx, float* out, void* ws, size_t ws_bytes, hipStream_t st, uint16_t* out_hi,
                     uint16_t* out_lo) {
    QH_REQUIRE(q && kc && vc && page_table && ctx && (out || (out_hi && out_lo)) && ws, QRAF_HIP_ERR_INVALID,
               "attention: null pointer");
    QH_REQUIRE(n > 0 && n <= 1024, QRAF_HIP_ERR_INVALID, "attention: batch %d outside 1..1024", n);
    QH_REQUIRE(Hkv > 0 && H % Hkv == 0, QRAF_HIP_ERR_INVALID, "attention: %d heads not a multiple of %d kv heads", H, Hkv);
    QH_REQUIRE(page_size > 0 && max_pages > 0 && max_ctx > 0 && max_ctx <= max_pages * page_size, QRAF_HIP_ERR_INVALID,
               "attention: bad page geometry");
    QH_REQUIRE(kv_dtype == DT_F32 || kv_dtype == DT_F16 || kv_dtype == DT_I8, QRAF_HIP_ERR_DTYPE,
               "attention: KV dtype %u", kv_dtype);
    QH_REQUIRE(kv_dtype != DT_I8 || ((hd == 64 || hd == 128) && H / Hkv <= 16 && page_size % 4 == 0 &&
                                     (page_size & (page_size - 1)) == 0),
               QRAF_HIP_ERR_INVALID,
               "attention: int8 pages need head_dim 64/128, group <= 16, page_size a power of two >= 4");
    QH_REQUIRE(ws_bytes >= attn_workspace_bytes(n, H, Hkv, hd, max_ctx), QRAF_HIP_ERR_INVALID,
               "attention: workspace too small");
    const int items = n * ((max_ctx + ACH - 1) / ACH);
    const size_t slots = attn_slots(n, Hkv, hd, max_ctx);
    AttnArgs a;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.page_table = page_table;
    a.ctx = ctx;
    a.out = out;
    a.out_hi = out_hi;
    a.out_lo = out_lo;
    uint8_t* w = (uint8_t*)ws;
    a.counters = (uint32_t*)w;  // reserved
    w += ((size_t)n * Hkv * 4 + 255) / 256 * 256;
    a.pref = (int32_t*)w;
    w += ((size_t)(n + 1) * 4 + 255) / 256 * 256;
    a.part_ml = (float*)w;
    w += slots * H * 2 * 4;
    a.part_o = (float*)w;
    a.gx = split_gx(n, Hkv, hd, max_ctx);
    a.ps_log2 = 0;
    while ((1 << a.ps_log2) < page_size) a.ps_log2++;
    const bool ps_pow2 = (1 << a.ps_log2) == page_size;
    a.n = n;
    a.H = H;
    a.Hkv = Hkv;
    a.page_size = page_size;
    a.max_pages = max_pages;
    a.max_ctx = max_ctx;
    a.scale = scale;
    const int G = H / Hkv;
    const bool mfma_shape = (hd == 64 || hd == 128) && G <= 16 && page_size % 4 == 0 && ps_pow2;
    // One sequence of at most one 256-position chunk on f32 pages at
    // head_dim 64 (batch-1 decode of a small model): the VALU kernel, whose
    // one round of K/V loads beats the matrix-core kernel's pipelined tiles
    // when a single workgroup per KV head is all there is (SmolLM2-135M
    // architecture decode on MI355X: 1,373 against 1,296 tok/s)
    const bool single_f32 = kv_dtype == DT_F32 && hd == 64 && n == 1 && max_ctx <= ACH && g_attn_form == 0;
    const bool valu = !mfma_shape || (g_attn_form == 3 && kv_dtype != DT_I8) || single_f32;
    const bool split = !valu && (g_attn_form == 2 || (g_attn_form != 1 && items > 1024));
    if (valu) {  // the plain fp32 VALU kernel
        if (kv_dtype == DT_F32) QH_TRY(launch_attn_t<float>(a, hd, G, items, st));
        else QH_TRY(launch_attn_t<_Float16>(a, hd, G, items, st));
    } else {
        const int kind = kv_dtype == DT_I8 ? KV_I8 : kv_dtype == DT_F32 ? KV_F32 : KV_F16;
        const dim3 grid(split ? a.gx : items, Hkv);
        const size_t lds = 4 * G * hd * sizeof(float);
        const bool upg = page_size >= 16;  // page ids uniform per wave (page_id)
#define QH_ATTN_MFMA(K, HDv, KINDv)                                                                    \
    if (kind == KINDv && hd == HDv) {                                                                  \
        if (upg) hipLaunchKernelGGL((K<HDv, KINDv, true>), grid, dim3(ACH), lds, st, a, G);            \
        else hipLaunchKernelGGL((K<HDv, KINDv, false>), grid, dim3(ACH), lds, st, a, G);               \
    }
        if (split) {
            QH_ATTN_MFMA(attn_split_kernel, 128, KV_F16) QH_ATTN_MFMA(attn_split_kernel, 64, KV_F16)
            QH_ATTN_MFMA(attn_split_kernel, 128, KV_I8) QH_ATTN_MFMA(attn_split_kernel, 64, KV_I8)
            QH_ATTN_MFMA(attn_split_kernel, 128, KV_F32) QH_ATTN_MFMA(attn_split_kernel, 64, KV_F32)
        } else {
            QH_ATTN_MFMA(attn_mfma_kernel, 128, KV_F16) QH_ATTN_MFMA(attn_mfma_kernel, 64, KV_F16)
            QH_ATTN_MFMA(attn_mfma_kernel, 128, KV_I8) QH_ATTN_MFMA(attn_mfma_kernel, 64, KV_I8)
            QH_ATTN_MFMA(attn_mfma_kernel, 128, KV_F32) QH_ATTN_MFMA(attn_mfma_kernel, 64, KV_F32)
        }
#undef QH_ATTN_MFMA
        QH_CHECK_HIP(hipGetLastError());
    }
    if (split) {  // a sequence may span several workgroups' shares
        const dim3 mg(n, H);
        if (hd == 128) hipLaunchKernelGGL((attn_merge_kernel<128, true>), mg, dim3(64), 0, st, a);
        else hipLaunchKernelGGL((attn_merge_kernel<64, true>), mg, dim3(64), 0, st, a);
        QH_CHECK_HIP(hipGetLastError());
    } else if (max_ctx > ACH) {  // some sequence may span several chunks
        const dim3 mg(n, H);
        if (hd == 128) hipLaunchKernelGGL((attn_merge_kernel<128, false>), mg, dim3(64), 0, st, a);
        else if (hd == 64) hipLaunchKernelGGL((attn_merge_kernel<64, false>), mg, dim3(64), 0, st, a);
        else if (hd == 32) hipLaunchKernelGGL((attn_merge_kernel<32, false>), mg, dim3(64), 0, st, a);
        else hipLaunchKernelGGL((attn_merge_kernel<16, false>), mg, dim3(64), 0, st, a);
        QH_CHECK_HIP(hipGetLastError());
    }
    return QRAF_HIP_OK;
}

// ----------------------------------------------------------------------------
// Per-token post-processing of the fused QKV projection (attention.cpp:100-119):
// bias add (F32 biases only, transformer.cpp:45-50), interleaved-pair RoPE on
// every q and k head (ops.cpp:158-177), and the store of k, v at the token's
// position into the paged cache.  Grid-stride over (sequence, work element):
// a rotated pair of a q or k head, or one v element.  qkv may be S slices
// (GEMM split-K partials) of `slice` floats, summed in slice order.
// ----------------------------------------------------------------------------
template <typename KT, int SC>
__global__ void rope_append_kernel(const float* __restrict__ qkv, const float* __restrict__ bias, int H, int Hkv,
                                   int hd, const int32_t* __restrict__ pos, const float* __restrict__ rope,
                                   float* __restrict__ q_out, KT* __restrict__ kc, KT* __restrict__ vc,
                                   const int32_t* __restrict__ page_table, int max_pages, int page_size, int n, int S,
                                   size_t slice) {
    const int qd = H * hd, kvd = Hkv * hd, row = qd + 2 * kvd;
    const int per = (qd + kvd) / 2 + kvd;  // work elements per sequence
    for (size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x; w < (size_t)n * per;
         w += (size_t)gridDim.x * blockDim.x) {
    const int s = (int)(w / per), e = (int)(w % per);
    const size_t rbase = (size_t)s * row;
    // SC: the slice count as a constant (0: S at run time)
    auto ld = [&](int i) {
        if (SC > 0) {
            float t[SC > 0 ? SC : 1];
#pragma unroll
            for (int u = 0; u < SC; u++) t[u] = qkv[(size_t)u * slice + rbase + i];
            float acc = t[0];
#pragma unroll
            for (int u = 1; u < SC; u++) acc += t[u];
            return acc;
        }
        return sum_slices(qkv, S, slice, rbase + i);
    };
    // Every operand is requested before any is waited for, except what needs
    // the position (its page and rotation): work element e is the rotated
    // pair (i0, i0 + 1) of the q|k part, or one v element (i0 = i1).
    const bool rot = e < (qd + kvd) / 2;
    const int i0 = rot ? 2 * e : qd + kvd + (e - (qd + kvd) / 2);
    const int i1 = rot ? i0 + 1 : i0;
    const int p = pos[s];
    float a = ld(i0), b = ld(i1);
    const float* bp = bias ? bias : qkv;  // without a bias these loads read qkv and are not used
    const float ba = bp[bias ? i0 : 0], bb = bp[bias ? i1 : 0];
    const int page = page_table[(size_t)s * max_pages + p / page_size], off = p % page_size;
    const int i = rot ? i0 % hd : 0;  // even index inside the head
    const float* cs = rope + (size_t)p * hd + i;  // (cos, sin) of pair i/2
    const float c = cs[0], sn = cs[1];
    // pairs (i, i+1) of q heads, then k heads: rotate; v: copy.  Products are
    // rounded separately (no FMA contraction), as the reference's scalar code.
    if (bias) {
        a = __fadd_rn(a, ba);
        b = __fadd_rn(b, bb);
    }
    if (rot) {
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
        const int j = i0 - (qd + kvd);  // v element
        const int vh = j / hd;
        if (sizeof(KT) == 4)
            vc[(((size_t)page * Hkv + vh) * page_size + off) * hd + j % hd] = (KT)a;
        else  // fp16 pages keep V dimension-major
            vc[(((size_t)page * Hkv + vh) * hd + j % hd) * page_size + off] = (KT)a;
    }
    }
}

// int8 pages: QuantizedKVCache::store (kv_cache_quant.h:61-95) of the rotated
// k and the v of each KV head.  Per sequence, workgroups y >= 1 rotate the q
// pairs and workgroup 0's wave w takes heads j = w, w + 4, ... of the 2*Hkv
// (K heads, then V heads); lane l holds elements 2l, 2l+1 of a K head (one
// rotated pair) or l, l+64 of a V head, the wave's absmax is a max-reduction,
// and scale = absmax / 127, q = clamp(round(x * (1 / scale)), +-127) with
// the reference's divisions (IEEE, correctly rounded) and rounding (half away
// from zero).  head_dim <= 128.
__global__ __launch_bounds__(256) void rope_append_i8_kernel(const float* __restrict__ qkv,
                                                             const float* __restrict__ bias, int H, int Hkv, int hd,
                                                             const int32_t* __restrict__ pos,
                                                             const float* __restrict__ rope, float* __restrict__ q_out,
                                                             int8_t* __restrict__ kc, int8_t* __restrict__ vc,
                                                             const int32_t* __restrict__ page_table, int max_pages,
                                                             int page_size, int S, size_t slice) {
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qd = H * hd, kvd = Hkv * hd;
    // blockIdx.y 0: the K and V heads; y >= 1: q pairs (y-1)*256 + tid, ...
    const size_t rbase = (size_t)s * (qd + 2 * kvd);
    auto ld = [&](int i) {
        const float x = sum_slices(qkv, S, slice, rbase + i);
        return bias ? __fadd_rn(x, bias[i]) : x;
    };
    const int p = pos[s];
    const int page = page_table[(size_t)s * max_pages + p / page_size], off = p % page_size;
    const float* cs = rope + (size_t)p * hd;
    // rotated pair (i0, i0 + 1) of the q|k part, as rope_append_kernel
    auto rot = [&](int i0, float& ra, float& rb) {
        const int i = i0 % hd;
        const float x = ld(i0), y = ld(i0 + 1), c = cs[i], sn = cs[i + 1];
        ra = __fsub_rn(__fmul_rn(x, c), __fmul_rn(y, sn));
        rb = __fadd_rn(__fmul_rn(x, sn), __fmul_rn(y, c));
    };
    if (blockIdx.y > 0) {
        for (int e = (blockIdx.y - 1) * 256 + tid; e < qd / 2; e += (gridDim.y - 1) * 256) {
            float ra, rb;
            rot(2 * e, ra, rb);
            q_out[(size_t)s * qd + 2 * e] = ra;
            q_out[(size_t)s * qd + 2 * e + 1] = rb;
        }
        return;
    }
    const size_t blk = (size_t)page_size * (hd + 4);
    for (int j = wave; j < 2 * Hkv; j += 4) {
        const bool isk = j < Hkv;
        const int h = isk ? j : j - Hkv;
        const int d0 = isk ? 2 * lane : lane, d1 = isk ? 2 * lane + 1 : lane + 64;
        const bool v0 = d0 < hd, v1 = d1 < hd;
        float x0 = 0.f, x1 = 0.f;
        if (isk) {
            if (v0) rot(qd + h * hd + d0, x0, x1);
        } else {
            if (v0) x0 = ld(qd + kvd + h * hd + d0);
            if (v1) x1 = ld(qd + kvd + h * hd + d1);
        }
        float amax = fmaxf(v0 ? fabsf(x0) : 0.f, v1 ? fabsf(x1) : 0.f);  // kv_cache_quant.h:75-78
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
        const float scale = amax / 127.0f;                      // :80
        const float inv = scale > 0.f ? 1.0f / scale : 0.0f;    // :82
        auto qz = [&](float x) {                                // :88-91
            return (int8_t)(int)fmaxf(-127.0f, fminf(127.0f, roundf(x * inv)));
        };
        int8_t* b = (isk ? kc : vc) + ((size_t)page * Hkv + h) * blk;
        if (isk) {
            if (v0) {
                b[(size_t)off * hd + d0] = qz(x0);
                b[(size_t)off * hd + d1] = qz(x1);
            }
        } else {  // dimension-major
            if (v0) b[(size_t)d0 * page_size + off] = qz(x0);
            if (v1) b[(size_t)d1 * page_size + off] = qz(x1);
        }
        if (lane == 0) *(float*)(b + (size_t)page_size * hd + 4 * off) = scale;
    }
}

int launch_rope_append(const float* qkv, const float* bias, int n, int H, int Hkv, int hd, const int32_t* pos,
                       const float* rope, float* q_out, void* kc, void* vc, uint32_t kv_dtype,
                       const int32_t* page_table, int max_pages, int page_size, hipStream_t st, int S, size_t slice) {
    QH_REQUIRE(qkv && pos && rope && q_out && kc && vc && page_table && n > 0 && hd % 2 == 0 && S >= 1,
               QRAF_HIP_ERR_INVALID, "rope_append: bad arguments");
    if (kv_dtype == DT_I8) {
        QH_REQUIRE(hd <= 128 && hd % 4 == 0 && page_size % 4 == 0, QRAF_HIP_ERR_INVALID,
                   "rope_append: int8 pages need head_dim <= 128 (multiple of 4) and page_size %% 4 == 0");
        const int qblocks = std::min(8, (H * hd / 2 + 255) / 256);
        hipLaunchKernelGGL(rope_append_i8_kernel, dim3(n, 1 + qblocks), dim3(256), 0, st, qkv, bias, H, Hkv, hd, pos,
                           rope, q_out, (int8_t*)kc, (int8_t*)vc, page_table, max_pages, page_size, S, slice);
        QH_CHECK_HIP(hipGetLastError());
        return QRAF_HIP_OK;
    }
    const size_t work = (size_t)n * ((H * hd + Hkv * hd) / 2 + Hkv * hd);
    const int grid = (int)std::min<size_t>((work + 255) / 256, 4096);
    if (kv_dtype != DT_F32 && kv_dtype != DT_F16) return set_error(QRAF_HIP_ERR_DTYPE, "rope_append: KV dtype %u", kv_dtype);
#define QH_RA(KTv, SCv)                                                                                              \
    hipLaunchKernelGGL((rope_append_kernel<KTv, SCv>), dim3(grid), dim3(256), 0, st, qkv, bias, H, Hkv, hd, pos, rope, \
                       q_out, (KTv*)kc, (KTv*)vc, page_table, max_pages, page_size, n, S, slice)
#define QH_RA_S(KTv)                  \
    switch (S) {                      \
        case 1: QH_RA(KTv, 1); break; \
        case 2: QH_RA(KTv, 2); break; \
        case 4: QH_RA(KTv, 4); break; \
        case 8: QH_RA(KTv, 8); break; \
        default: QH_RA(KTv, 0); break; \
    }
    if (kv_dtype == DT_F32) {
        QH_RA_S(float)
    } else {
        QH_RA_S(_Float16)
    }
#undef QH_RA_S
#undef QH_RA
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

// ---------------------------------------------------------------------------
// Workspace of the no-allocation entry point (qraf_hip_paged_attention_noalloc_dev):
// a file-scope device array, one copy per GPU, held until the process ends.
// Host code never passes the array's name to a kernel (on the host it names a
// stand-in, not device memory): qraf_hip_init resolves the array's device
// address once per device with hipGetSymbolAddress, and only that address is
// used afterwards.  Every call on one GPU shares the array; it keeps the last
// call's contents, and nothing in it must start at zero (every partial a
// merge reads is written earlier in the same call).
// ---------------------------------------------------------------------------
constexpr size_t ATTN_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[ATTN_SCRATCH_BYTES];
constexpr int ATTN_SCRATCH_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[ATTN_SCRATCH_DEVICES];

int attn_scratch_init(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    QH_REQUIRE(device >= 0 && device < ATTN_SCRATCH_DEVICES, QRAF_HIP_ERR_INVALID,
               "attention scratch: device %d beyond %d", device, ATTN_SCRATCH_DEVICES);
    if (g_scratch_ptr[device]) return QRAF_HIP_OK;
    void* p = nullptr;
    QH_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    QH_REQUIRE(p, QRAF_HIP_ERR_HIP, "attention scratch: no device address on device %d", device);
    g_scratch_ptr[device] = p;
    return QRAF_HIP_OK;
}

static void* attn_scratch(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return device >= 0 && device < ATTN_SCRATCH_DEVICES ? g_scratch_ptr[device] : nullptr;
}

}  // namespace qraf_hip

extern "C" {

int qraf_hip_paged_attention_noalloc_dev(const float* q, const void* k_cache, const void* v_cache, uint32_t kv_dtype,
                                         const int32_t* page_table, int32_t max_pages_per_seq, const int32_t* ctx_lens,
                                         int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                         int32_t page_size, float scale, int32_t max_ctx, float* out, void* stream) {
    qraf_hip::clear_error();
    QH_REQUIRE(n_seqs > 0 && n_seqs <= 1024 && n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && max_ctx > 0,
               QRAF_HIP_ERR_INVALID, "attention: bad shape (n_seqs %d, heads %d / %d, head_dim %d, max_ctx %d)",
               n_seqs, n_heads, n_kv_heads, head_dim, max_ctx);
    const size_t need = qraf_hip::attn_workspace_bytes(n_seqs, n_heads, n_kv_heads, head_dim, max_ctx);
    QH_REQUIRE(need <= qraf_hip::ATTN_SCRATCH_BYTES, QRAF_HIP_ERR_INVALID,
               "attention (no-allocation form): this shape needs %zu bytes of workspace, the scratch holds %zu "
               "(n_seqs %d, heads %d, head_dim %d, max_ctx %d)",
               need, qraf_hip::ATTN_SCRATCH_BYTES, n_seqs, n_heads, head_dim, max_ctx);
    int dev = 0;
    QH_CHECK_HIP(hipGetDevice(&dev));
    void* ws = qraf_hip::attn_scratch(dev);
    QH_REQUIRE(ws, QRAF_HIP_ERR_STATE, "attention (no-allocation form): qraf_hip_init was not called on device %d",
               dev);
    return qraf_hip::launch_attention(q, k_cache, v_cache, kv_dtype, page_table, max_pages_per_seq, ctx_lens, n_seqs,
                                      n_heads, n_kv_heads, head_dim, page_size, scale, max_ctx, out, ws,
                                      qraf_hip::ATTN_SCRATCH_BYTES, qraf_hip::as_stream(stream));
}

uint64_t qraf_hip_attention_noalloc_max_bytes(void) { return qraf_hip::ATTN_SCRATCH_BYTES; }

int qraf_hip_set_attention_tuning(int32_t form) {
    qraf_hip::clear_error();
    QH_REQUIRE(form >= 0 && form <= 3, QRAF_HIP_ERR_INVALID, "attention tuning: form %d", form);
    if (qraf_hip::g_attn_form != form) {
        qraf_hip::g_attn_form = form;
        qraf_hip::bump_tuning_generation();  // captured engine steps are rebuilt with the new form
    }
    return QRAF_HIP_OK;
}

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
