// sampler.hip -- Sampler on the device: repetition penalty, greedy argmax,
// temperature + top-k + top-p sampling, for many rows of logits at once.
//
// Replaces Sampler::apply_repetition_penalty (reference
// src/sampling/sampler.cpp:37-49) and Sampler::sample (:57-128) so that a
// decode step's logits never leave HBM.  The uniform draw of each sampled row
// comes from the caller (the reference draws it from its std::mt19937 member;
// the host layer reproduces that stream), so the device work is a pure
// function of (logits, recent tokens, parameters, uniform).
//
// Sampling a row (one workgroup of 1024 threads):
//   1. probs p_i = logit_i / T, computed where used (the reference's vector).
//   2. The cutoff-th largest p by radix select over order-preserving 32-bit
//      keys, 8 bits per pass (4 passes, LDS histograms).
//   3. The cutoff candidates (keys above the selected one, then the lowest
//      indices of equal keys) gathered in index order, then bitonic-sorted in
//      LDS by (p descending, index ascending).  The reference's std::sort
//      leaves the order of equal p unspecified; this order is one of its
//      possible results.
//   4. The reference's arithmetic on the sorted candidates in its order:
//      exp(p - max) and the divisions elementwise (all threads), the
//      sequential sums, top-p prefix, renormalisation and the cumulative sum
//      against the uniform by one thread.
// cutoff = top_k when 0 < top_k < vocab, else vocab (sampler.cpp:73-77).
// cutoff <= CAND_CAP takes the steps above.  cutoff = vocab > that
// (top_k 0, the whole vocabulary) takes the absorbed-tail path: in the
// reference's descending order the running sum only grows, so once a term
// exp(p - max) is below half an ulp of the running sum it and every later
// term leave every sum unchanged.  With S = sum_i exp(p_i - max) (a parallel
// estimate), every token with exp(p - max) >= S * 2^-28 is gathered (the
// terms that can change a sum, with a 2^3 margin: a term below S * 2^-25 is
// below half an ulp of a running sum >= S / 2 ... and the running sum there
// is >= S (1 - V 2^-28)); the reference's loops over the vocabulary then
// equal the same loops over the gathered candidates, except that its
// fallback (no cumulative sum reaches the uniform) is its last sorted token,
// the smallest p (largest index among equal p in this order).
//
// Rows whose candidates do not fit in LDS (a whole-vocabulary row whose
// gathered set exceeds CAND_CAP, or CAND_CAP < top_k < vocab) keep their
// (p, index) pairs in a per-row region of global sort storage: every pair
// of the row (whole vocabulary), or the top_k pairs of step 2 gathered in
// index order.  A stable LSD radix sort over the order-preserving keys (4
// passes of 8 bits, descending digit order) sorts them by p descending with
// equal p in index order, the LDS path's order; the reference's loops then
// run over the sorted pairs, staged through LDS CAND_CAP at a time for the
// sequential sums.
#include <math.h>

#include <mutex>

#include "common.h"

namespace qraf_hip {

constexpr int CAND_CAP = 4096;  // candidates gathered and sorted in LDS at most

constexpr int SNT = 1024;  // threads per row (16 waves)

// Row loops: each thread reads 4 float4 (16 logits) before using any, so a
// workgroup has 16K logits in flight per round trip; f(i, value) is called
// for every i < V, in increasing i within a thread.
template <typename F>
__device__ __forceinline__ void for_row(const float* __restrict__ l, int V, int tid, F&& f) {
    if ((V & 3) == 0) {
        const int V4 = V >> 2;
        const float4* l4 = (const float4*)l;
        for (int base = tid; base < V4; base += SNT * 4) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = l4[min(base + SNT * u, V4 - 1)];
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (base + SNT * u < V4) {
                    const int i = 4 * (base + SNT * u);
                    f(i, v[u].x);
                    f(i + 1, v[u].y);
                    f(i + 2, v[u].z);
                    f(i + 3, v[u].w);
                }
        }
    } else {
        for (int base = tid; base < V; base += SNT * 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = l[min(base + SNT * u, V - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (base + SNT * u < V) f(base + SNT * u, v[u]);
        }
    }
}

// order-preserving key: a < b  <=>  key(a) < key(b) for non-NaN floats
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Sampler::apply_repetition_penalty: one thread per row, the row's recent
// tokens in order (a token listed twice is penalised twice, as in the loop);
// for histories longer than PEN_LDS
__global__ void penalty_rows_kernel(float* __restrict__ logits, int V, int rows, const uint32_t* __restrict__ recent,
                                    const int32_t* __restrict__ counts, int stride, float penalty) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    float* l = logits + (size_t)row * V;
    const uint32_t* r = recent + (size_t)row * stride;
    const int n = min(counts[row], stride);
    for (int i = 0; i < n; i++) {
        const uint32_t tok = r[i];
        if (tok >= (uint32_t)V) continue;
        const float v = l[tok];
        l[tok] = v > 0.f ? v / penalty : v * penalty;
    }
}

// The same, one workgroup per row for histories of at most PEN_LDS tokens:
// the history is sorted in LDS, and the first thread of each run of one
// token applies the penalty run-length times to that token.  Distinct
// tokens are independent and a token's value keeps its sign, so this equals
// the sequential loop.
constexpr int PEN_LDS = 4096;
__global__ __launch_bounds__(256) void penalty_rows_lds_kernel(float* __restrict__ logits, int V,
                                                               const uint32_t* __restrict__ recent,
                                                               const int32_t* __restrict__ counts, int stride,
                                                               float penalty) {
    __shared__ uint32_t s[PEN_LDS];
    const int row = blockIdx.x, tid = threadIdx.x;
    float* l = logits + (size_t)row * V;
    const uint32_t* r = recent + (size_t)row * stride;
    const int n = min(counts[row], stride);
    int P = 1;
    while (P < n) P <<= 1;
    for (int i = tid; i < P; i += 256) s[i] = i < n ? r[i] : 0xFFFFFFFFu;  // padding sorts last, is >= V
    __syncthreads();
    for (int k = 2; k <= P; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < P; i += 256) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint32_t a = s[i], b = s[ixj];
                    if ((a > b) == ((i & k) == 0)) {
                        s[i] = b;
                        s[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    for (int i = tid; i < n; i += 256) {
        const uint32_t tok = s[i];
        if (tok >= (uint32_t)V || (i > 0 && s[i - 1] == tok)) continue;
        int c = 1;
        while (i + c < n && s[i + c] == tok) c++;
        float v = l[tok];
        for (int k = 0; k < c; k++) v = v > 0.f ? v / penalty : v * penalty;
        l[tok] = v;
    }
}

// Stable LSD radix sort of n (p, index) pairs in global memory by p
// descending, one workgroup: 4 passes of 8 key bits, each a histogram, an
// exclusive scan and a scatter of SNT-pair tiles in pair order.  Within a
// tile, a pair's rank among the earlier pairs of its digit is its rank among
// its wave's lanes of that digit (lanes with the same digit found by 8
// ballots, one per digit bit) plus the counts of that digit in the earlier
// waves.  The pairs end in (pa, ia); (pb, ib) is the other buffer.
// Waves of one workgroup share the CU's write-through L1, so a barrier
// orders their global stores and loads.
__device__ void radix_sort_pairs(float* pa, int* ia, float* pb, int* ib, int n, uint32_t* hist, int (*wcnt)[256],
                                 int (*base)[256]) {
    constexpr int NW = SNT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t below = (1ull << lane) - 1;
    float* sp = pa;
    int* si = ia;
    float* dp = pb;
    int* di = ib;
    for (int shift = 0; shift < 32; shift += 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += SNT) atomicAdd(&hist[255u - ((order_key(sp[i]) >> shift) & 255u)], 1u);
        __syncthreads();
        if (tid == 0) {
            int acc = 0;
            for (int d = 0; d < 256; d++) {
                base[0][d] = acc;
                acc += (int)hist[d];
            }
        }
        __syncthreads();
        int cur = 0;
        float np_ = tid < n ? sp[tid] : 0.f;  // the next tile's pair, requested a tile ahead
        int ni = tid < n ? si[tid] : 0;
        for (int t0 = 0; t0 < n; t0 += SNT) {
            const int i = t0 + tid;
            const bool ok = i < n;
            const float p = np_;
            const int ix = ni;
            if (t0 + SNT + tid < n) {
                np_ = sp[t0 + SNT + tid];
                ni = si[t0 + SNT + tid];
            }
            const uint32_t d = 255u - ((order_key(p) >> shift) & 255u);
            uint64_t peers = __ballot(ok);
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint64_t m = __ballot((d >> b) & 1u);
                peers &= ((d >> b) & 1u) ? m : ~m;
            }
#pragma unroll
            for (int k = 0; k < 4; k++) wcnt[wave][lane + 64 * k] = 0;  // the wave's own row: no barrier
            if (ok && (peers & below) == 0) wcnt[wave][d] = __popcll(peers);
            __syncthreads();
            if (ok) {
                int off = base[cur][d] + __popcll(peers & below);
                for (int w = 0; w < wave; w++) off += wcnt[w][d];
                dp[off] = p;
                di[off] = ix;
            }
            if (tid < 256) {
                int c = 0;
#pragma unroll
                for (int w = 0; w < NW; w++) c += wcnt[w][tid];
                base[cur ^ 1][tid] = base[cur][tid] + c;
            }
            cur ^= 1;
            __syncthreads();
        }
        float* tp = sp;
        sp = dp;
        dp = tp;
        int* ti = si;
        si = di;
        di = ti;
    }
}

// The reference's loops (sampler.cpp:79-127) over n sorted pairs in global
// memory: exponentials and divisions elementwise by all threads, the
// sequential sums by thread 0 over LDS-staged chunks of CAND_CAP, stopping
// at the chunk where a cumulative sum reaches its bound.  Returns the token
// (thread 0's value is the one used).
__device__ uint32_t sorted_pairs_pick(float* pv, const int* iv, int n, float top_p, float r, float* stage,
                                      float* s_val, int* s_pos) {
    const int tid = threadIdx.x;
    const float max_val = pv[0];
    __syncthreads();
    for (int i = tid; i < n; i += SNT) pv[i] = expf(pv[i] - max_val);
    __syncthreads();
    // sequential sum (or first reach of `bound`) over pv[0..m): thread 0's
    // running sum over staged chunks; pos = index where cs >= bound, or -1
    auto scan = [&](int m, float bound, bool stop_ge, float& total, int& pos) {
        float cs = 0.f;
        int at = -1;
        for (int c0 = 0; c0 < m; c0 += CAND_CAP) {
            const int cn = min(CAND_CAP, m - c0);
            for (int j = tid; j < cn; j += SNT) stage[j] = pv[c0 + j];
            __syncthreads();
            if (tid == 0) {
                for (int j = 0; j < cn; j++) {
                    cs += stage[j];
                    if (stop_ge ? cs >= bound : bound <= cs) {
                        at = c0 + j;
                        break;
                    }
                }
                *s_val = cs;
                *s_pos = at;
            }
            __syncthreads();
            cs = *s_val;
            at = *s_pos;
            __syncthreads();
            if (at >= 0) break;
        }
        total = cs;
        pos = at;
    };
    float sum;
    int unused;
    scan(n, INFINITY, true, sum, unused);  // cs >= inf never holds: the whole sum
    for (int i = tid; i < n; i += SNT) pv[i] /= sum;
    __syncthreads();
    int m = n;
    if (top_p > 0.f && top_p < 1.f) {
        // the nucleus sum is the same additions as the cumulative sum up to
        // and including the nucleus' last term (both start from 0)
        float ns;
        int at;
        scan(n, top_p, true, ns, at);
        m = at < 0 ? n : at + 1;
        for (int i = tid; i < m; i += SNT) pv[i] /= ns;
        __syncthreads();
    }
    float cs;
    int at;
    scan(m, r, false, cs, at);
    return (uint32_t)iv[at < 0 ? m - 1 : at];
}

__global__ __launch_bounds__(SNT) void sample_rows_kernel(const float* __restrict__ logits, int V, float T, int cutoff,
                                                          float top_p, const float* __restrict__ uniforms,
                                                          uint32_t* __restrict__ out, float* __restrict__ sort_ws) {
    const int tid = threadIdx.x, row = blockIdx.x;
    const float* l = logits + (size_t)row * V;
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_prefix, s_need;
    __shared__ int s_cgt[SNT], s_ceq[SNT];
    __shared__ float cval[CAND_CAP];
    __shared__ int cidx[CAND_CAP];
    constexpr int NW = SNT / 64;
    __shared__ float s_red[2][NW];
    __shared__ int s_cnt[NW][8];
    __shared__ int s_n;
    __shared__ int s_wcnt[NW][256], s_base[2][256];  // the global sort
    __shared__ float s_sv;
    __shared__ int s_sp;

    if (!(T > 0.f)) {  // Sampler::argmax (sampler.cpp:25-35): first index of the maximum
        float best = -INFINITY;
        int bi = V;
        for_row(l, V, tid, [&](int i, float v) {  // increasing i per thread
            if (bi == V || v > best) {
                best = v;
                bi = i;
            }
        });
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(best, o);
            const int oi = __shfl_xor(bi, o);
            if (ov > best || (ov == best && oi < bi)) {
                best = ov;
                bi = oi;
            }
        }
        __shared__ float wv[NW];
        __shared__ int wi[NW];
        if ((tid & 63) == 0) {
            wv[tid >> 6] = best;
            wi[tid >> 6] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < NW; w++)
                if (wv[w] > best || (wv[w] == best && wi[w] < bi)) {
                    best = wv[w];
                    bi = wi[w];
                }
            out[row] = (uint32_t)(bi < V ? bi : 0);
        }
        return;
    }

    // ---- the whole vocabulary (cutoff = V > CAND_CAP): gather the tokens
    // whose terms are not absorbed (see the file comment); more than
    // CAND_CAP of them, or CAND_CAP < top_k < V: the global sort
    const bool trunc = cutoff == V && cutoff > CAND_CAP;
    bool big = cutoff != V && cutoff > CAND_CAP;
    __shared__ uint32_t s_last;  // trunc: the reference's last sorted token
    int nsort = cutoff;
    bool fast = cutoff == V;  // every token a candidate
    float t = -INFINITY;
    // the row's sort storage: pairs (pa, ia), the radix sort's other buffer (pb, ib)
    float* pa = sort_ws + (size_t)row * 4 * V;
    int* ia = (int*)(pa + V);
    float* pb = pa + 2 * (size_t)V;
    int* ib = (int*)(pa + 3 * (size_t)V);
    if (trunc) {
        float mx = -INFINITY, mn = INFINITY;
        int imn = -1;
        for_row(l, V, tid, [&](int i, float v) {  // increasing i per thread
            const float p = v / T;
            mx = fmaxf(mx, p);
            if (imn < 0 || p <= mn) {  // the smallest p, largest index among equal
                mn = p;
                imn = i;
            }
        });
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            mx = fmaxf(mx, __shfl_xor(mx, o));
            const float omn = __shfl_xor(mn, o);
            const int oi = __shfl_xor(imn, o);
            if (omn < mn || (omn == mn && oi > imn)) {
                mn = omn;
                imn = oi;
            }
        }
        __shared__ float wmn[NW];
        __shared__ int wimn[NW];
        if ((tid & 63) == 0) {
            s_red[0][tid >> 6] = mx;
            wmn[tid >> 6] = mn;
            wimn[tid >> 6] = imn;
        }
        __syncthreads();
        for (int w = 0; w < NW; w++) {
            mx = fmaxf(mx, s_red[0][w]);
            if (wmn[w] < mn || (wmn[w] == mn && wimn[w] > imn)) {
                mn = wmn[w];
                imn = wimn[w];
            }
        }
        if (tid == 0) s_last = (uint32_t)imn;
        float S = 0.f;
        for_row(l, V, tid, [&](int, float v) { S += __expf(v / T - mx); });
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) S += __shfl_xor(S, o);
        __syncthreads();  // the reads of s_red above are done
        if ((tid & 63) == 0) s_red[1][tid >> 6] = S;
        __syncthreads();
        S = 0.f;
        for (int w = 0; w < NW; w++) S += s_red[1][w];
        t = mx + logf(S) - 28.0f * 0.69314718f;  // exp(p - max) >= S * 2^-28
        int c = 0;
        for_row(l, V, tid, [&](int, float v) { c += v / T >= t; });
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o);
        if ((tid & 63) == 0) s_cnt[tid >> 6][0] = c;
        __syncthreads();
        c = 0;
        for (int w = 0; w < NW; w++) c += s_cnt[w][0];
        big = c > CAND_CAP;
        fast = !big;  // gather p >= t below, or sort every pair
    }

    // ---- fast path: a threshold t with cutoff <= #{p >= t} <= CAND_CAP, by an
    // 8-way search between the row's smallest and largest p; then every
    // p >= t is gathered and sorted.  The sort makes the result independent
    // of the gather order, and equal to the radix path's.
    if (!fast && !big) {
        float mx = -INFINITY, mn = INFINITY;
        for_row(l, V, tid, [&](int, float v) {
            const float p = v / T;
            mx = fmaxf(mx, p);
            mn = fminf(mn, p);
        });
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            mx = fmaxf(mx, __shfl_xor(mx, o));
            mn = fminf(mn, __shfl_xor(mn, o));
        }
        if ((tid & 63) == 0) {
            s_red[0][tid >> 6] = mx;
            s_red[1][tid >> 6] = mn;
        }
        __syncthreads();
        for (int w = 0; w < NW; w++) {
            mx = fmaxf(mx, s_red[0][w]);
            mn = fminf(mn, s_red[1][w]);
        }
        const int target = max(2 * cutoff, 512);
        if (mx > mn && mx < INFINITY && mn > -INFINITY) {
            float lo = mn, hi = mx;  // #{p >= lo} = V >= cutoff
            int clo = V;
            for (int pass = 0; pass < 16 && clo > target; pass++) {
                float th[8];
#pragma unroll
                for (int j = 0; j < 8; j++) th[j] = lo + (hi - lo) * ((float)(j + 1) / 9.0f);
                int c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for_row(l, V, tid, [&](int, float v) {
                    const float p = v / T;
#pragma unroll
                    for (int j = 0; j < 8; j++) c[j] += p >= th[j];
                });
#pragma unroll
                for (int j = 0; j < 8; j++) {
#pragma unroll
                    for (int o = 32; o >= 1; o >>= 1) c[j] += __shfl_xor(c[j], o);
                }
                __syncthreads();  // the previous pass's reads of s_cnt are done
                if ((tid & 63) == 0) {
#pragma unroll
                    for (int j = 0; j < 8; j++) s_cnt[tid >> 6][j] = c[j];
                }
                __syncthreads();
                int jb = -1, cb = clo;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    int cj = 0;
                    for (int w = 0; w < NW; w++) cj += s_cnt[w][j];
                    if (cj >= cutoff) {
                        jb = j;
                        cb = cj;
                    }
                }
                const float nlo = jb >= 0 ? th[jb] : lo, nhi = jb < 7 ? th[jb + 1] : hi;
                if (!(nlo > lo || nhi < hi)) break;  // no progress: values too close together
                lo = nlo;
                hi = nhi;
                clo = cb;
            }
            if (clo <= CAND_CAP) {
                fast = true;
                t = lo;
                nsort = clo;
            }
        }
    }
    if (fast) {
        if (tid == 0) s_n = 0;
        __syncthreads();
        for_row(l, V, tid, [&](int i, float v) {
            const float p = v / T;
            if (p >= t) {
                const int k = atomicAdd(&s_n, 1);
                cval[k] = p;
                cidx[k] = i;
            }
        });
        __syncthreads();
        nsort = s_n;
    } else if (big && trunc) {  // every pair of the row, in index order
        for (int i = tid; i < V; i += SNT) {
            pa[i] = l[i] / T;
            ia[i] = i;
        }
        nsort = V;
    } else {
    // ---- radix select of the cutoff-th largest key
    uint32_t prefix = 0, mask = 0, need = (uint32_t)cutoff;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for_row(l, V, tid, [&](int, float v) {
            const uint32_t k = order_key(v / T);
            if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (tid == 0) {
            uint32_t acc = 0;
            int d = 255;
            for (; d > 0; d--) {
                if (acc + hist[d] >= need) break;
                acc += hist[d];
            }
            s_prefix = prefix | ((uint32_t)d << shift);
            s_need = need - acc;
        }
        __syncthreads();
        prefix = s_prefix;
        need = s_need;
        mask |= 255u << shift;
        __syncthreads();
    }
    const uint32_t tau = prefix;          // key of the cutoff-th largest p
    const int n_gt = cutoff - (int)need;  // candidates strictly above it

    // ---- gather in index order: thread t owns [t*ch, (t+1)*ch); into LDS,
    // or the row's sort storage
    float* gv = big ? pa : cval;
    int* gi = big ? ia : cidx;
    const int ch = (V + SNT - 1) / SNT;
    const int lo = min(V, tid * ch), hi = min(V, lo + ch);
    int gt = 0, eq = 0;
    for (int i = lo; i < hi; i++) {
        const uint32_t k = order_key(l[i] / T);
        gt += k > tau;
        eq += k == tau;
    }
    s_cgt[tid] = gt;
    s_ceq[tid] = eq;
    __syncthreads();
    if (tid == 0) {  // exclusive prefix sums, in thread (index) order
        int a = 0, b = 0;
        for (int t = 0; t < SNT; t++) {
            const int x = s_cgt[t], y = s_ceq[t];
            s_cgt[t] = a;
            s_ceq[t] = b;
            a += x;
            b += y;
        }
    }
    __syncthreads();
    int pg = s_cgt[tid], pe = s_ceq[tid];
    for (int i = lo; i < hi; i++) {
        const float p = l[i] / T;
        const uint32_t k = order_key(p);
        if (k > tau) {
            gv[pg] = p;
            gi[pg] = i;
            pg++;
        } else if (k == tau) {
            if (pe < (int)need) {
                gv[n_gt + pe] = p;
                gi[n_gt + pe] = i;
            }
            pe++;
        }
    }
    }  // radix path
    if (big) {  // global sort, then the reference's loops over the sorted pairs
        __syncthreads();
        radix_sort_pairs(pa, ia, pb, ib, nsort, hist, s_wcnt, s_base);
        const uint32_t pick = sorted_pairs_pick(pa, ia, nsort, top_p, uniforms[row], cval, &s_sv, &s_sp);
        if (tid == 0) out[row] = pick;
        return;
    }
    int P = 1;
    while (P < nsort) P <<= 1;
    for (int i = nsort + tid; i < P; i += SNT) {
        cval[i] = -INFINITY;
        cidx[i] = 0x7FFFFFFF;
    }
    __syncthreads();

    // ---- bitonic sort: p descending, index ascending
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < P; i += SNT) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const float a = cval[i], b = cval[ixj];
                    const int ia = cidx[i], ib = cidx[ixj];
                    const bool a_first = a > b || (a == b && ia < ib);
                    const bool up = (i & k) == 0;  // this half ends in "first" order
                    if (a_first != up) {
                        cval[i] = b;
                        cval[ixj] = a;
                        cidx[i] = ib;
                        cidx[ixj] = ia;
                    }
                }
            }
            __syncthreads();
        }
    }

    // ---- the reference's arithmetic, in its order (sampler.cpp:79-127);
    // exponentials and divisions are elementwise, so all threads take them
    const int nc = trunc ? nsort : cutoff;  // the candidates the loops run over
    __shared__ float s_sum;
    __shared__ int s_nucleus;
    const float max_val = cval[0];
    __syncthreads();
    for (int i = tid; i < nc; i += SNT) cval[i] = expf(cval[i] - max_val);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.f;
        for (int i = 0; i < nc; i++) sum += cval[i];
        s_sum = sum;
    }
    __syncthreads();
    const float sum = s_sum;
    for (int i = tid; i < nc; i += SNT) cval[i] /= sum;
    __syncthreads();
    const bool topp = top_p > 0.f && top_p < 1.f;
    if (topp && tid == 0) {
        float cs = 0.f;
        int nucleus = -1;  // -1: the prefix never reaches top_p (the whole list)
        for (int i = 0; i < nc; i++) {
            cs += cval[i];
            if (cs >= top_p) {
                nucleus = i + 1;
                break;
            }
        }
        const int m = nucleus < 0 ? nc : nucleus;
        float ns = 0.f;
        for (int i = 0; i < m; i++) ns += cval[i];
        s_sum = ns;
        s_nucleus = nucleus;
    }
    __syncthreads();
    int nucleus = -1;
    if (topp) {
        nucleus = s_nucleus;
        const int m = nucleus < 0 ? nc : nucleus;
        const float ns = s_sum;
        for (int i = tid; i < m; i += SNT) cval[i] /= ns;
        __syncthreads();
    }
    if (tid == 0) {
        const int n = nucleus < 0 ? nc : nucleus;
        const float r = uniforms[row];
        float cs = 0.f;
        // fallback: the reference's last candidate; with an absorbed tail and
        // no nucleus that is its last sorted token of the whole vocabulary
        uint32_t pick = trunc && nucleus < 0 ? s_last : (uint32_t)cidx[n - 1];
        for (int i = 0; i < n; i++) {
            cs += cval[i];
            if (r <= cs) {
                pick = (uint32_t)cidx[i];
                break;
            }
        }
        out[row] = pick;
    }
}

size_t sample_sort_bytes(int rows, int V, const qraf_sampling_params& sp) {
    const bool greedy = !(sp.temperature > 0.f);
    const int cutoff = (sp.top_k > 0 && sp.top_k < V) ? sp.top_k : V;
    return greedy || cutoff <= CAND_CAP ? 0 : (size_t)rows * V * 16;
}

int launch_sample(float* logits, int rows, int V, const qraf_sampling_params& sp, const uint32_t* recent,
                  const int32_t* counts, int stride, const float* uniforms, uint32_t* out, void* sort_ws,
                  size_t sort_bytes, hipStream_t s) {
    QH_REQUIRE(logits && out && rows > 0 && V > 0, QRAF_HIP_ERR_INVALID, "sample: bad arguments");
    const bool greedy = !(sp.temperature > 0.f);
    const int cutoff = (sp.top_k > 0 && sp.top_k < V) ? sp.top_k : V;
    QH_REQUIRE(greedy || uniforms, QRAF_HIP_ERR_INVALID, "sample: temperature %g needs uniforms", sp.temperature);
    QH_REQUIRE(sort_bytes >= sample_sort_bytes(rows, V, sp) && (sort_ws || !sample_sort_bytes(rows, V, sp)),
               QRAF_HIP_ERR_INVALID, "sample: sort storage of %zu bytes, %zu needed", sort_bytes,
               sample_sort_bytes(rows, V, sp));
    (void)cutoff;
    if (sp.repetition_penalty != 1.0f) {  // sampler.cpp:39
        QH_REQUIRE(!recent || (counts && stride > 0), QRAF_HIP_ERR_INVALID, "sample: recent tokens need counts");
        if (recent) {
            if (stride <= PEN_LDS)
                hipLaunchKernelGGL(penalty_rows_lds_kernel, dim3(rows), dim3(256), 0, s, logits, V, recent, counts,
                                   stride, sp.repetition_penalty);
            else
                hipLaunchKernelGGL(penalty_rows_kernel, dim3((rows + 63) / 64), dim3(64), 0, s, logits, V, rows,
                                   recent, counts, stride, sp.repetition_penalty);
            QH_CHECK_HIP(hipGetLastError());
        }
    }
    hipLaunchKernelGGL(sample_rows_kernel, dim3(rows), dim3(SNT), 0, s, logits, V, sp.temperature, cutoff, sp.top_p,
                       uniforms, out, (float*)sort_ws);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip

using namespace qraf_hip;

// Sort storage of qraf_hip_sample_dev, per device, grown on demand and held
// until the process ends.
namespace {
std::mutex g_sort_mu;
void* g_sort_ws[64];
size_t g_sort_bytes[64];
}  // namespace

extern "C" int qraf_hip_sample_dev(float* logits, int32_t rows, int32_t vocab, const qraf_sampling_params* params,
                                   const uint32_t* recent, const int32_t* recent_count, int32_t recent_stride,
                                   const float* uniforms, uint32_t* tokens, void* stream) {
    clear_error();
    QH_REQUIRE(params && rows > 0 && vocab > 0, QRAF_HIP_ERR_INVALID, "sample: bad arguments");
    const size_t need = sample_sort_bytes(rows, vocab, *params);
    void* ws = nullptr;
    if (need) {
        int dev = 0;
        QH_CHECK_HIP(hipGetDevice(&dev));
        QH_REQUIRE(dev >= 0 && dev < 64, QRAF_HIP_ERR_INVALID, "sample: device %d", dev);
        std::lock_guard<std::mutex> lk(g_sort_mu);
        if (g_sort_bytes[dev] < need) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            QH_CHECK_HIP(hipStreamIsCapturing(as_stream(stream), &cs));
            QH_REQUIRE(cs == hipStreamCaptureStatusNone, QRAF_HIP_ERR_STATE,
                       "sample: the sort storage (%zu bytes) is allocated by a first call outside stream capture",
                       need);
            if (g_sort_ws[dev]) QH_CHECK_HIP(hipFree(g_sort_ws[dev]));  // waits for work that may use it
            g_sort_ws[dev] = nullptr;
            g_sort_bytes[dev] = 0;
            QH_CHECK_HIP(hipMalloc(&g_sort_ws[dev], need));
            g_sort_bytes[dev] = need;
        }
        ws = g_sort_ws[dev];
    }
    return launch_sample(logits, rows, vocab, *params, recent, recent_count, recent_stride, uniforms, tokens, ws,
                         need, as_stream(stream));
}
