/*
 * oracle.c -- CPU restatement of QRAF's scalar x86 decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Reference citations are
 * file:line in simonpierreboucher02/qraf.
 *
 * Build: gcc -std=gnu11 -O3 -ffp-contract=off (no -march: baseline x86-64,
 * as the reference's Release build, CMakeLists.txt:18-22), so every
 * `a += b * c` below rounds the product and the sum separately, exactly as
 * the reference's scalar loops do.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------- fp16 (dtype.cpp:9-59) ---------------- */

float or_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, r;
    if (ex == 0) {
        if (mant == 0) {
            r = sign << 31;
        } else { /* subnormal: renormalise */
            int e = 1;
            while (!(mant & 0x400u)) { mant <<= 1; e--; }
            mant &= 0x3FFu;
            r = (sign << 31) | ((uint32_t)(e + 127 - 15) << 23) | (mant << 13);
        }
    } else if (ex == 31) {
        r = (sign << 31) | 0x7F800000u | (mant << 13);
    } else {
        r = (sign << 31) | ((ex + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &r, 4);
    return f;
}

/* truncating, flush-to-zero, overflow (and NaN) -> inf: dtype.cpp:39-59 */
uint16_t or_fp32_to_fp16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t sign = (bits >> 31) & 1u;
    int32_t ex = (int32_t)((bits >> 23) & 0xFFu) - 127;
    uint32_t mant = bits & 0x7FFFFFu;
    if (ex > 15) return (uint16_t)((sign << 15) | 0x7C00u);
    if (ex > -15) return (uint16_t)((sign << 15) | ((uint32_t)(ex + 15) << 10) | (mant >> 13));
    return (uint16_t)(sign << 15);
}

/* ---------------- block geometry ---------------- */

size_t or_q_block_bytes(uint32_t dtype, int bs) {
    if (dtype == OR_Q8_0) return 4 + (size_t)bs;       /* quantize.cpp:107 */
    if (dtype == OR_Q4_0) return 2 + (size_t)(bs / 2); /* quantize.cpp:146 */
    return 0;
}

size_t or_q_tensor_bytes(uint32_t dtype, size_t count, int bs) {
    if (dtype == OR_F32) return count * 4;
    if (dtype == OR_F16) return count * 2;
    return ((count + bs - 1) / bs) * or_q_block_bytes(dtype, bs);
}

/* std::min(hi, v) / std::max(lo, v) with the reference's argument order, so
 * NaN resolves the way libstdc++ resolves it (quantize.cpp:133, :173). */
static inline float std_min(float a, float b) { return (b < a) ? b : a; }
static inline float std_max(float a, float b) { return (a < b) ? b : a; }

/* ---------------- quantizers ---------------- */

/* quantize.cpp:105-140 */
size_t or_quantize_q8_0(const float* data, size_t count, int bs, uint8_t* out) {
    size_t nb = (count + bs - 1) / bs, bb = 4 + (size_t)bs;
    memset(out, 0, nb * bb);
    for (size_t b = 0; b < nb; b++) {
        size_t off = b * (size_t)bs;
        int tb = (int)((size_t)bs < count - off ? (size_t)bs : count - off);
        float max_abs = 0.0f;
        for (int i = 0; i < tb; i++) {
            float a = fabsf(data[off + i]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 127.0f;
        float inv = (scale > 0.0f) ? 1.0f / scale : 0.0f;
        uint8_t* blk = out + b * bb;
        memcpy(blk, &scale, 4);
        int8_t* q = (int8_t*)(blk + 4);
        for (int i = 0; i < tb; i++) {
            float v = data[off + i] * inv;
            v = std_max(-127.0f, std_min(127.0f, v));
            q[i] = (int8_t)roundf(v);
        }
    }
    return nb * bb;
}

/* quantize.cpp:144-183 */
size_t or_quantize_q4_0(const float* data, size_t count, int bs, uint8_t* out) {
    size_t nb = (count + bs - 1) / bs, bb = 2 + (size_t)(bs / 2);
    memset(out, 0, nb * bb);
    for (size_t b = 0; b < nb; b++) {
        size_t off = b * (size_t)bs;
        int tb = (int)((size_t)bs < count - off ? (size_t)bs : count - off);
        float max_abs = 0.0f;
        for (int i = 0; i < tb; i++) {
            float a = fabsf(data[off + i]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 7.0f;
        float inv = (scale > 0.0f) ? 1.0f / scale : 0.0f;
        uint16_t sh = or_fp32_to_fp16(scale);
        uint8_t* blk = out + b * bb;
        memcpy(blk, &sh, 2);
        uint8_t* p = blk + 2;
        for (int i = 0; i < tb / 2; i++) {
            float v0 = data[off + 2 * i] * inv;
            float v1 = data[off + 2 * i + 1] * inv;
            v0 = std_max(-8.0f, std_min(7.0f, roundf(v0)));
            v1 = std_max(-8.0f, std_min(7.0f, roundf(v1)));
            uint8_t lo = (uint8_t)((uint8_t)((int)v0 + 8) & 0x0F);
            uint8_t hi = (uint8_t)((uint8_t)((int)v1 + 8) & 0x0F);
            p[i] = (uint8_t)(lo | (hi << 4));
        }
    }
    return nb * bb;
}

/* quantize.cpp:17-28, :35-51, :55-101 */
int or_dequantize(const void* data, uint32_t dtype, size_t count, int bs, float* out) {
    const uint8_t* p = (const uint8_t*)data;
    if (dtype == OR_F32) { memcpy(out, data, count * 4); return 0; }
    if (dtype == OR_F16) {
        for (size_t i = 0; i < count; i++) {
            uint16_t h;
            memcpy(&h, p + 2 * i, 2);
            out[i] = or_fp16_to_fp32(h);
        }
        return 0;
    }
    size_t nb = (count + bs - 1) / bs;
    for (size_t b = 0; b < nb; b++) {
        size_t off = b * (size_t)bs;
        int tb = (int)((size_t)bs < count - off ? (size_t)bs : count - off);
        if (dtype == OR_Q8_0) {
            float s;
            memcpy(&s, p, 4);
            const int8_t* q = (const int8_t*)(p + 4);
            for (int i = 0; i < tb; i++) out[off + i] = (float)q[i] * s;
            p += 4 + bs;
        } else if (dtype == OR_Q4_0) {
            uint16_t sh;
            memcpy(&sh, p, 2);
            float s = or_fp16_to_fp32(sh);
            /* dequantize_block_q4_0 writes block_size/2 pairs of this_block;
             * quantize.cpp:43-50 uses the passed (this) block size */
            for (int i = 0; i < tb / 2; i++) {
                uint8_t v = p[2 + i];
                out[off + 2 * i] = (float)((v & 0x0F) - 8) * s;
                out[off + 2 * i + 1] = (float)(((v >> 4) & 0x0F) - 8) * s;
            }
            if (tb & 1) out[off + tb - 1] = 0.0f; /* Tensor::zeros default */
            p += 2 + bs / 2;
        } else {
            return -1;
        }
    }
    return 0;
}

/* ---------------- dot products ---------------- */

/* quantize.cpp:187-210 */
float or_dot_q8_0_f32(const void* q8, const float* x, size_t count, int bs) {
    const uint8_t* p = (const uint8_t*)q8;
    float total = 0.0f;
    size_t nb = (count + bs - 1) / bs;
    for (size_t b = 0; b < nb; b++) {
        float scale;
        memcpy(&scale, p, 4);
        p += 4;
        const int8_t* q = (const int8_t*)p;
        size_t off = b * (size_t)bs;
        int tb = (int)((size_t)bs < count - off ? (size_t)bs : count - off);
        float bsum = 0.0f;
        for (int i = 0; i < tb; i++) bsum += (float)q[i] * x[off + i];
        total += bsum * scale;
        p += bs;
    }
    return total;
}

/* quantize.cpp:212-239 */
float or_dot_q4_0_f32(const void* q4, const float* x, size_t count, int bs) {
    const uint8_t* p = (const uint8_t*)q4;
    float total = 0.0f;
    size_t nb = (count + bs - 1) / bs;
    for (size_t b = 0; b < nb; b++) {
        uint16_t sh;
        memcpy(&sh, p, 2);
        float scale = or_fp16_to_fp32(sh);
        p += 2;
        size_t off = b * (size_t)bs;
        int tb = (int)((size_t)bs < count - off ? (size_t)bs : count - off);
        float bsum = 0.0f;
        for (int i = 0; i < tb / 2; i++) {
            uint8_t v = p[i];
            int lo = (v & 0x0F) - 8, hi = ((v >> 4) & 0x0F) - 8;
            bsum += (float)lo * x[off + 2 * i];
            bsum += (float)hi * x[off + 2 * i + 1];
        }
        total += bsum * scale;
        p += bs / 2;
    }
    return total;
}

/* backend.cpp:131-199 (scalar branches :162-165, :191-194; unknown :195-198) */
int or_matvec_q(const void* w, uint32_t dtype, int bs, uint32_t out_dim, uint32_t in_dim,
                const float* x, float* y) {
    const uint8_t* p = (const uint8_t*)w;
    size_t nb = (in_dim + bs - 1) / bs;
    if (dtype == OR_Q8_0) {
        size_t rb = nb * (4 + (size_t)bs);
        for (uint32_t i = 0; i < out_dim; i++) y[i] = or_dot_q8_0_f32(p + i * rb, x, in_dim, bs);
        return 0;
    }
    if (dtype == OR_Q4_0) {
        size_t rb = nb * (2 + (size_t)(bs / 2));
        for (uint32_t i = 0; i < out_dim; i++) y[i] = or_dot_q4_0_f32(p + i * rb, x, in_dim, bs);
        return 0;
    }
    memset(y, 0, out_dim * sizeof(float));
    return -1;
}

/* backend.cpp:92-103 */
void or_matvec_f32(const float* W, const float* x, float* y, uint32_t out_dim, uint32_t in_dim) {
    for (uint32_t i = 0; i < out_dim; i++) {
        float sum = 0.0f;
        const float* row = W + (size_t)i * in_dim;
        for (uint32_t j = 0; j < in_dim; j++) sum += row[j] * x[j];
        y[i] = sum;
    }
}

/* backend.cpp:124-126 */
float or_dot_f32(const float* a, const float* b, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* ---------------- elementwise (ops.cpp) ---------------- */

/* ops.cpp:107-118 */
void or_rms_norm(float* x, const float* w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n + eps;
    float r = 1.0f / sqrtf(ss);
    for (int i = 0; i < n; i++) x[i] = x[i] * r * w[i];
}

/* ops.cpp:158-177, applied to one vector (attention.cpp:105-116 rotates q
 * heads and k heads in separate calls with the same formula) */
void or_rope(float* v, int hd, int pos, float theta) {
    for (int i = 0; i < hd; i += 2) {
        float freq = 1.0f / powf(theta, (float)i / (float)hd);
        float val = (float)pos * freq;
        float c = cosf(val), s = sinf(val);
        float a = v[i], b = v[i + 1];
        v[i] = a * c - b * s;
        v[i + 1] = a * s + b * c;
    }
}

/* ops.cpp:218-222 */
void or_silu(float* x, int n) {
    for (int i = 0; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* ops.cpp:242-259 */
void or_softmax(float* x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* ops.cpp:269-285 */
void or_add(float* x, const float* y, int n) { for (int i = 0; i < n; i++) x[i] += y[i]; }
void or_mul(float* x, const float* y, int n) { for (int i = 0; i < n; i++) x[i] *= y[i]; }
void or_scale(float* x, float s, int n) { for (int i = 0; i < n; i++) x[i] *= s; }

/* attention.cpp:122-150 (after q/k/v projection, bias, RoPE and the cache
 * store): per query head h, kv head h / (H/Hkv); scores = dot * scale;
 * softmax over ctx positions; out = sum_t p_t V_t accumulated in t order. */
void or_attention_decode(const float* q, const float* K, const float* V, int ctx, int H,
                         int Hkv, int hd, float* out) {
    int rep = H / Hkv, kvd = Hkv * hd;
    float scale = 1.0f / sqrtf((float)hd);
    float* sc = (float*)malloc(sizeof(float) * (size_t)(ctx > 0 ? ctx : 1));
    for (int h = 0; h < H; h++) {
        int kh = h / rep;
        const float* qh = q + (size_t)h * hd;
        float* oh = out + (size_t)h * hd;
        for (int t = 0; t < ctx; t++) sc[t] = or_dot_f32(qh, K + (size_t)t * kvd + kh * hd, hd) * scale;
        or_softmax(sc, ctx);
        memset(oh, 0, sizeof(float) * hd);
        for (int t = 0; t < ctx; t++) {
            const float* vt = V + (size_t)t * kvd + kh * hd;
            float s = sc[t];
            for (int d = 0; d < hd; d++) oh[d] += s * vt[d];
        }
    }
    free(sc);
}

/* ---------------- int8 KV (kv_cache_quant.h) ---------------- */

/* QuantizedKVCache::store for one head (kv_cache_quant.h:61-95): amax over
 * the head, scale = amax / 127, inv = scale > 0 ? 1 / scale : 0,
 * q = (int8) clamp(round(x * inv), -127, 127), round half away from zero. */
void or_kv_quant_head(const float* x, int hd, int8_t* q, float* scale) {
    float amax = 0.0f;
    for (int d = 0; d < hd; d++) amax = fmaxf(amax, fabsf(x[d]));
    float s = amax / 127.0f;
    float inv = (s > 0) ? 1.0f / s : 0.0f;
    *scale = s;
    for (int d = 0; d < hd; d++) {
        float r = roundf(x[d] * inv);
        q[d] = (int8_t)fmaxf(-127.0f, fminf(127.0f, r));
    }
}

/* QuantizedKVCache::dot_with_key (kv_cache_quant.h:118-128) */
float or_kv_dot_key(const int8_t* kq, float scale, const float* query, int hd) {
    float sum = 0.0f;
    for (int d = 0; d < hd; d++) sum += (float)kq[d] * query[d];
    return sum * scale;
}

/* attention_forward's scores and weighted sum (attention.cpp:122-150) over
 * int8 K/V as kv_cache_quant.h reads them: score = dot_with_key (:118-128,
 * sum of (float)q8 * query, then * scale) * (1/sqrt(hd)); V rows through
 * dequant_value (:108-116, (float)q8 * scale), accumulated in t order.
 * K8, V8: [ctx][Hkv][hd]; Ks, Vs: [ctx][Hkv]. */
void or_attention_decode_i8(const float* q, const int8_t* K8, const float* Ks, const int8_t* V8, const float* Vs,
                            int ctx, int H, int Hkv, int hd, float* out) {
    int rep = H / Hkv, kvd = Hkv * hd;
    float scale = 1.0f / sqrtf((float)hd);
    float* sc = (float*)malloc(sizeof(float) * (size_t)(ctx > 0 ? ctx : 1));
    float* vrow = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int h = 0; h < H; h++) {
        int kh = h / rep;
        const float* qh = q + (size_t)h * hd;
        float* oh = out + (size_t)h * hd;
        for (int t = 0; t < ctx; t++)
            sc[t] = or_kv_dot_key(K8 + (size_t)t * kvd + kh * hd, Ks[(size_t)t * Hkv + kh], qh, hd) * scale;
        or_softmax(sc, ctx);
        memset(oh, 0, sizeof(float) * hd);
        for (int t = 0; t < ctx; t++) {
            const int8_t* vq = V8 + (size_t)t * kvd + kh * hd;
            float vsc = Vs[(size_t)t * Hkv + kh];
            for (int d = 0; d < hd; d++) vrow[d] = (float)vq[d] * vsc;
            float s = sc[t];
            for (int d = 0; d < hd; d++) oh[d] += s * vrow[d];
        }
    }
    free(vrow);
    free(sc);
}

/* ---------------- sampling (sampler.cpp) ---------------- */

/* sampler.cpp:25-35: strict '>', lowest index wins ties */
uint32_t or_argmax(const float* l, int n) {
    uint32_t best = 0;
    float bv = l[0];
    for (int i = 1; i < n; i++)
        if (l[i] > bv) { bv = l[i]; best = (uint32_t)i; }
    return best;
}

/* sampler.cpp:37-49: once per occurrence */
void or_repetition_penalty(float* l, int n, const uint32_t* toks, int nt, float p) {
    if (p == 1.0f) return;
    for (int i = 0; i < nt; i++) {
        uint32_t t = toks[i];
        if (t >= (uint32_t)n) continue;
        if (l[t] > 0) l[t] /= p;
        else l[t] *= p;
    }
}

/* ---------------- repo-defined synthetic weights ---------------- */

uint64_t or_mix64(uint64_t z) { /* splitmix64 finaliser */
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* format.h:136-147 */
uint64_t or_fnv1a(const char* s) {
    uint64_t h = 14695981039346656037ULL;
    for (; *s; s++) {
        h ^= (uint64_t)(unsigned char)*s;
        h *= 1099511628211ULL;
    }
    return h;
}

/* D = 2*S - 8*65535 has variance 4 * 8 * (65536^2 - 1) / 12 */
float or_gen_scale(float stddev) {
    double sd = 2.0 * sqrt(8.0 * (65536.0 * 65536.0 - 1.0) / 12.0);
    return (float)((double)stddev / sd);
}

static inline float gen_one(uint64_t base, uint64_t idx, float c) {
    uint64_t h1 = or_mix64(base + 2 * idx), h2 = or_mix64(base + 2 * idx + 1);
    int32_t s = 0;
    for (int k = 0; k < 4; k++) s += (int32_t)((h1 >> (16 * k)) & 0xFFFFu) + (int32_t)((h2 >> (16 * k)) & 0xFFFFu);
    int32_t d = 2 * s - 8 * 65535;
    return (float)d * c;
}

void or_gen_normal(uint64_t seed, uint64_t stream, size_t n, float stddev, float* out) {
    uint64_t base = or_mix64(seed ^ or_mix64(stream + 0x9E3779B97F4A7C15ULL));
    float c = or_gen_scale(stddev);
    for (size_t i = 0; i < n; i++) out[i] = gen_one(base, (uint64_t)i, c);
}

uint32_t or_gen_token(uint64_t seed, uint64_t idx, uint32_t vocab) {
    return (uint32_t)(or_mix64(or_mix64(seed ^ 0x70726F6D7074ULL) + idx) % vocab);
}

/* ---------------- model ---------------- */

typedef struct {
    char name[96];
    uint32_t dtype, ndim, shape[2];
    uint8_t* data;
    uint64_t size;
} or_tensor;

struct or_model {
    or_config c;
    uint32_t hd;
    int nt;
    or_tensor* t;
    /* per-layer indices into t[] */
    int *wq, *wk, *wv, *wo, *wg, *wu, *wd, *bq, *bk, *bv, *an, *fn;
    int emb, onorm, head;
    float* emb_f32; /* load_tensor_f32 of the embedding (transformer.cpp:321-334) */
    int kv_cap;
    float *kc, *vc; /* [layer][pos][kv_dim] f32, attention.cpp:14-31 */
    /* int8 KV mode (or_model_set_kv_int8): QuantizedKVCache in place of the
     * f32 KVCache, kv_cache_quant.h:16-50 ([layer][pos][kv_dim] int8 and
     * [layer][pos][kv_heads] scales) */
    int8_t *k8, *v8;
    float *ks, *vs;
    float *x, *res, *nrm, *att, *mlp, *q, *k, *v, *ao, *g, *u;
};

static int add_tensor(or_model* m, const char* name, uint32_t dtype, uint32_t r, uint32_t c,
                      int is_norm, uint64_t seed) {
    or_tensor* t = &m->t[m->nt];
    snprintf(t->name, sizeof(t->name), "%s", name);
    t->dtype = dtype;
    t->ndim = c ? 2 : 1;
    t->shape[0] = r;
    t->shape[1] = c;
    size_t n = (size_t)r * (c ? c : 1);
    float* f = (float*)malloc(n * sizeof(float));
    if (is_norm) {
        for (size_t i = 0; i < n; i++) f[i] = 1.0f;
    } else {
        or_gen_normal(seed, or_fnv1a(name), n, 0.02f, f);
    }
    t->size = or_q_tensor_bytes(dtype, n, m->c.block_size);
    t->data = (uint8_t*)malloc(t->size ? t->size : 1);
    if (dtype == OR_F32) memcpy(t->data, f, n * 4);
    else if (dtype == OR_Q8_0) or_quantize_q8_0(f, n, m->c.block_size, t->data);
    else if (dtype == OR_Q4_0) or_quantize_q4_0(f, n, m->c.block_size, t->data);
    else if (dtype == OR_F16) {
        for (size_t i = 0; i < n; i++) {
            uint16_t h = or_fp32_to_fp16(f[i]);
            memcpy(t->data + 2 * i, &h, 2);
        }
    }
    free(f);
    return m->nt++;
}

or_model* or_model_generate(const or_config* cfg, uint64_t seed) {
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->c = *cfg;
    if (m->c.block_size <= 0) m->c.block_size = 32;
    m->hd = cfg->hidden / cfg->heads; /* types.h:122 */
    uint32_t L = cfg->layers, D = cfg->hidden, qd = cfg->heads * m->hd, kvd = cfg->kv_heads * m->hd;
    m->t = (or_tensor*)calloc(16 * L + 8, sizeof(or_tensor));
#define ALLOC(f) m->f = (int*)malloc(sizeof(int) * L)
    ALLOC(wq); ALLOC(wk); ALLOC(wv); ALLOC(wo); ALLOC(wg); ALLOC(wu); ALLOC(wd);
    ALLOC(bq); ALLOC(bk); ALLOC(bv); ALLOC(an); ALLOC(fn);
#undef ALLOC
    char nm[96];
    m->emb = add_tensor(m, "model.embed_tokens.weight", cfg->embed_dtype, cfg->vocab, D, 0, seed);
    for (uint32_t l = 0; l < L; l++) {
#define T(field, suffix, r, c, dt, isn)                                       \
    snprintf(nm, sizeof(nm), "model.layers.%u.%s", l, suffix);              \
    m->field[l] = add_tensor(m, nm, dt, r, c, isn, seed)
        T(wq, "self_attn.q_proj.weight", qd, D, cfg->wdtype, 0);
        T(wk, "self_attn.k_proj.weight", kvd, D, cfg->wdtype, 0);
        T(wv, "self_attn.v_proj.weight", kvd, D, cfg->wdtype, 0);
        T(wo, "self_attn.o_proj.weight", D, qd, cfg->wdtype, 0);
        if (cfg->qkv_bias) {
            T(bq, "self_attn.q_proj.bias", qd, 0, OR_F32, 0);
            T(bk, "self_attn.k_proj.bias", kvd, 0, OR_F32, 0);
            T(bv, "self_attn.v_proj.bias", kvd, 0, OR_F32, 0);
        } else {
            m->bq[l] = m->bk[l] = m->bv[l] = -1;
        }
        T(wg, "mlp.gate_proj.weight", cfg->inter, D, cfg->wdtype, 0);
        T(wu, "mlp.up_proj.weight", cfg->inter, D, cfg->wdtype, 0);
        T(wd, "mlp.down_proj.weight", D, cfg->inter, cfg->wdtype, 0);
        T(an, "input_layernorm.weight", D, 0, OR_F32, 1);
        T(fn, "post_attention_layernorm.weight", D, 0, OR_F32, 1);
#undef T
    }
    m->onorm = add_tensor(m, "model.norm.weight", OR_F32, D, 0, 1, seed);
    m->head = cfg->tied ? -1 : add_tensor(m, "lm_head.weight", cfg->head_dtype, cfg->vocab, D, 0, seed);

    size_t ne = (size_t)cfg->vocab * D;
    m->emb_f32 = (float*)malloc(ne * sizeof(float));
    or_dequantize(m->t[m->emb].data, cfg->embed_dtype, ne, m->c.block_size, m->emb_f32);

    m->kv_cap = (int)(cfg->max_seq < 8192u ? cfg->max_seq : 8192u); /* transformer.cpp:425-428 */
    m->kc = (float*)calloc((size_t)L * m->kv_cap * kvd, sizeof(float));
    m->vc = (float*)calloc((size_t)L * m->kv_cap * kvd, sizeof(float));
    size_t big = D > cfg->inter ? D : cfg->inter;
    if (qd > big) big = qd;
    m->x = (float*)malloc(D * 4); m->res = (float*)malloc(D * 4); m->nrm = (float*)malloc(D * 4);
    m->att = (float*)malloc(D * 4); m->mlp = (float*)malloc(D * 4);
    m->q = (float*)malloc(qd * 4); m->k = (float*)malloc(kvd * 4); m->v = (float*)malloc(kvd * 4);
    m->ao = (float*)malloc(qd * 4); m->g = (float*)malloc(big * 4); m->u = (float*)malloc(big * 4);
    return m;
}

void or_model_free(or_model* m) {
    if (!m) return;
    for (int i = 0; i < m->nt; i++) free(m->t[i].data);
    free(m->t);
    free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->wg); free(m->wu); free(m->wd);
    free(m->bq); free(m->bk); free(m->bv); free(m->an); free(m->fn);
    free(m->emb_f32); free(m->kc); free(m->vc);
    free(m->k8); free(m->v8); free(m->ks); free(m->vs);
    free(m->x); free(m->res); free(m->nrm); free(m->att); free(m->mlp);
    free(m->q); free(m->k); free(m->v); free(m->ao); free(m->g); free(m->u);
    free(m);
}

int or_model_num_tensors(const or_model* m) { return m->nt; }

int or_model_tensor(const or_model* m, int i, const char** name, uint32_t* dtype, uint32_t* ndim,
                    uint32_t* shape, const void** data, uint64_t* size) {
    if (i < 0 || i >= m->nt) return -1;
    const or_tensor* t = &m->t[i];
    *name = t->name;
    *dtype = t->dtype;
    *ndim = t->ndim;
    shape[0] = t->shape[0];
    shape[1] = t->shape[1];
    *data = t->data;
    *size = t->size;
    return 0;
}

void or_model_reset(or_model* m) { /* attention.cpp:33-37 */
    size_t n = (size_t)m->c.layers * m->kv_cap * m->c.kv_heads * m->hd;
    memset(m->kc, 0, n * 4);
    memset(m->vc, 0, n * 4);
    if (m->k8) { /* kv_cache_quant.h:52-58 */
        size_t ns = (size_t)m->c.layers * m->kv_cap * m->c.kv_heads;
        memset(m->k8, 0, n); memset(m->v8, 0, n);
        memset(m->ks, 0, ns * 4); memset(m->vs, 0, ns * 4);
    }
}

/* Switch the model's cache to QuantizedKVCache (kv_cache_quant.h:30-50),
 * emptied.  The reference defines that cache without wiring it into its
 * Transformer; here it takes the f32 KVCache's two places: the store after
 * RoPE (attention.cpp:119) quantizes, and the attention reads scores through
 * dot_with_key and values through dequant_value. */
int or_model_set_kv_int8(or_model* m) {
    size_t n = (size_t)m->c.layers * m->kv_cap * m->c.kv_heads * m->hd;
    size_t ns = (size_t)m->c.layers * m->kv_cap * m->c.kv_heads;
    if (!m->k8) {
        m->k8 = (int8_t*)calloc(n, 1); m->v8 = (int8_t*)calloc(n, 1);
        m->ks = (float*)calloc(ns, 4); m->vs = (float*)calloc(ns, 4);
        if (!m->k8 || !m->v8 || !m->ks || !m->vs) return -1;
    }
    or_model_reset(m);
    return 0;
}

/* attention.cpp:56-65 do_matvec */
static void mv(const or_model* m, int ti, uint32_t out, uint32_t in, const float* x, float* y) {
    const or_tensor* t = &m->t[ti];
    if (t->dtype == OR_F32) or_matvec_f32((const float*)t->data, x, y, out, in);
    else or_matvec_q(t->data, t->dtype, m->c.block_size, out, in, x, y);
}

int or_model_forward(or_model* m, uint32_t token, int pos, float* logits) {
    const or_config* c = &m->c;
    if (token >= c->vocab || pos < 0 || pos >= m->kv_cap) return -1; /* transformer.cpp:623 */
    int D = (int)c->hidden, H = (int)c->heads, Hkv = (int)c->kv_heads, hd = (int)m->hd;
    int qd = H * hd, kvd = Hkv * hd, F = (int)c->inter;
    memcpy(m->x, m->emb_f32 + (size_t)token * D, D * 4); /* transformer.cpp:577 */
    for (uint32_t l = 0; l < c->layers; l++) {           /* transformer.cpp:582-603 */
        memcpy(m->res, m->x, D * 4);
        memcpy(m->nrm, m->x, D * 4);
        or_rms_norm(m->nrm, (const float*)m->t[m->an[l]].data, D, c->eps);
        /* attention_forward, attention.cpp:69-155 */
        mv(m, m->wq[l], qd, D, m->nrm, m->q);
        mv(m, m->wk[l], kvd, D, m->nrm, m->k);
        mv(m, m->wv[l], kvd, D, m->nrm, m->v);
        if (m->bq[l] >= 0) or_add(m->q, (const float*)m->t[m->bq[l]].data, qd);
        if (m->bk[l] >= 0) or_add(m->k, (const float*)m->t[m->bk[l]].data, kvd);
        if (m->bv[l] >= 0) or_add(m->v, (const float*)m->t[m->bv[l]].data, kvd);
        for (int h = 0; h < H; h++) or_rope(m->q + h * hd, hd, pos, c->rope_theta);
        for (int h = 0; h < Hkv; h++) or_rope(m->k + h * hd, hd, pos, c->rope_theta);
        if (m->k8) { /* QuantizedKVCache::store (kv_cache_quant.h:61-95) */
            size_t lo = (size_t)l * m->kv_cap * kvd, so = (size_t)l * m->kv_cap * Hkv;
            for (int h = 0; h < Hkv; h++) {
                size_t e = lo + (size_t)pos * kvd + h * hd, sc = so + (size_t)pos * Hkv + h;
                or_kv_quant_head(m->k + h * hd, hd, m->k8 + e, m->ks + sc);
                or_kv_quant_head(m->v + h * hd, hd, m->v8 + e, m->vs + sc);
            }
            or_attention_decode_i8(m->q, m->k8 + lo, m->ks + so, m->v8 + lo, m->vs + so, pos + 1, H, Hkv, hd, m->ao);
        } else {
            float* kl = m->kc + (size_t)l * m->kv_cap * kvd;
            float* vl = m->vc + (size_t)l * m->kv_cap * kvd;
            memcpy(kl + (size_t)pos * kvd, m->k, kvd * 4);
            memcpy(vl + (size_t)pos * kvd, m->v, kvd * 4);
            or_attention_decode(m->q, kl, vl, pos + 1, H, Hkv, hd, m->ao);
        }
        mv(m, m->wo[l], D, qd, m->ao, m->att);
        or_add(m->att, m->res, D);
        memcpy(m->res, m->att, D * 4);
        memcpy(m->nrm, m->att, D * 4);
        or_rms_norm(m->nrm, (const float*)m->t[m->fn[l]].data, D, c->eps);
        /* mlp_forward, attention.cpp:159-184 */
        mv(m, m->wg[l], F, D, m->nrm, m->g);
        mv(m, m->wu[l], F, D, m->nrm, m->u);
        or_silu(m->g, F);
        or_mul(m->g, m->u, F);
        mv(m, m->wd[l], D, F, m->g, m->mlp);
        or_add(m->mlp, m->res, D);
        memcpy(m->x, m->mlp, D * 4);
    }
    or_rms_norm(m->x, (const float*)m->t[m->onorm].data, D, c->eps); /* :605 */
    if (m->head < 0) or_matvec_f32(m->emb_f32, m->x, logits, c->vocab, D); /* tied, :608-610 */
    else mv(m, m->head, c->vocab, D, m->x, logits);
    return 0;
}

/* inference.cpp:68-159, greedy (sampler.cpp:56-60 -> argmax) */
int or_generate(or_model* m, const uint32_t* prompt, int np, int max_tokens, float penalty, int eos,
                uint32_t* out) {
    if (np <= 0) return -1;
    int V = (int)m->c.vocab;
    float* logits = (float*)malloc(sizeof(float) * V);
    uint32_t* recent = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(np + max_tokens));
    or_model_reset(m);
    for (int i = 0; i < np; i++)
        if (or_model_forward(m, prompt[i], i, logits)) { free(logits); free(recent); return -1; }
    memcpy(recent, prompt, sizeof(uint32_t) * np);
    int nr = np, ng = 0, pos = np;
    for (int t = 0; t < max_tokens; t++) {
        or_repetition_penalty(logits, V, recent, nr, penalty);
        uint32_t nx = or_argmax(logits, V);
        if (eos >= 0 && nx == (uint32_t)eos) break;
        out[ng++] = nx;
        recent[nr++] = nx;
        if (or_model_forward(m, nx, pos, logits)) break;
        pos++;
    }
    free(logits);
    free(recent);
    return ng;
}
