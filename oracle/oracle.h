/*
 * oracle.h -- CPU restatement of QRAF's scalar x86 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (qraf_amd/) links,
 * loads or calls this code.  It is the checker that tests/, the smoke()
 * entry point and the cpu_baseline leg of bench.py compare against.
 *
 * Every function cites the reference file:line it restates.  Build flags
 * follow the reference's Release build on baseline x86-64 (-O3, no
 * -ffast-math, no FMA contraction), so the fp32 rounding sequence is the
 * reference's own.
 *
 * Parity pins (each function is checked in tests/test_oracle_*.py):
 *   fp16 conversions      exhaustive 2^16 decode vs IEEE; encode vs golden
 *   quantizers            golden vectors from the compiled reference, closed form
 *   dot / matvec          golden vectors; one-hot and all-ones closed forms;
 *                         float64 brute force bound
 *   rms_norm/rope/silu/
 *   softmax/attention     golden vectors; closed forms; float64 textbook attention
 *   forward / generate    golden logits + greedy streams from the compiled reference
 *   weight RNG            repo-defined; pinned by moments and by the GPU generator
 *                         producing the same bytes (no reference counterpart)
 */
#ifndef QRAF_ORACLE_H
#define QRAF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 10, OR_Q4_0 = 20 };

/* dtype.cpp:9-37 / :39-59 */
float    or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);

/* block geometry: quantize.cpp:105-108 / :144-147 */
size_t or_q_block_bytes(uint32_t dtype, int block_size);
size_t or_q_tensor_bytes(uint32_t dtype, size_t count, int block_size);

/* quantize.cpp:105-140 / :144-183 ; returns bytes written */
size_t or_quantize_q8_0(const float* data, size_t count, int block_size, uint8_t* out);
size_t or_quantize_q4_0(const float* data, size_t count, int block_size, uint8_t* out);

/* quantize.cpp:55-101 (Q8_0 / Q4_0 / F16 / F32 branches) */
int or_dequantize(const void* data, uint32_t dtype, size_t count, int block_size, float* out);

/* quantize.cpp:187-210 / :212-239 */
float or_dot_q8_0_f32(const void* q8, const float* x, size_t count, int block_size);
float or_dot_q4_0_f32(const void* q4, const float* x, size_t count, int block_size);

/* backend.cpp:131-199 scalar branch; returns 0, or -1 for an unknown dtype
 * (the reference zero-fills y in that case, which this also does) */
int or_matvec_q(const void* w, uint32_t dtype, int block_size, uint32_t out_dim,
                uint32_t in_dim, const float* x, float* y);
/* backend.cpp:92-103 */
void or_matvec_f32(const float* W, const float* x, float* y, uint32_t out_dim, uint32_t in_dim);
/* backend.cpp:124-126 */
float or_dot_f32(const float* a, const float* b, int n);

/* ops.cpp:107-118, :158-177 (one vector), :218-222, :242-259, :269-285 */
void or_rms_norm(float* x, const float* w, int n, float eps);
void or_rope(float* v, int head_dim, int pos, float theta);
void or_silu(float* x, int n);
void or_softmax(float* x, int n);
void or_add(float* x, const float* y, int n);
void or_mul(float* x, const float* y, int n);
void or_scale(float* x, float s, int n);

/* attention.cpp:122-150 for one sequence: q [H*hd]; K,V [ctx][Hkv*hd] f32;
 * out [H*hd].  scores buffer is internal. */
void or_kv_quant_head(const float* x, int hd, int8_t* q, float* scale);
float or_kv_dot_key(const int8_t* kq, float scale, const float* query, int hd);

void or_attention_decode_i8(const float* q, const int8_t* K8, const float* Ks, const int8_t* V8, const float* Vs,
                            int ctx, int H, int Hkv, int hd, float* out);
void or_attention_decode(const float* q, const float* K, const float* V, int ctx,
                         int H, int Hkv, int hd, float* out);

/* sampler.cpp:25-35 / :37-49 */
uint32_t or_argmax(const float* logits, int n);
void or_repetition_penalty(float* logits, int n, const uint32_t* toks, int ntoks, float penalty);

/* ---- repo-defined synthetic weights (no reference counterpart; the
 * reference's tools/dummy_model.cpp:12-17 uses std::mt19937 +
 * std::normal_distribution, which a GPU cannot reproduce).  An 8-term
 * Irwin-Hall sum of 16-bit hash fields, scaled to the requested std with one
 * correctly-rounded fp32 multiply, so CPU and GPU produce identical bits. */
uint64_t or_mix64(uint64_t z);
uint64_t or_fnv1a(const char* s);                 /* format.h fnv1a_hash */
float    or_gen_scale(float stddev);              /* the fp32 multiplier */
void     or_gen_normal(uint64_t seed, uint64_t stream, size_t count, float stddev, float* out);
uint32_t or_gen_token(uint64_t seed, uint64_t idx, uint32_t vocab);

/* ---- model (transformer.cpp:96-126, :310-439, :573-643) ---- */
typedef struct or_config {
    uint32_t vocab, hidden, layers, heads, kv_heads, inter, max_seq;
    float rope_theta, eps;
    uint32_t wdtype;        /* dtype of the 7 projection matrices: 0 / 10 / 20 */
    uint32_t embed_dtype;   /* dtype of model.embed_tokens.weight            */
    uint32_t head_dtype;    /* dtype of lm_head.weight                        */
    int32_t  tied;          /* 1: no lm_head.weight (head = f32 embedding)    */
    int32_t  qkv_bias;      /* 1: F32 q/k/v biases present (qwen2)            */
    int32_t  block_size;
} or_config;

typedef struct or_model or_model;

/* Build a model of synthetic weights from (cfg, seed).  Every tensor is
 * N(0, 0.02) from or_gen_normal with stream = fnv1a(tensor name); norms = 1. */
or_model* or_model_generate(const or_config* cfg, uint64_t seed);
void      or_model_free(or_model* m);
int       or_model_num_tensors(const or_model* m);
/* tensor i: name, dtype, ndim, shape[2], bytes, size */
int       or_model_tensor(const or_model* m, int i, const char** name, uint32_t* dtype,
                          uint32_t* ndim, uint32_t* shape, const void** data, uint64_t* size);
void      or_model_reset(or_model* m);                       /* transformer.cpp:641-643 */
int       or_model_set_kv_int8(or_model* m);                 /* QuantizedKVCache, kv_cache_quant.h */
int       or_model_forward(or_model* m, uint32_t token, int pos, float* logits); /* :573-639 */
/* inference.cpp:68-159 with temperature 0 (argmax); eos < 0 disables the stop
 * token; returns the number of generated tokens. */
int       or_generate(or_model* m, const uint32_t* prompt, int n_prompt, int max_tokens,
                      float penalty, int eos, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
