// ref_shim.cpp -- extern "C" access to the reference implementation itself.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's own
// sources (read in place under the reference checkout, never copied) into
// oracle/_ref/libqraf_ref.so by oracle/Makefile.  Tests use it to validate the
// C restatement in oracle.c and to write the golden fixtures; bench.py may
// time it as the CPU baseline.  Every function calls the reference's code
// unchanged: the backend is the scalar x86 one that backend_init() selects
// (backend.cpp:28-31).
#include "core/logging.h"
#include "nn/backend.h"
#include "nn/kv_cache_quant.h"
#include "nn/ops.h"
#include "nn/transformer.h"
#include "qraf/loader.h"
#include "qraf/writer.h"
#include "runtime/inference.h"
#include "sampling/sampler.h"
#include "tensor/quantize.h"

#include <cstring>
#include <memory>
#include <random>
#include <string>
#include <vector>

namespace qraf {
f32 fp16_to_fp32(f16 h);  // dtype.cpp:9
f16 fp32_to_fp16(f32 f);  // dtype.cpp:39
}  // namespace qraf

using namespace qraf;

static void quiet() {
    static bool done = false;
    if (!done) {
        log::set_level(log::Level::ERROR);
        backend_init();
        done = true;
    }
}

extern "C" {

float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }

size_t ref_quantize(uint32_t dtype, const float* data, size_t count, int bs, uint8_t* out) {
    std::vector<u8> r = dtype == 10 ? quantize_q8_0(data, count, bs) : quantize_q4_0(data, count, bs);
    memcpy(out, r.data(), r.size());
    return r.size();
}

float ref_dot(uint32_t dtype, const void* q, const float* x, size_t count, int bs) {
    return dtype == 10 ? dot_q8_0_f32(q, x, count, bs) : dot_q4_0_f32(q, x, count, bs);
}

void ref_matvec_q(const void* w, uint32_t dtype, int bs, uint32_t out_dim, uint32_t in_dim,
                  const float* x, float* y) {
    quiet();
    QuantScheme qs{};
    qs.type = dtype;
    qs.block_size = static_cast<u32>(bs);
    dispatch_matvec_q(w, 0, static_cast<DType>(dtype), &qs, out_dim, in_dim, x, y);
}

void ref_matvec_f32(const float* W, const float* x, float* y, uint32_t out_dim, uint32_t in_dim) {
    quiet();
    dispatch_matvec_opt(W, x, y, out_dim, in_dim);
}

void ref_rms_norm(float* x, const float* w, int n, float eps) { quiet(); dispatch_rms_norm(x, w, n, eps); }
void ref_softmax(float* x, int n) { quiet(); dispatch_softmax(x, n); }
void ref_silu(float* x, int n) { quiet(); dispatch_silu(x, n); }
void ref_rope(float* q, float* k, int hd, int pos, float theta) { ops::rope(q, k, hd, pos, theta); }
void ref_dequantize(const void* data, uint32_t dtype, size_t count, int bs, float* out) {
    quiet();
    QuantScheme qs{};
    qs.block_size = static_cast<u32>(bs);
    Tensor t = dequantize_tensor(data, 0, {static_cast<u32>(count)}, static_cast<DType>(dtype), &qs);
    memcpy(out, t.data_f32(), count * sizeof(float));
}
uint32_t ref_argmax(const float* l, int n) { return Sampler::argmax(l, n); }
void ref_penalty(float* l, int n, const uint32_t* toks, int nt, float p) {
    SamplingConfig sc;
    sc.repetition_penalty = p;
    sc.seed = 1;
    Sampler s(sc);
    s.apply_repetition_penalty(l, n, std::vector<u32>(toks, toks + nt));
}

// Sampler::sample (sampler.cpp:57-128) with a seeded config, n_draws times on
// the same logits; every non-greedy draw takes one uniform from the Sampler's
// std::mt19937.  Penalty 1: apply_repetition_penalty is a separate call.
void ref_sample(const float* logits, int V, float temperature, int top_k, float top_p, uint64_t seed, int n_draws,
                uint32_t* out) {
    SamplingConfig sc;
    sc.temperature = temperature;
    sc.top_k = top_k;
    sc.top_p = top_p;
    sc.repetition_penalty = 1.0f;
    sc.seed = seed;
    Sampler s(sc);
    for (int i = 0; i < n_draws; i++) out[i] = s.sample(logits, V);
}
// the uniforms a Sampler with this seed draws: std::mt19937 seeded as
// Sampler::Sampler does (sampler.cpp:9-16), std::uniform_real_distribution<f32>(0, 1)
void ref_uniforms(uint64_t seed, int n, float* out) {
    std::mt19937 rng;
    rng.seed(static_cast<unsigned>(seed));
    std::uniform_real_distribution<f32> d(0.0f, 1.0f);
    for (int i = 0; i < n; i++) out[i] = d(rng);
}

// QuantizedKVCache (kv_cache_quant.h, header-only, unused by the reference's
// own attention): store one position of k and v ([Hkv][hd]) and read back the
// int8 values, scales, dot_with_key against `query` per head, dequant_value.
void ref_kv_quant(const float* k, const float* v, int Hkv, int hd, const float* query, int8_t* kq, float* ks,
                  int8_t* vq, float* vs, float* dots, float* vdeq) {
    QuantizedKVCache c;
    c.init(1, Hkv, hd, 1);
    c.store(0, 0, k, v);
    memcpy(kq, c.keys_q[0].data(), (size_t)Hkv * hd);
    memcpy(vq, c.values_q[0].data(), (size_t)Hkv * hd);
    memcpy(ks, c.key_scales[0].data(), (size_t)Hkv * 4);
    memcpy(vs, c.value_scales[0].data(), (size_t)Hkv * 4);
    for (int h = 0; h < Hkv; h++) {
        dots[h] = c.dot_with_key(0, 0, h, query + (size_t)h * hd);
        c.dequant_value(0, 0, h, vdeq + (size_t)h * hd);
    }
}

// ---- QRAF file writing through the reference's QrafWriter (writer.cpp) ----
void* ref_writer_new() { quiet(); return new QrafWriter(); }
void ref_writer_free(void* w) { delete static_cast<QrafWriter*>(w); }
void ref_writer_config_u32(void* w, const char* k, uint32_t v) { static_cast<QrafWriter*>(w)->set_config(k, v); }
void ref_writer_config_f32(void* w, const char* k, float v) { static_cast<QrafWriter*>(w)->set_config(k, v); }
void ref_writer_config_str(void* w, const char* k, const char* v) {
    static_cast<QrafWriter*>(w)->set_config_string(k, v);
}
uint32_t ref_writer_quant_scheme(void* w, uint32_t dtype, uint32_t bs) {
    return static_cast<QrafWriter*>(w)->add_quant_scheme(static_cast<DType>(dtype), bs);
}
void ref_writer_tensor(void* w, const char* name, const uint32_t* shape, uint32_t ndim, uint32_t dtype,
                       const void* data, uint64_t size, uint32_t scheme) {
    std::vector<u32> sh(shape, shape + ndim);
    static_cast<QrafWriter*>(w)->add_tensor(name, sh, static_cast<DType>(dtype), data, size, scheme);
}
int ref_writer_write(void* w, const char* path) { return static_cast<QrafWriter*>(w)->write(path) ? 0 : -1; }

// ---- model: QrafModel::load + Transformer::init/forward/reset ----
struct RefModel {
    QrafModel model;
    Transformer tf;
};
void* ref_model_load(const char* path) {
    quiet();
    auto* m = new RefModel();
    if (!m->model.load(path) || !m->tf.init(m->model)) {
        delete m;
        return nullptr;
    }
    return m;
}
void ref_model_free(void* m) { delete static_cast<RefModel*>(m); }
void ref_model_reset(void* m) { static_cast<RefModel*>(m)->tf.reset(); }
int ref_model_forward(void* m, uint32_t token, int pos, float* logits) {
    try {
        Tensor t = static_cast<RefModel*>(m)->tf.forward(token, pos);
        memcpy(logits, t.data_f32(), t.nbytes());
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// ---- InferenceEngine::generate_tokens, greedy (inference.cpp:68-159) ----
void* ref_engine_load(const char* path) {
    quiet();
    auto* e = new InferenceEngine();
    if (!e->load_model(path)) {
        delete e;
        return nullptr;
    }
    return e;
}
void ref_engine_free(void* e) { delete static_cast<InferenceEngine*>(e); }
int ref_engine_generate(void* e, const uint32_t* prompt, int n, int max_tokens, float penalty,
                        uint32_t* out, double* ms) {
    GenerateConfig gc;
    gc.max_tokens = static_cast<u32>(max_tokens);
    gc.sampling.temperature = 0.0f;
    gc.sampling.repetition_penalty = penalty;
    gc.sampling.seed = 1;
    GenerateResult r = static_cast<InferenceEngine*>(e)->generate_tokens(std::vector<u32>(prompt, prompt + n), gc);
    for (size_t i = 0; i < r.tokens.size(); i++) out[i] = r.tokens[i];
    if (ms) *ms = r.generation_time_ms;
    return static_cast<int>(r.tokens.size());
}

// InferenceEngine::generate_tokens with a sampling configuration
int ref_engine_generate_sampled(void* e, const uint32_t* prompt, int n, int max_tokens, float temperature, int top_k,
                                float top_p, float penalty, uint64_t seed, uint32_t* out) {
    GenerateConfig gc;
    gc.max_tokens = static_cast<u32>(max_tokens);
    gc.sampling.temperature = temperature;
    gc.sampling.top_k = top_k;
    gc.sampling.top_p = top_p;
    gc.sampling.repetition_penalty = penalty;
    gc.sampling.seed = seed;
    GenerateResult r = static_cast<InferenceEngine*>(e)->generate_tokens(std::vector<u32>(prompt, prompt + n), gc);
    for (size_t i = 0; i < r.tokens.size(); i++) out[i] = r.tokens[i];
    return static_cast<int>(r.tokens.size());
}

}  // extern "C"
