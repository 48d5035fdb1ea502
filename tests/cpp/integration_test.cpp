// integration_test.cpp -- the reference-side bindings of libqraf_hip.so,
// compiled against the reference's own headers and run against the
// reference's own code.
//
//     integration_test <model.qraf> <tokens>
//
// Two bindings, written as a maintainer would add them to the reference:
//   * the Backend::HIP branch of dispatch_matvec_q (nn/backend.h:31-34,
//     src/nn/backend.cpp:131-199): hip_dispatch_matvec_q below, checked
//     against the reference's dispatch_matvec_q on the same quantized rows
//     (reference quantize_q8_0 / quantize_q4_0, tensor/quantize.h:52-55);
//   * HipTransformer, the Transformer::init / forward / reset triple
//     (nn/transformer.h:55-61) over qraf_engine_*: the model file is opened
//     with the reference's QrafModel (qraf/loader.h:29-46), both engines are
//     initialised from it, and every forward's logits are compared with the
//     reference Transformer's (|hip - ref| <= 1e-3 |ref| + 1e-4, the same
//     greedy token), for a greedy run of <tokens> positions, then again
//     after reset() of both.
// Exit status 0 when every check holds.  The reference's code comes from
// oracle/_ref/libqraf_ref.so (its sources compiled in place); this file
// holds only the bindings and the checks.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "core/error.h"
#include "core/logging.h"
#include "nn/backend.h"
#include "nn/transformer.h"
#include "qraf/loader.h"
#include "qraf_hip.h"
#include "tensor/quantize.h"

namespace qraf {

static inline void hip_check(int rc) {
    if (rc != QRAF_HIP_OK) throw InferenceError(qraf_hip_last_error());  // core/error.h:23-26
}

// The Backend::HIP branch of dispatch_matvec_q: host pointers in and out.
void hip_dispatch_matvec_q(const void* w_data, u64 w_size, DType w_dtype, const QuantScheme* quant, u32 out_dim,
                           u32 in_dim, const f32* x, f32* y) {
    hip_check(qraf_hip_matvec_q(w_data, w_size, static_cast<uint32_t>(w_dtype), quant ? quant->block_size : 32,
                                out_dim, in_dim, x, y));
}

// A Transformer whose forward runs entirely on the GPU.
class HipTransformer {
public:
    bool init(QrafModel& model) {
        const auto& c = model.config();
        qraf_model_config mc{c.vocab_size, c.hidden_size, c.num_layers,  c.num_heads,   c.num_kv_heads,
                             c.intermediate_size, c.max_seq_len, c.rope_theta, c.rms_norm_eps};
        qraf_engine_options eo{/*kv_dtype*/ 0 /*F32*/, /*page_size*/ 16, /*max_batch*/ 1, /*num_pages*/ 0};
        hip_check(qraf_engine_create(&mc, &eo, &e_));
        for (const auto& n : model.tensor_names()) {
            TensorView t = model.get_tensor(n);
            hip_check(qraf_engine_set_tensor(e_, t.name.c_str(), static_cast<uint32_t>(t.dtype),
                                             t.quant ? t.quant->block_size : 32, t.shape.data(), t.ndim(), t.data,
                                             t.data_size));
        }
        hip_check(qraf_engine_finalize(e_));
        logits_.resize(c.vocab_size);
        return true;
    }
    const std::vector<f32>& forward(u32 token, int pos) {
        hip_check(qraf_engine_forward(e_, token, pos, logits_.data()));
        return logits_;
    }
    void reset() { hip_check(qraf_engine_reset(e_)); }
    ~HipTransformer() {
        if (e_) qraf_engine_destroy(e_);
    }

private:
    qraf_engine* e_ = nullptr;
    std::vector<f32> logits_;
};

}  // namespace qraf

using namespace qraf;

static int g_fail = 0;

static u32 argmax(const f32* v, size_t n) {
    size_t b = 0;
    for (size_t i = 1; i < n; i++)
        if (v[i] > v[b]) b = i;
    return (u32)b;
}

// The Backend::HIP matvec against the reference's dispatch_matvec_q: the
// bound of the scalar dot's reassociation, 2 (K + 2) 2^-24 sum |w x| per row
// (w dequantized), plus 1e-6 of the row's magnitude for the dequantization
// products that are rounded differently.
static void check_matvec(DType dt, u32 N, u32 K, std::mt19937& rng) {
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<f32> w((size_t)N * K), x(K), yr(N), yh(N);
    for (auto& v : w) v = 0.02f * nd(rng);
    for (auto& v : x) v = nd(rng);
    std::vector<u8> q = dt == DType::Q8_0 ? quantize_q8_0(w.data(), w.size()) : quantize_q4_0(w.data(), w.size());
    QuantScheme qs{};
    qs.type = static_cast<u32>(dt);
    qs.block_size = 32;
    dispatch_matvec_q(q.data(), q.size(), dt, &qs, N, K, x.data(), yr.data());
    hip_dispatch_matvec_q(q.data(), q.size(), dt, &qs, N, K, x.data(), yh.data());
    double worst = 0;
    for (u32 i = 0; i < N; i++) {
        double mag = 0;
        for (u32 k = 0; k < K; k++) mag += std::fabs((double)w[(size_t)i * K + k] * x[k]);
        const double tol = 2.0 * (K + 2) * std::ldexp(1.0, -24) * mag * 1.5 + 1e-6 * mag + 1e-30;
        worst = std::max(worst, std::fabs((double)yh[i] - yr[i]) / tol);
    }
    std::printf("matvec %s %ux%u: worst error / bound %.3g\n", dt == DType::Q8_0 ? "q8_0" : "q4_0", N, K, worst);
    if (!(worst <= 1.0)) g_fail = 1;
}

// Greedy run of n positions through both engines, logits compared at every one.
static void run_both(Transformer& ref, HipTransformer& hip, u32 vocab, u32 tok0, int n, const char* what) {
    u32 tok = tok0;
    double worst = 0;
    int same = 0;
    for (int pos = 0; pos < n; pos++) {
        Tensor lr = ref.forward(tok, pos);
        const f32* r = lr.data_f32();
        const std::vector<f32>& h = hip.forward(tok, pos);
        for (u32 i = 0; i < vocab; i++) {
            const double tol = 1e-3 * std::fabs((double)r[i]) + 1e-4;
            worst = std::max(worst, std::fabs((double)h[i] - r[i]) / tol);
        }
        const u32 tr = argmax(r, vocab), th = argmax(h.data(), vocab);
        same += tr == th;
        tok = tr;
    }
    std::printf("%s: %d positions, worst logit error / tolerance %.4f, greedy tokens equal %d/%d\n", what, n, worst,
                same, n);
    if (!(worst <= 1.0) || same != n) g_fail = 1;
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s <model.qraf> <tokens>\n", argv[0]);
        return 2;
    }
    const int n = std::atoi(argv[2]);
    log::set_level(log::Level::ERROR);
    backend_init();  // the reference's scalar x86 backend
    try {
        int devs = 0;
        hip_check(qraf_hip_device_count(&devs));
        if (devs < 1) throw InferenceError("no GPU");
        hip_check(qraf_hip_init(0));

        std::mt19937 rng(2024);
        check_matvec(DType::Q8_0, 300, 2048, rng);
        check_matvec(DType::Q4_0, 300, 2048, rng);
        check_matvec(DType::Q8_0, 1000, 576, rng);

        QrafModel model;
        if (!model.load(argv[1])) throw InferenceError(std::string("cannot load ") + argv[1]);
        Transformer ref;
        if (!ref.init(model)) throw InferenceError("reference Transformer::init failed");
        HipTransformer hip;
        hip.init(model);
        const u32 vocab = model.config().vocab_size;
        run_both(ref, hip, vocab, 1 % vocab, n, "forward");
        ref.reset();
        hip.reset();
        run_both(ref, hip, vocab, 7 % vocab, n / 2 + 1, "forward after reset");
    } catch (const std::exception& e) {
        std::printf("error: %s\n", e.what());
        return 1;
    }
    std::printf(g_fail ? "FAIL\n" : "PASS\n");
    return g_fail;
}
