// batch_integration_test.cpp -- the reference-side continuous-batching and
// elementwise bindings of libqraf_hip.so, compiled against the reference's
// own headers and run against the reference's own code.
//
//     batch_integration_test <model.qraf> <requests> <seed>
//
// Two bindings, written as a maintainer would add them to the reference:
//   * the Backend::HIP branches of the elementwise dispatch functions
//     (nn/backend.h:27-45, src/nn/backend.cpp:62-127, 203-320), checked
//     against the reference's dispatch_* on the same data;
//   * HipBatchScheduler, the BatchScheduler interface
//     (runtime/batch_scheduler.h:54-101: BatchConfig, BatchRequest,
//     submit / start / stop / active_requests / queued_requests /
//     total_processed) over the engine's batched steps: every active request
//     owns an engine sequence, one step advances every decoding request by
//     one token and feeds prompt chunks within a row budget, and requests are
//     admitted into the slots of finished ones.  Greedy requests (temperature
//     <= 0 or deterministic, repetition penalty 1) run pipelined
//     (qraf_engine_step_async / qraf_engine_step_collect: a decode row takes
//     its token from the previous step's argmax on the device); others run
//     one step at a time with qraf_engine_sample (the reference Sampler's
//     penalty and draw, the draw's uniform from the request's own
//     std::mt19937 as Sampler seeds it).
// The check: <requests> ragged requests (prompts of 1-40 tokens, 8-40
// generated tokens, EOS = the tokenizer's) through 6 slots with a 32-row
// budget, against the reference's own Transformer decoding each request
// alone with the per-request loop of BatchScheduler::decode_step
// (batch_scheduler.h:187-228): the pipelined run's token streams equal, and
// a run that reads back every logit row has each logit vector of the first
// 32 tokens within 1e-3 relative + 1e-4 absolute of the reference's and the
// same streams.  Exit status 0 when every check holds.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <deque>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "core/error.h"
#include "core/logging.h"
#include "nn/backend.h"
#include "nn/transformer.h"
#include "qraf/loader.h"
#include "qraf_hip.h"
#include "runtime/batch_scheduler.h"
#include "runtime/tokenizer.h"
#include "sampling/sampler.h"

namespace qraf {

static inline void hip_check(int rc) {
    if (rc != QRAF_HIP_OK) throw InferenceError(qraf_hip_last_error());  // core/error.h:23-26
}

// ---- Backend::HIP branches of the elementwise dispatch functions (host pointers)
f32 hip_dispatch_dot_f32(const f32* a, const f32* b, int n) {
    f32 r = 0.f;
    hip_check(qraf_hip_dot_f32(a, b, n, &r));
    return r;
}
void hip_dispatch_rms_norm(f32* x, const f32* w, int n, f32 eps) { hip_check(qraf_hip_rms_norm(x, w, n, eps)); }
void hip_dispatch_softmax(f32* x, int n) { hip_check(qraf_hip_softmax(x, n)); }
void hip_dispatch_silu(f32* x, int n) { hip_check(qraf_hip_silu(x, n)); }
void hip_dispatch_add(f32* x, const f32* y, int n) { hip_check(qraf_hip_add(x, y, n)); }
void hip_dispatch_mul(f32* x, const f32* y, int n) { hip_check(qraf_hip_mul(x, y, n)); }
void hip_dispatch_scale(f32* x, f32 s, int n) { hip_check(qraf_hip_scale(x, s, n)); }
void hip_dispatch_matvec_opt(const f32* W, const f32* x, f32* y, u32 out_dim, u32 in_dim) {
    hip_check(qraf_hip_matvec_f32(W, x, y, out_dim, in_dim));
}

// ---- HipBatchScheduler
class HipBatchScheduler {
public:
    // engine: created with max_batch >= max_rows rows per step and enough KV
    // pages for config.max_batch_size sequences of config.max_seq_len positions
    // eos: the end-of-sequence token (-1: the tokenizer's)
    HipBatchScheduler(qraf_engine* engine, u32 vocab, const Tokenizer& tokenizer, const BatchConfig& config = {},
                      u32 max_rows = 256, int64_t eos = -1)
        : e_(engine),
          vocab_(vocab),
          tokenizer_(tokenizer),
          config_(config),
          max_rows_(max_rows),
          eos_(eos >= 0 ? static_cast<u32>(eos) : tokenizer.eos_token()) {}
    ~HipBatchScheduler() { stop(); }

    u32 submit(const std::string& prompt, u32 max_tokens, const SamplingConfig& sampling = {},
               std::function<void(u32, const std::string&)> on_token = nullptr,
               std::function<void(const std::string&, u32, double)> on_complete = nullptr) {
        return submit_tokens(tokenizer_.encode(prompt), max_tokens, sampling, on_token, on_complete);
    }
    // the same for a caller that tokenized the prompt itself
    u32 submit_tokens(std::vector<u32> prompt_tokens, u32 max_tokens, const SamplingConfig& sampling = {},
                      std::function<void(u32, const std::string&)> on_token = nullptr,
                      std::function<void(const std::string&, u32, double)> on_complete = nullptr) {
        auto r = std::make_unique<Req>();
        r->req.id = next_id_++;
        r->req.prompt_tokens = std::move(prompt_tokens);
        r->req.max_tokens = max_tokens;
        r->req.sampling = sampling;
        r->req.on_token = on_token;
        r->req.on_complete = on_complete;
        const u32 id = r->req.id;
        {
            std::lock_guard<std::mutex> lk(mutex_);
            pending_.push_back(std::move(r));
        }
        cv_.notify_one();
        return id;
    }
    void start() {
        running_ = true;
        worker_ = std::thread([this]() { loop(); });
    }
    void stop() {
        running_ = false;
        cv_.notify_all();
        if (worker_.joinable()) worker_.join();
    }
    u32 active_requests() const { return active_count_; }
    u32 queued_requests() {
        std::lock_guard<std::mutex> lk(mutex_);
        return static_cast<u32>(pending_.size());
    }
    u32 total_processed() const { return total_processed_; }
    // The first error the worker met (empty: none); the worker stops at it.
    std::string error() {
        std::lock_guard<std::mutex> lk(mutex_);
        return error_;
    }
    // Logit rows read back to the host for every token chosen (turns the
    // pipelined path off): (request id, token index, logits [vocab]).
    std::function<void(u32, u32, const f32*)> on_logits;
    u64 steps_issued() const { return steps_; }
    u64 dropped_rows() const { return dropped_; }

private:
    struct Req {
        BatchRequest req;
        int32_t seq = -1;
        u32 fed = 0;          // prompt tokens fed
        u32 inflight = 0;     // its logit rows in steps not yet collected
        bool done = false;    // finished: rows still in flight are dropped
        std::mt19937 rng;
        std::chrono::steady_clock::time_point t0;
        bool greedy() const {
            const SamplingConfig& s = req.sampling;
            return (s.deterministic || s.temperature <= 0.f) && s.repetition_penalty == 1.0f;
        }
    };
    struct Flight {  // a step issued and not yet collected: the owner of each logit row
        std::vector<Req*> owners;
    };

    void loop() {
        try {
            while (true) {
                admit();
                if (!running_ && active_.empty() && flight_.empty()) break;
                if (active_.empty() && flight_.empty()) {
                    std::unique_lock<std::mutex> lk(mutex_);
                    cv_.wait_for(lk, std::chrono::milliseconds(1), [this]() { return !pending_.empty() || !running_; });
                    continue;
                }
                bool pipelined = !on_logits;
                for (auto& r : active_) pipelined = pipelined && r->greedy();
                // greedy-only steps need no logits: the head's argmax runs in
                // its GEMM where it can; the sampling path keeps them
                hip_check(qraf_engine_set_keep_logits(e_, pipelined ? 0 : 1));
                if (pipelined) step_pipelined();
                else step_sync();
                retire();
            }
        } catch (const std::exception& x) {
            std::lock_guard<std::mutex> lk(mutex_);
            error_ = x.what();
        }
    }

    // After stop() the active requests finish and queued ones stay queued.
    void admit() {
        std::lock_guard<std::mutex> lk(mutex_);
        while (running_ && !pending_.empty() && active_.size() < config_.max_batch_size) {
            std::unique_ptr<Req> r = std::move(pending_.front());
            pending_.pop_front();
            hip_check(qraf_engine_seq_create(e_, &r->seq));
            const SamplingConfig& s = r->req.sampling;
            r->rng.seed(s.seed != 0 ? static_cast<unsigned>(s.seed) : std::random_device{}());  // as Sampler does
            r->req.state = BatchRequest::State::PREFILLING;
            r->t0 = std::chrono::steady_clock::now();
            active_.push_back(std::move(r));
        }
        active_count_ = static_cast<u32>(active_.size());
    }

    // Rows of the next step: a decode row for every decoding request that
    // may still produce a token (decode rows first), then prompt chunks
    // within the row budget; a request's prompt ends with a logit row.
    // prev: the step in flight (decode rows take their token from it where
    // the request's last token is still there).
    void plan(const Flight* prev, std::vector<int32_t>& seq, std::vector<u32>& tok, std::vector<int32_t>& src,
              std::vector<int32_t>& pos, std::vector<uint8_t>& want, Flight& f) {
        for (auto& rp : active_) {
            Req& r = *rp;
            if (r.done || r.fed < r.req.prompt_tokens.size()) continue;
            if (r.req.generated_tokens.size() + r.inflight >= r.req.max_tokens) continue;
            int32_t s = -1;
            if (r.inflight) {  // its last token is still in the step in flight
                for (size_t k = 0; prev && k < prev->owners.size(); k++)
                    if (prev->owners[k] == &r) s = static_cast<int32_t>(k);
                if (s < 0) continue;  // older than the previous step: wait for it
            }
            if (r.req.generated_tokens.empty() && s < 0) continue;
            seq.push_back(r.seq);
            tok.push_back(s < 0 ? r.req.generated_tokens.back() : 0);
            src.push_back(s);
            pos.push_back(r.req.current_pos++);
            want.push_back(1);
            f.owners.push_back(&r);
            r.inflight++;
        }
        for (auto& rp : active_) {
            Req& r = *rp;
            const u32 n = static_cast<u32>(r.req.prompt_tokens.size());
            while (!r.done && r.fed < n && seq.size() < max_rows_) {
                const bool last = r.fed + 1 == n;
                seq.push_back(r.seq);
                tok.push_back(r.req.prompt_tokens[r.fed]);
                src.push_back(-1);
                pos.push_back(r.req.current_pos++);
                want.push_back(last ? 1 : 0);
                if (last) {
                    f.owners.push_back(&r);
                    r.inflight++;
                    r.req.state = BatchRequest::State::DECODING;
                }
                r.fed++;
            }
        }
    }

    // A token chosen for r: EOS or the token budget ends it (EOS is not
    // kept), as BatchScheduler::decode_step (batch_scheduler.h:205-222).
    void deliver(Req& r, u32 token) {
        r.inflight--;
        if (r.done) {
            dropped_++;
            return;
        }
        if (token == eos_ || r.req.generated_tokens.size() >= r.req.max_tokens) {
            r.done = true;
            return;
        }
        r.req.generated_tokens.push_back(token);
        if (r.req.on_token) r.req.on_token(token, tokenizer_.decode(token));
        if (r.req.generated_tokens.size() >= r.req.max_tokens) r.done = true;
    }

    void step_pipelined() {
        std::vector<int32_t> seq, src, pos;
        std::vector<u32> tok;
        std::vector<uint8_t> want;
        Flight f;
        plan(flight_.empty() ? nullptr : &flight_.back(), seq, tok, src, pos, want, f);
        if (!seq.empty()) {
            hip_check(qraf_engine_step_async(e_, static_cast<int32_t>(seq.size()), seq.data(), tok.data(), src.data(),
                                             pos.data(), want.data()));
            steps_++;
            flight_.push_back(std::move(f));
        }
        // collect the oldest step when two are in flight (or nothing new was issued)
        if (flight_.size() == 2 || (seq.empty() && !flight_.empty())) collect();
    }

    void collect() {
        Flight f = std::move(flight_.front());
        flight_.pop_front();
        std::vector<u32> toks(f.owners.size());
        int32_t k = 0;
        hip_check(qraf_engine_step_collect(e_, toks.data(), &k));
        if (k != static_cast<int32_t>(f.owners.size())) throw InferenceError("step_collect: row count mismatch");
        for (size_t i = 0; i < f.owners.size(); i++) deliver(*f.owners[i], toks[i]);
    }

    void step_sync() {
        while (!flight_.empty()) collect();  // leaving the pipelined path
        std::vector<int32_t> seq, src, pos;
        std::vector<u32> tok;
        std::vector<uint8_t> want;
        Flight f;
        plan(nullptr, seq, tok, src, pos, want, f);
        if (seq.empty()) return;
        const size_t k = f.owners.size();
        std::vector<f32> logits(on_logits ? k * vocab_ : 0);
        hip_check(qraf_engine_step(e_, static_cast<int32_t>(seq.size()), seq.data(), tok.data(), pos.data(),
                                   want.data(), on_logits ? logits.data() : nullptr, nullptr));
        steps_++;
        for (size_t i = 0; i < k; i++) {
            Req& r = *f.owners[i];
            const SamplingConfig& s = r.req.sampling;
            qraf_sampling_params sp{(s.deterministic ? 0.f : s.temperature), s.top_k, s.top_p, s.repetition_penalty};
            const std::vector<u32>& hist = r.req.generated_tokens;  // the recent tokens decode_step passes
            const int32_t cnt = static_cast<int32_t>(hist.size());
            float u = 0.f;
            if (sp.temperature > 0.f) u = std::uniform_real_distribution<f32>(0.0f, 1.0f)(r.rng);  // Sampler::sample
            u32 t = 0;
            if (on_logits) {  // host copy for the caller first: the sampler penalises the device rows in place
                on_logits(r.req.id, static_cast<u32>(hist.size()), logits.data() + i * vocab_);
            }
            hip_check(qraf_engine_sample(e_, static_cast<int32_t>(i), 1, &sp, cnt ? hist.data() : nullptr,
                                         cnt ? &cnt : nullptr, cnt, sp.temperature > 0.f ? &u : nullptr, &t));
            deliver(r, t);
        }
    }

    void retire() {
        for (size_t i = 0; i < active_.size();) {
            Req& r = *active_[i];
            if (!(r.done && r.inflight == 0)) {
                i++;
                continue;
            }
            r.req.state = BatchRequest::State::DONE;
            hip_check(qraf_engine_seq_release(e_, r.seq));
            const double ms =
                std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - r.t0).count();
            if (r.req.on_complete)
                r.req.on_complete(tokenizer_.decode(r.req.generated_tokens),
                                  static_cast<u32>(r.req.generated_tokens.size()), ms);
            active_.erase(active_.begin() + static_cast<long>(i));
            total_processed_++;
        }
        active_count_ = static_cast<u32>(active_.size());
    }

    qraf_engine* e_;
    u32 vocab_;
    const Tokenizer& tokenizer_;
    BatchConfig config_;
    u32 max_rows_;
    u32 eos_;
    std::deque<std::unique_ptr<Req>> pending_;
    std::vector<std::unique_ptr<Req>> active_;
    std::deque<Flight> flight_;
    std::thread worker_;
    std::mutex mutex_;
    std::condition_variable cv_;
    std::atomic<bool> running_{false};
    std::atomic<u32> next_id_{1};
    std::atomic<u32> total_processed_{0};
    std::atomic<u32> active_count_{0};
    std::string error_;
    u64 steps_ = 0, dropped_ = 0;
};

}  // namespace qraf

using namespace qraf;

static int g_fail = 0;

static void expect(bool ok, const char* what) {
    std::printf("%s: %s\n", what, ok ? "ok" : "FAILED");
    if (!ok) g_fail = 1;
}

// The elementwise branches against the reference's dispatch_* (scalar x86
// backend): add / mul / scale bit for bit; rms_norm, softmax, silu to a few
// fp32 ulp (a reduction tree instead of the sequential sum; the device expf);
// dot and the f32 matvec within 2 (n + 2) 2^-24 sum |a b|.
static void check_elementwise(std::mt19937& rng) {
    std::normal_distribution<float> nd(0.f, 1.f);
    std::uniform_real_distribution<float> ud(0.5f, 1.5f);
    for (int n : {576, 2048, 3000}) {
        std::vector<f32> x(n), y(n), w(n);
        for (int i = 0; i < n; i++) {
            x[i] = 3.f * nd(rng);
            y[i] = nd(rng);
            w[i] = ud(rng);
        }
        double worst = 0;
        auto rel = [&](const std::vector<f32>& a, const std::vector<f32>& b, double rtol, double atol) {
            for (int i = 0; i < n; i++)
                worst = std::max(worst, std::fabs((double)a[i] - b[i]) / (rtol * std::fabs((double)b[i]) + atol));
        };
        std::vector<f32> a = x, b = x;
        dispatch_rms_norm(a.data(), w.data(), n, 1e-5f);
        hip_dispatch_rms_norm(b.data(), w.data(), n, 1e-5f);
        rel(b, a, 2e-6, 1e-7);
        a = x;
        b = x;
        dispatch_softmax(a.data(), n);
        hip_dispatch_softmax(b.data(), n);
        rel(b, a, 1e-5, 1e-9);
        a = x;
        b = x;
        dispatch_silu(a.data(), n);
        hip_dispatch_silu(b.data(), n);
        rel(b, a, 4e-7, 1e-30);
        bool exact = true;
        a = x;
        b = x;
        dispatch_add(a.data(), y.data(), n);
        hip_dispatch_add(b.data(), y.data(), n);
        exact = exact && a == b;
        a = x;
        b = x;
        dispatch_mul(a.data(), y.data(), n);
        hip_dispatch_mul(b.data(), y.data(), n);
        exact = exact && a == b;
        a = x;
        b = x;
        dispatch_scale(a.data(), 0.37f, n);
        hip_dispatch_scale(b.data(), 0.37f, n);
        exact = exact && a == b;
        double mag = 0;
        for (int i = 0; i < n; i++) mag += std::fabs((double)x[i] * y[i]);
        const f32 dr = dispatch_dot_f32(x.data(), y.data(), n), dh = hip_dispatch_dot_f32(x.data(), y.data(), n);
        const bool dot_ok = std::fabs((double)dr - dh) <= 2.0 * (n + 2) * std::ldexp(1.0, -24) * mag;
        // f32 matvec (dispatch_matvec_opt) on a 300 x n matrix
        const u32 N = 300;
        std::vector<f32> W((size_t)N * n), yr(N), yh(N);
        for (auto& v : W) v = 0.02f * nd(rng);
        dispatch_matvec_opt(W.data(), x.data(), yr.data(), N, n);
        hip_dispatch_matvec_opt(W.data(), x.data(), yh.data(), N, n);
        double mv = 0;
        for (u32 i = 0; i < N; i++) {
            double m = 0;
            for (int k = 0; k < n; k++) m += std::fabs((double)W[(size_t)i * n + k] * x[k]);
            mv = std::max(mv, std::fabs((double)yh[i] - yr[i]) / (2.0 * (n + 2) * std::ldexp(1.0, -24) * m + 1e-30));
        }
        std::printf("elementwise n=%d: rms_norm/softmax/silu worst error / tolerance %.3g, add/mul/scale %s, dot %s, "
                    "matvec_opt worst / bound %.3g\n",
                    n, worst, exact ? "bit-identical" : "DIFFER", dot_ok ? "within bound" : "OUT OF BOUND", mv);
        if (!(worst <= 1.0) || !exact || !dot_ok || !(mv <= 1.0)) g_fail = 1;
    }
}

struct RefStream {
    std::vector<u32> tokens;
    std::vector<std::vector<f32>> logits;  // the logits each token was chosen from
};

// One request decoded alone by the reference Transformer with
// BatchScheduler::decode_step's loop (batch_scheduler.h:187-228), greedy.
static RefStream reference_decode(Transformer& ref, const std::vector<u32>& prompt, u32 max_tokens, u32 eos,
                                  u32 vocab) {
    RefStream out;
    ref.reset();
    int pos = 0;
    Tensor last;
    for (u32 t : prompt) last = ref.forward(t, pos++);
    SamplingConfig sc;
    sc.temperature = 0.f;
    sc.repetition_penalty = 1.0f;
    Sampler s(sc);
    while (true) {
        const f32* lg = last.data_f32();
        std::vector<f32> copy(lg, lg + vocab);
        const u32 t = s.sample(lg, static_cast<int>(vocab));
        if (t == eos || out.tokens.size() >= max_tokens) break;
        out.tokens.push_back(t);
        out.logits.push_back(std::move(copy));
        last = ref.forward(t, pos++);
    }
    return out;
}

struct Work {
    std::vector<u32> prompt;
    u32 max_tokens;
};

// Runs the requests through a HipBatchScheduler; `with_logits` reads every
// logit row back (the unpipelined path).  Requests are submitted in two
// halves, the second while the first runs.
static std::vector<RefStream> run_scheduler(qraf_engine* e, u32 vocab, const Tokenizer& tk, const std::vector<Work>& w,
                                            bool with_logits, u64* steps, u64* dropped, int64_t eos = -1) {
    BatchConfig bc;
    bc.max_batch_size = 6;
    bc.max_seq_len = 128;
    HipBatchScheduler sched(e, vocab, tk, bc, 32, eos);
    std::vector<RefStream> got(w.size());
    std::mutex mu;
    std::vector<u32> ids;
    if (with_logits)
        sched.on_logits = [&](u32 id, u32 index, const f32* lg) {
            std::lock_guard<std::mutex> lk(mu);
            RefStream& g = got[id - 1];
            if (g.logits.size() == index) g.logits.emplace_back(lg, lg + vocab);
        };
    SamplingConfig greedy;
    greedy.temperature = 0.f;
    greedy.repetition_penalty = 1.0f;
    auto submit = [&](size_t i) {
        sched.submit_tokens(w[i].prompt, w[i].max_tokens, greedy, [&got, &mu, i](u32 t, const std::string&) {
            std::lock_guard<std::mutex> lk(mu);
            got[i].tokens.push_back(t);
        });
    };
    const size_t half = w.size() / 2;
    for (size_t i = 0; i < half; i++) submit(i);
    sched.start();
    std::this_thread::sleep_for(std::chrono::milliseconds(5));
    for (size_t i = half; i < w.size(); i++) submit(i);
    const auto t0 = std::chrono::steady_clock::now();
    while (sched.total_processed() < w.size() && sched.error().empty()) {
        std::this_thread::sleep_for(std::chrono::milliseconds(1));
        if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(60)) throw InferenceError("scheduler timeout");
    }
    sched.stop();
    if (!sched.error().empty()) throw InferenceError("scheduler: " + sched.error());
    *steps = sched.steps_issued();
    *dropped = sched.dropped_rows();
    return got;
}

int main(int argc, char** argv) {
    if (argc < 4) {
        std::fprintf(stderr, "usage: %s <model.qraf> <requests> <seed>\n", argv[0]);
        return 2;
    }
    const int nreq = std::atoi(argv[2]);
    log::set_level(log::Level::ERROR);
    backend_init();  // the reference's scalar x86 backend
    try {
        int devs = 0;
        hip_check(qraf_hip_device_count(&devs));
        if (devs < 1) throw InferenceError("no GPU");
        hip_check(qraf_hip_init(0));
        std::mt19937 rng(static_cast<unsigned>(std::atoi(argv[3])));
        check_elementwise(rng);

        QrafModel model;
        if (!model.load(argv[1])) throw InferenceError(std::string("cannot load ") + argv[1]);
        Transformer ref;
        if (!ref.init(model)) throw InferenceError("reference Transformer::init failed");
        const u32 vocab = model.config().vocab_size;
        Tokenizer tk;  // no vocabulary: token ids in, token ids out; EOS = its default id
        const u32 eos = tk.eos_token();

        std::vector<Work> w(nreq);
        std::uniform_int_distribution<int> plen(1, 40), glen(8, 40);
        std::uniform_int_distribution<u32> tokd(0, vocab - 1);
        for (auto& x : w) {
            x.prompt.resize(plen(rng));
            for (auto& t : x.prompt) t = tokd(rng);
            x.max_tokens = static_cast<u32>(glen(rng));
        }
        std::vector<RefStream> want;
        size_t eos_stops = 0;
        for (const auto& x : w) {
            want.push_back(reference_decode(ref, x.prompt, x.max_tokens, eos, vocab));
            eos_stops += want.back().tokens.size() < x.max_tokens;
        }
        std::printf("%d requests, reference streams of %zu tokens in all, %zu stopped by EOS\n", nreq,
                    [&]() {
                        size_t s = 0;
                        for (auto& r : want) s += r.tokens.size();
                        return s;
                    }(),
                    eos_stops);

        qraf_engine* e = nullptr;
        qraf_engine_options eo{/*kv_dtype*/ 0 /*F32*/, /*page_size*/ 16, /*max_batch*/ 32, /*num_pages*/ 0};
        hip_check(qraf_engine_create_from_file(argv[1], &eo, &e));
        u64 steps = 0, dropped = 0;
        std::vector<RefStream> got = run_scheduler(e, vocab, tk, w, false, &steps, &dropped);
        size_t same = 0;
        for (int i = 0; i < nreq; i++) same += got[i].tokens == want[i].tokens;
        std::printf("pipelined: %llu steps, %llu rows dropped after EOS, streams equal %zu/%d\n",
                    (unsigned long long)steps, (unsigned long long)dropped, same, nreq);
        expect(same == (size_t)nreq, "pipelined streams equal the reference's");

        got = run_scheduler(e, vocab, tk, w, true, &steps, &dropped);
        same = 0;
        double worst = 0;
        size_t checked = 0;
        for (int i = 0; i < nreq; i++) {
            same += got[i].tokens == want[i].tokens;
            const size_t n = std::min<size_t>({32, got[i].logits.size(), want[i].logits.size()});
            for (size_t j = 0; j < n; j++, checked++)
                for (u32 v = 0; v < vocab; v++) {
                    const double r = want[i].logits[j][v], h = got[i].logits[j][v];
                    worst = std::max(worst, std::fabs(h - r) / (1e-3 * std::fabs(r) + 1e-4));
                }
        }
        std::printf("logit rows read back: %llu steps, streams equal %zu/%d, %zu logit vectors of the first 32 "
                    "tokens, worst error / tolerance %.4f\n",
                    (unsigned long long)steps, same, nreq, checked, worst);
        expect(same == (size_t)nreq && worst <= 1.0 && checked > 0, "logits and streams against the reference");

        // EOS stops: the token the reference generates most often as EOS, so that
        // requests end early and the pipelined run drops the rows it had already
        // issued for them
        std::vector<size_t> freq(vocab, 0);
        for (const auto& r : want)
            for (u32 t : r.tokens) freq[t]++;
        const u32 eos2 = static_cast<u32>(std::max_element(freq.begin(), freq.end()) - freq.begin());
        std::vector<RefStream> want2;
        eos_stops = 0;
        for (const auto& x : w) {
            want2.push_back(reference_decode(ref, x.prompt, x.max_tokens, eos2, vocab));
            eos_stops += want2.back().tokens.size() < x.max_tokens;
        }
        got = run_scheduler(e, vocab, tk, w, false, &steps, &dropped, eos2);
        same = 0;
        for (int i = 0; i < nreq; i++) same += got[i].tokens == want2[i].tokens;
        std::printf("EOS = token %u: %zu requests stopped by it, pipelined %llu steps, %llu rows dropped after EOS, "
                    "streams equal %zu/%d\n",
                    eos2, eos_stops, (unsigned long long)steps, (unsigned long long)dropped, same, nreq);
        expect(same == (size_t)nreq && eos_stops > 0 && dropped > 0, "EOS stops against the reference");
        hip_check(qraf_engine_destroy(e));
    } catch (const std::exception& x) {
        std::printf("error: %s\n", x.what());
        return 1;
    }
    std::printf(g_fail ? "FAIL\n" : "PASS\n");
    return g_fail;
}
