// api.hip -- the extern "C" surface declared in include/qraf_hip.h:
// runtime helpers, the op-level mirror of the reference's dispatch layer
// (backend.h:27-45) and the device-level entry points.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <vector>

#include "common.h"

namespace qraf_hip {

// Per-process device state.  One default stream per device the library was
// initialised on; op-level calls serialise on g_mu (the reference's dispatch
// layer is single-threaded as well, backend.cpp:16).  g_dev itself is guarded
// by g_dev_mu, since device-level calls with a NULL stream look up their
// device's default stream without taking g_mu.
struct DeviceState {
    hipStream_t stream = nullptr;
    // op-level staging buffers, grown on demand
    void* buf[3] = {nullptr, nullptr, nullptr};
    size_t cap[3] = {0, 0, 0};
};
static std::mutex g_mu;
static std::mutex g_dev_mu;
static std::map<int, DeviceState> g_dev;
struct Registered {
    void* dev;
    uint64_t bytes;
};
static std::map<const void*, Registered> g_weights;  // host ptr -> HBM copy

// The current device's default stream, created on first use (g_dev_mu held).
static int stream_of_current(hipStream_t* out) {
    int d = 0;
    QH_CHECK_HIP(hipGetDevice(&d));
    DeviceState& st = g_dev[d];
    if (!st.stream) QH_CHECK_HIP(hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking));
    *out = st.stream;
    return QRAF_HIP_OK;
}

static int ensure_init() {
    std::lock_guard<std::mutex> lk(g_dev_mu);
    hipStream_t s;
    return stream_of_current(&s);
}

hipStream_t default_stream() {
    std::lock_guard<std::mutex> lk(g_dev_mu);
    hipStream_t s = nullptr;
    return stream_of_current(&s) == QRAF_HIP_OK ? s : nullptr;
}

// Staging buffer `i` of at least `bytes` on the current device (callers hold
// g_mu, which serialises the buffers' use; g_dev_mu covers the lookup).
static int staging(int i, size_t bytes, void** out) {
    int d = 0;
    QH_CHECK_HIP(hipGetDevice(&d));
    DeviceState* stp;
    {
        std::lock_guard<std::mutex> lk(g_dev_mu);
        stp = &g_dev[d];  // std::map nodes stay where they are when others are inserted
    }
    DeviceState& st = *stp;
    if (st.cap[i] < bytes) {
        if (st.buf[i]) QH_CHECK_HIP(hipFree(st.buf[i]));
        st.buf[i] = nullptr;
        st.cap[i] = 0;
        size_t n = bytes < 4096 ? 4096 : bytes;
        QH_CHECK_HIP(hipMalloc(&st.buf[i], n));
        st.cap[i] = n;
    }
    *out = st.buf[i];
    return QRAF_HIP_OK;
}

}  // namespace qraf_hip

using namespace qraf_hip;

extern "C" {


const char* qraf_hip_version(void) { return "gfx950 " __VERSION__; }

int qraf_hip_init(int device) {
    clear_error();
    std::lock_guard<std::mutex> lk(g_mu);
    int n = 0;
    QH_CHECK_HIP(hipGetDeviceCount(&n));
    QH_REQUIRE(device >= 0 && device < n, QRAF_HIP_ERR_INVALID, "device %d out of range (%d devices)", device, n);
    QH_CHECK_HIP(hipSetDevice(device));
    QH_TRY(ensure_init());
    QH_TRY(qgemm_kw_init());
    return attn_scratch_init(device);
}

int qraf_hip_device_count(int* count) {
    QH_REQUIRE(count, QRAF_HIP_ERR_INVALID, "null count");
    hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) {
        *count = 0;
        return set_error(QRAF_HIP_ERR_HIP, "hipGetDeviceCount: %s", hipGetErrorString(e));
    }
    return QRAF_HIP_OK;
}

int qraf_hip_malloc(void** p, uint64_t bytes) {
    QH_REQUIRE(p, QRAF_HIP_ERR_INVALID, "null out pointer");
    *p = nullptr;
    if (bytes == 0) return QRAF_HIP_OK;
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipErrorOutOfMemory)
        return set_error(QRAF_HIP_ERR_NOMEM, "hipMalloc(%llu) out of memory", (unsigned long long)bytes);
    QH_CHECK_HIP(e);
    return QRAF_HIP_OK;
}
int qraf_hip_free(void* p) {
    if (p) QH_CHECK_HIP(hipFree(p));
    return QRAF_HIP_OK;
}
int qraf_hip_memcpy_h2d(void* dst, const void* src, uint64_t n) {
    if (n) QH_CHECK_HIP(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
    return QRAF_HIP_OK;
}
int qraf_hip_memcpy_d2h(void* dst, const void* src, uint64_t n) {
    if (n) QH_CHECK_HIP(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
    return QRAF_HIP_OK;
}
int qraf_hip_memcpy_d2d(void* dst, const void* src, uint64_t n, void* stream) {
    if (n) QH_CHECK_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, as_stream(stream)));
    return QRAF_HIP_OK;
}
int qraf_hip_read_probe_dev(const void* p, uint64_t bytes, float* out, void* stream) {
    return qraf_hip::launch_read_probe(p, bytes, out, as_stream(stream));
}
uint64_t qraf_hip_read_probe_out_bytes(void) { return qraf_hip::read_probe_out_floats() * sizeof(float); }
int qraf_hip_launch_floor_dev(int32_t workgroups, void* stream) {
    return qraf_hip::launch_empty(workgroups, as_stream(stream));
}
int qraf_hip_memset(void* p, int v, uint64_t n) {
    if (n) QH_CHECK_HIP(hipMemset(p, v, n));
    return QRAF_HIP_OK;
}
int qraf_hip_stream_create(void** s) {
    QH_REQUIRE(s, QRAF_HIP_ERR_INVALID, "null out pointer");
    hipStream_t st;
    QH_CHECK_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = st;
    return QRAF_HIP_OK;
}
int qraf_hip_stream_destroy(void* s) {
    if (s) QH_CHECK_HIP(hipStreamDestroy((hipStream_t)s));
    return QRAF_HIP_OK;
}
int qraf_hip_stream_synchronize(void* s) {
    QH_CHECK_HIP(hipStreamSynchronize(as_stream(s)));
    return QRAF_HIP_OK;
}
int qraf_hip_device_synchronize(void) {
    QH_CHECK_HIP(hipDeviceSynchronize());
    return QRAF_HIP_OK;
}
int qraf_hip_event_create(void** e) {
    QH_REQUIRE(e, QRAF_HIP_ERR_INVALID, "null out pointer");
    hipEvent_t ev;
    QH_CHECK_HIP(hipEventCreate(&ev));
    *e = ev;
    return QRAF_HIP_OK;
}
int qraf_hip_event_destroy(void* e) {
    if (e) QH_CHECK_HIP(hipEventDestroy((hipEvent_t)e));
    return QRAF_HIP_OK;
}
int qraf_hip_event_record(void* e, void* s) {
    QH_CHECK_HIP(hipEventRecord((hipEvent_t)e, as_stream(s)));
    return QRAF_HIP_OK;
}
int qraf_hip_event_elapsed_ms(void* a, void* b, float* ms) {
    QH_REQUIRE(a && b && ms, QRAF_HIP_ERR_INVALID, "null event or out pointer");
    QH_CHECK_HIP(hipEventSynchronize((hipEvent_t)b));
    QH_CHECK_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return QRAF_HIP_OK;
}
int qraf_hip_graph_begin(void* s) {
    QH_CHECK_HIP(hipStreamBeginCapture(as_stream(s), hipStreamCaptureModeThreadLocal));
    return QRAF_HIP_OK;
}
int qraf_hip_graph_end(void* s, void** exec) {
    QH_REQUIRE(exec, QRAF_HIP_ERR_INVALID, "null out pointer");
    hipGraph_t g;
    QH_CHECK_HIP(hipStreamEndCapture(as_stream(s), &g));
    hipGraphExec_t ge;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    QH_CHECK_HIP(e);
    *exec = ge;
    return QRAF_HIP_OK;
}
int qraf_hip_graph_launch(void* exec, void* s) {
    QH_CHECK_HIP(hipGraphLaunch((hipGraphExec_t)exec, as_stream(s)));
    return QRAF_HIP_OK;
}
int qraf_hip_graph_destroy(void* exec) {
    if (exec) QH_CHECK_HIP(hipGraphExecDestroy((hipGraphExec_t)exec));
    return QRAF_HIP_OK;
}

// ------------------------------------------------------------ op level

int qraf_hip_register_weights(const void* host, uint64_t bytes) {
    clear_error();
    QH_REQUIRE(host && bytes, QRAF_HIP_ERR_INVALID, "null or empty weight buffer");
    std::lock_guard<std::mutex> lk(g_mu);
    QH_TRY(ensure_init());
    auto it = g_weights.find(host);
    if (it != g_weights.end()) {
        if (it->second.bytes >= bytes) return QRAF_HIP_OK;
        hipFree(it->second.dev);
        g_weights.erase(it);
    }
    void* d = nullptr;
    QH_CHECK_HIP(hipMalloc(&d, bytes));
    hipError_t e = hipMemcpy(d, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(d);
        return set_error(QRAF_HIP_ERR_HIP, "weight upload failed: %s", hipGetErrorString(e));
    }
    g_weights[host] = {d, bytes};
    return QRAF_HIP_OK;
}

int qraf_hip_unregister_weights(const void* host) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_weights.find(host);
    QH_REQUIRE(it != g_weights.end(), QRAF_HIP_ERR_INVALID, "weights not registered");
    QH_CHECK_HIP(hipFree(it->second.dev));
    g_weights.erase(it);
    return QRAF_HIP_OK;
}

// Device copy of host weights: the registered HBM copy, or a staging upload.
static int device_weights(const void* host, size_t need, void** dev) {
    auto it = g_weights.find(host);
    if (it != g_weights.end()) {
        QH_REQUIRE(it->second.bytes >= need, QRAF_HIP_ERR_INVALID,
                   "registered weight buffer is %llu bytes, matvec needs %llu",
                   (unsigned long long)it->second.bytes, (unsigned long long)need);
        *dev = it->second.dev;
        return QRAF_HIP_OK;
    }
    QH_TRY(staging(2, need, dev));
    QH_CHECK_HIP(hipMemcpy(*dev, host, need, hipMemcpyHostToDevice));
    return QRAF_HIP_OK;
}

int qraf_hip_matvec_q(const void* w, uint64_t w_size, uint32_t dtype, uint32_t block_size, uint32_t out_dim,
                      uint32_t in_dim, const float* x, float* y) {
    clear_error();
    QH_REQUIRE(w && x && y, QRAF_HIP_ERR_INVALID, "null pointer");
    QH_REQUIRE(dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "unsupported quantized dtype %u", dtype);
    int bs = block_size ? (int)block_size : 32;
    QH_REQUIRE(out_dim > 0 && in_dim > 0, QRAF_HIP_ERR_INVALID, "empty matvec");
    size_t need = q_row_bytes(dtype, bs, in_dim) * out_dim;
    QH_REQUIRE(w_size == 0 || w_size >= need, QRAF_HIP_ERR_INVALID,
               "weight buffer is %llu bytes, %u x %u needs %llu", (unsigned long long)w_size, out_dim, in_dim,
               (unsigned long long)need);
    std::lock_guard<std::mutex> lk(g_mu);
    QH_TRY(ensure_init());
    void *dw, *dx, *dy;
    QH_TRY(device_weights(w, need, &dw));
    QH_TRY(staging(0, (size_t)in_dim * 4, &dx));
    QH_TRY(staging(1, (size_t)out_dim * 4, &dy));
    hipStream_t s = default_stream();
    QH_CHECK_HIP(hipMemcpyAsync(dx, x, (size_t)in_dim * 4, hipMemcpyHostToDevice, s));
    QH_TRY(launch_matvec_q(dw, dtype, bs, out_dim, in_dim, (const float*)dx, (float*)dy, s));
    QH_CHECK_HIP(hipMemcpyAsync(y, dy, (size_t)out_dim * 4, hipMemcpyDeviceToHost, s));
    QH_CHECK_HIP(hipStreamSynchronize(s));
    return QRAF_HIP_OK;
}

int qraf_hip_matvec_f32(const float* W, const float* x, float* y, uint32_t out_dim, uint32_t in_dim) {
    clear_error();
    QH_REQUIRE(W && x && y && out_dim && in_dim, QRAF_HIP_ERR_INVALID, "bad f32 matvec arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    QH_TRY(ensure_init());
    size_t need = (size_t)out_dim * in_dim * 4;
    void *dw, *dx, *dy;
    QH_TRY(device_weights(W, need, &dw));
    QH_TRY(staging(0, (size_t)in_dim * 4, &dx));
    QH_TRY(staging(1, (size_t)out_dim * 4, &dy));
    hipStream_t s = default_stream();
    QH_CHECK_HIP(hipMemcpyAsync(dx, x, (size_t)in_dim * 4, hipMemcpyHostToDevice, s));
    QH_TRY(launch_matvec_f32((const float*)dw, (const float*)dx, (float*)dy, out_dim, in_dim, s));
    QH_CHECK_HIP(hipMemcpyAsync(y, dy, (size_t)out_dim * 4, hipMemcpyDeviceToHost, s));
    QH_CHECK_HIP(hipStreamSynchronize(s));
    return QRAF_HIP_OK;
}

// x (in/out, n floats) through the device; y (n floats, optional) as input.
static int run_vec_op(float* x, const float* y, int n, int (*body)(float*, const float*, int, hipStream_t, void*),
                      void* ctx, float* scalar_out) {
    QH_REQUIRE(x && n > 0, QRAF_HIP_ERR_INVALID, "bad vector arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    QH_TRY(ensure_init());
    void *dx, *dy = nullptr;
    QH_TRY(staging(0, (size_t)n * 4 + 16, &dx));
    if (y) QH_TRY(staging(1, (size_t)n * 4, &dy));
    hipStream_t s = default_stream();
    QH_CHECK_HIP(hipMemcpyAsync(dx, x, (size_t)n * 4, hipMemcpyHostToDevice, s));
    if (y) QH_CHECK_HIP(hipMemcpyAsync(dy, y, (size_t)n * 4, hipMemcpyHostToDevice, s));
    QH_TRY(body((float*)dx, (const float*)dy, n, s, ctx));
    if (scalar_out)
        QH_CHECK_HIP(hipMemcpyAsync(scalar_out, (float*)dx + n, 4, hipMemcpyDeviceToHost, s));
    else
        QH_CHECK_HIP(hipMemcpyAsync(x, dx, (size_t)n * 4, hipMemcpyDeviceToHost, s));
    QH_CHECK_HIP(hipStreamSynchronize(s));
    return QRAF_HIP_OK;
}

int qraf_hip_dot_f32(const float* a, const float* b, int n, float* result) {
    clear_error();
    QH_REQUIRE(a && b && result, QRAF_HIP_ERR_INVALID, "null pointer");
    return run_vec_op(
        const_cast<float*>(a), b, n,
        [](float* x, const float* y, int n, hipStream_t s, void*) { return launch_dot(x, y, n, x + n, s); },
        nullptr, result);
}

int qraf_hip_rms_norm(float* x, const float* weight, int size, float eps) {
    clear_error();
    QH_REQUIRE(weight, QRAF_HIP_ERR_INVALID, "null weight");
    return run_vec_op(
        x, weight, size,
        [](float* x, const float* w, int n, hipStream_t s, void* c) {
            return launch_rms_norm(x, w, n, *(float*)c, s);
        },
        &eps, nullptr);
}

int qraf_hip_softmax(float* x, int size) {
    clear_error();
    return run_vec_op(
        x, nullptr, size, [](float* x, const float*, int n, hipStream_t s, void*) { return launch_softmax(x, n, s); },
        nullptr, nullptr);
}

int qraf_hip_silu(float* x, int size) {
    clear_error();
    return run_vec_op(
        x, nullptr, size,
        [](float* x, const float*, int n, hipStream_t s, void*) { return launch_ew(0, x, nullptr, 0.f, n, s); },
        nullptr, nullptr);
}

int qraf_hip_add(float* x, const float* y, int size) {
    clear_error();
    QH_REQUIRE(y, QRAF_HIP_ERR_INVALID, "null y");
    return run_vec_op(
        x, y, size, [](float* x, const float* y, int n, hipStream_t s, void*) { return launch_ew(1, x, y, 0.f, n, s); },
        nullptr, nullptr);
}

int qraf_hip_mul(float* x, const float* y, int size) {
    clear_error();
    QH_REQUIRE(y, QRAF_HIP_ERR_INVALID, "null y");
    return run_vec_op(
        x, y, size, [](float* x, const float* y, int n, hipStream_t s, void*) { return launch_ew(2, x, y, 0.f, n, s); },
        nullptr, nullptr);
}

int qraf_hip_scale(float* x, float sc, int size) {
    clear_error();
    return run_vec_op(
        x, nullptr, size,
        [](float* x, const float*, int n, hipStream_t s, void* c) { return launch_ew(3, x, nullptr, *(float*)c, n, s); },
        &sc, nullptr);
}

// ------------------------------------------------------------ device level

int qraf_hip_matvec_q_dev(const void* w, uint32_t dtype, uint32_t block_size, uint32_t out_dim, uint32_t in_dim,
                          const float* x, float* y, void* stream) {
    clear_error();
    return launch_matvec_q(w, dtype, block_size ? (int)block_size : 32, out_dim, in_dim, x, y, as_stream(stream));
}

int qraf_hip_matvec_q_batch_dev(const void* w, uint32_t dtype, uint32_t out_dim, uint32_t in_dim, const float* x,
                                int32_t batch, float* y, void* stream) {
    clear_error();
    return launch_matvec_q_batch(w, dtype, out_dim, in_dim, x, (int)in_dim, (int)batch, y, (int)out_dim,
                                 as_stream(stream));
}

int qraf_hip_matvec_f32_dev(const float* W, const float* x, float* y, uint32_t out_dim, uint32_t in_dim,
                            void* stream) {
    clear_error();
    return launch_matvec_f32(W, x, y, out_dim, in_dim, as_stream(stream));
}

int qraf_hip_set_matvec_tuning(int kernel, int rows, int wgs_per_cu) {
    return set_matvec_tuning(kernel, rows, wgs_per_cu);
}

}  // extern "C"
