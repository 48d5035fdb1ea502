/*
 * qraf_hip.h -- C ABI of the MI355X (gfx950) QRAF decode hot path.
 *
 * A drop-in for the dispatch layer of simonpierreboucher02/qraf
 * (include/nn/backend.h, src/nn/backend.cpp) and for the per-token engine
 * below it (src/nn/transformer.cpp, src/nn/attention.cpp).  Plain C types
 * only: pointers, sizes, dtype codes of include/core/types.h:27-39
 * (F32 = 0, F16 = 1, Q8_0 = 10, Q4_0 = 20) and block sizes from
 * QuantScheme.block_size (include/qraf/format.h:88-97).
 *
 * Every function returns QRAF_HIP_OK (0) or a negative QRAF_HIP_ERR_* code;
 * qraf_hip_last_error() describes the calling thread's last failure.  Where
 * the reference silently zero-fills (unknown dtype in dispatch_matvec_q,
 * backend.cpp:195-198) this library returns QRAF_HIP_ERR_DTYPE instead; the
 * C++ shim in INTEGRATION.md turns nonzero codes into qraf::QrafError.
 *
 * Pointer kinds: functions named *_dev take device pointers and a stream
 * (hipStream_t passed as void*, NULL = the library's default stream) and
 * are stream-ordered; every other compute function takes host pointers and
 * returns after its result is in host memory.
 */
#ifndef QRAF_HIP_H
#define QRAF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QRAF_HIP_OK 0
#define QRAF_HIP_ERR_INVALID (-1) /* bad argument or shape            */
#define QRAF_HIP_ERR_DTYPE (-2)   /* unsupported dtype / block size    */
#define QRAF_HIP_ERR_HIP (-3)     /* HIP runtime failure               */
#define QRAF_HIP_ERR_NOMEM (-4)   /* device or page-pool exhaustion    */
#define QRAF_HIP_ERR_STATE (-5)   /* call not valid in the current state */

#define QRAF_DTYPE_F32 0u
#define QRAF_DTYPE_F16 1u
#define QRAF_DTYPE_Q8_0 10u
#define QRAF_DTYPE_Q4_0 20u

/* ------------------------------------------------------------ runtime */

/* Last error of the calling thread ("" if none). */
const char* qraf_hip_last_error(void);
/* Select the device and create the library's default stream.  Replaces
 * backend_init() (backend.cpp:18-50) for the HIP backend; idempotent. */
int qraf_hip_init(int device);
int qraf_hip_device_count(int* count);
/* Build information: "gfx950 <compiler version>". */
const char* qraf_hip_version(void);

/* Device memory, streams, events and graphs, so callers need no HIP headers. */
int qraf_hip_malloc(void** dev_ptr, uint64_t bytes);
int qraf_hip_free(void* dev_ptr);
int qraf_hip_memcpy_h2d(void* dst_dev, const void* src_host, uint64_t bytes);
int qraf_hip_memcpy_d2h(void* dst_host, const void* src_dev, uint64_t bytes);
int qraf_hip_memcpy_d2d(void* dst_dev, const void* src_dev, uint64_t bytes, void* stream);
int qraf_hip_memset(void* dev_ptr, int value, uint64_t bytes);
int qraf_hip_stream_create(void** stream);
int qraf_hip_stream_destroy(void* stream);
int qraf_hip_stream_synchronize(void* stream);
int qraf_hip_device_synchronize(void);
int qraf_hip_event_create(void** event);
int qraf_hip_event_destroy(void* event);
int qraf_hip_event_record(void* event, void* stream);
int qraf_hip_event_elapsed_ms(void* start, void* stop, float* ms);
/* Capture stream-ordered library calls made on `stream` into a graph. */
int qraf_hip_graph_begin(void* stream);
int qraf_hip_graph_end(void* stream, void** graph_exec);
int qraf_hip_graph_launch(void* graph_exec, void* stream);
int qraf_hip_graph_destroy(void* graph_exec);

/* ------------------------------------------------ op level (backend.h) */

/* Weight residency for the op-level calls: a host weight buffer registered
 * here is copied to HBM once and every later op-level call that passes the
 * same host pointer reads the HBM copy.  Mirrors how the reference keeps
 * weights as immutable mmap views (loader.cpp:236-258). */
int qraf_hip_register_weights(const void* host_ptr, uint64_t bytes);
int qraf_hip_unregister_weights(const void* host_ptr);

/* dispatch_matvec_q (backend.h:35-38, backend.cpp:131-199):
 * y[i] = dot(row_i(w), x) for i < out_dim; w in the reference's Q8_0/Q4_0
 * block layout with `block_size` (0 means 32, as backend.cpp:135).
 * w_size may be 0 (unchecked, as the reference) or the buffer size. */
int qraf_hip_matvec_q(const void* w, uint64_t w_size, uint32_t dtype, uint32_t block_size,
                      uint32_t out_dim, uint32_t in_dim, const float* x, float* y);
/* dispatch_matvec_opt (backend.h:31-32, backend.cpp:62-105). */
int qraf_hip_matvec_f32(const float* W, const float* x, float* y, uint32_t out_dim, uint32_t in_dim);
/* dispatch_dot_f32 (backend.h:41, backend.cpp:109-127). */
int qraf_hip_dot_f32(const float* a, const float* b, int n, float* result);
/* dispatch_rms_norm / softmax / silu / add / mul / scale
 * (backend.h:44-49, backend.cpp:203-320). */
int qraf_hip_rms_norm(float* x, const float* weight, int size, float eps);
int qraf_hip_softmax(float* x, int size);
int qraf_hip_silu(float* x, int size);
int qraf_hip_add(float* x, const float* y, int size);
int qraf_hip_mul(float* x, const float* y, int size);
int qraf_hip_scale(float* x, float s, int size);

/* --------------------------------------------------- device level */

/* Device-pointer form of qraf_hip_matvec_q; stream-ordered. */
int qraf_hip_matvec_q_dev(const void* w, uint32_t dtype, uint32_t block_size, uint32_t out_dim,
                          uint32_t in_dim, const float* x, float* y, void* stream);
int qraf_hip_matvec_f32_dev(const float* W, const float* x, float* y, uint32_t out_dim,
                            uint32_t in_dim, void* stream);
/* Tuning of the batch-1 kernel (process-wide): kernel 0 = automatic,
 * 1 = one-shot, 2 = persistent streaming; rows per wave 0 (automatic), 1, 2,
 * 4 or 8; workgroups per CU for the persistent kernel (0 = automatic). */
int qraf_hip_set_matvec_tuning(int kernel, int rows, int wgs_per_cu);

/* quantize_q8_0 / quantize_q4_0 (quantize.cpp:105-183) on the device, block
 * size 32, bit-exact with the reference: `count` fp32 values -> `dst` in the
 * reference block layout (ceil(count/32) blocks). */
int qraf_hip_quantize_dev(const float* src, uint64_t count, uint32_t dtype, void* dst, void* stream);
/* Synthetic weights for benchmarks and tests (the role of
 * tools/dummy_model.cpp:12-17): `count` values N(0, stddev) from the
 * repository's counter-based generator (seed, stream_id), written as F32 or
 * quantized to Q8_0/Q4_0 as by qraf_hip_quantize_dev.  stream_id is
 * conventionally qraf_hip_name_hash(tensor name). */
int qraf_hip_gen_weights_dev(void* dst, uint32_t dtype, uint64_t count, uint64_t seed, uint64_t stream_id,
                             float stddev, void* stream);
/* FNV-1a of a tensor name (format.h:296-303); returns the hash itself. */
uint64_t qraf_hip_name_hash(const char* name);

#ifdef __cplusplus
}
#endif
#endif
