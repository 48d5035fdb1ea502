// quant.hip -- device Q8_0 / Q4_0 quantizer and synthetic weight generator.
//
// quantize_q8_0 / quantize_q4_0 (reference quantize.cpp:105-183) and the
// truncating fp32->fp16 encoder they use (dtype.cpp:39-59), one thread per
// 32-element block, bit-exact with the reference: every step is a correctly
// rounded fp32 operation (the build keeps IEEE division and fp32 denormals)
// or integer bit manipulation.  The generator produces the repository's
// synthetic N(0, std) weights: an 8-term Irwin-Hall sum of 16-bit fields of
// two splitmix64 hashes per element, scaled by one fp32 multiply (the scale
// is computed once on the host in double precision), so a CPU restatement
// reproduces the same bits.  It stands in for tools/dummy_model.cpp:12-17,
// whose std::mt19937 stream a GPU cannot reproduce.
#include <math.h>

#include "common.h"

namespace qraf_hip {

constexpr int QB = 32;  // device quantizer block size

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
static inline uint64_t mix64_host(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float gen_value(uint64_t base, uint64_t idx, float c) {
    uint64_t h1 = mix64(base + 2 * idx), h2 = mix64(base + 2 * idx + 1);
    int32_t s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) s += (int32_t)((h1 >> (16 * k)) & 0xFFFFu) + (int32_t)((h2 >> (16 * k)) & 0xFFFFu);
    return (float)(2 * s - 8 * 65535) * c;
}

// dtype.cpp:39-59
__device__ __forceinline__ uint16_t fp32_to_fp16_trunc(float f) {
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (b >> 31) & 1u;
    int32_t ex = (int32_t)((b >> 23) & 0xFFu) - 127;
    if (ex > 15) return (uint16_t)((sign << 15) | 0x7C00u);
    if (ex > -15) return (uint16_t)((sign << 15) | ((uint32_t)(ex + 15) << 10) | ((b & 0x7FFFFFu) >> 13));
    return (uint16_t)(sign << 15);
}

// std::min(hi, v) / std::max(lo, v) with libstdc++'s comparison order.
__device__ __forceinline__ float std_min(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ float std_max(float a, float b) { return (a < b) ? b : a; }

// Quantize v[0..tb) (tb <= 32) of one block into `out` (block layout of
// quantize.cpp).  Bytes of elements >= tb stay zero.
__device__ void quantize_block(const float* v, int tb, uint32_t dtype, uint8_t* out) {
    float max_abs = 0.0f;
    for (int i = 0; i < tb; i++) {
        float a = fabsf(v[i]);
        if (a > max_abs) max_abs = a;
    }
    if (dtype == DT_Q8_0) {
        float scale = max_abs / 127.0f;
        float inv = (scale > 0.0f) ? 1.0f / scale : 0.0f;
        uint32_t w[9];
        w[0] = __builtin_bit_cast(uint32_t, scale);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t d = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                int i = 4 * j + k;
                if (i < tb) {
                    float x = std_max(-127.0f, std_min(127.0f, v[i] * inv));
                    d |= ((uint32_t)(uint8_t)(int8_t)roundf(x)) << (8 * k);
                }
            }
            w[1 + j] = d;
        }
        uint32_t* o = (uint32_t*)out;  // 4-byte aligned: blocks are 36 B
#pragma unroll
        for (int j = 0; j < 9; j++) o[j] = w[j];
    } else {
        float scale = max_abs / 7.0f;
        float inv = (scale > 0.0f) ? 1.0f / scale : 0.0f;
        uint16_t h[9];
        h[0] = fp32_to_fp16_trunc(scale);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint16_t d = 0;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                int p = 2 * j + k;  // byte index
                if (p < tb / 2) {
                    float v0 = std_max(-8.0f, std_min(7.0f, roundf(v[2 * p] * inv)));
                    float v1 = std_max(-8.0f, std_min(7.0f, roundf(v[2 * p + 1] * inv)));
                    uint32_t lo = (uint32_t)((uint8_t)((int)v0 + 8) & 0x0F), hi = (uint32_t)((uint8_t)((int)v1 + 8) & 0x0F);
                    d |= (uint16_t)((lo | (hi << 4)) << (8 * k));
                }
            }
            h[1 + j] = d;
        }
        uint16_t* o = (uint16_t*)out;  // 2-byte aligned: blocks are 18 B
#pragma unroll
        for (int j = 0; j < 9; j++) o[j] = h[j];
    }
}

// mode 0: quantize src; mode 1: generate then quantize; mode 2: generate f32
__global__ void quant_gen_kernel(int mode, const float* __restrict__ src, uint64_t count, uint32_t dtype,
                                 uint8_t* __restrict__ dst, uint64_t base, float c) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t nb = (count + QB - 1) / QB;
    if (b >= nb) return;
    const uint64_t off = b * QB;
    const int tb = (int)min((uint64_t)QB, count - off);
    float v[QB];
#pragma unroll
    for (int i = 0; i < QB; i++) {
        if (i < tb) v[i] = mode == 0 ? src[off + i] : gen_value(base, off + i, c);
        else v[i] = 0.f;
    }
    if (mode == 2) {
        float* o = (float*)dst + off;
        for (int i = 0; i < tb; i++) o[i] = v[i];
        return;
    }
    quantize_block(v, tb, dtype, dst + b * q_block_bytes(dtype, QB));
}

static int launch_quant_gen(int mode, const float* src, uint64_t count, uint32_t dtype, void* dst, uint64_t seed,
                            uint64_t stream_id, float stddev, hipStream_t s) {
    QH_REQUIRE(dst && count, QRAF_HIP_ERR_INVALID, "null destination or empty tensor");
    QH_REQUIRE(mode != 0 || src, QRAF_HIP_ERR_INVALID, "null source");
    QH_REQUIRE(mode == 2 || dtype == DT_Q8_0 || dtype == DT_Q4_0, QRAF_HIP_ERR_DTYPE, "unsupported dtype %u", dtype);
    QH_REQUIRE(dtype != DT_Q8_0 || ((uintptr_t)dst & 3) == 0, QRAF_HIP_ERR_INVALID, "Q8_0 output must be 4-byte aligned");
    QH_REQUIRE(((uintptr_t)dst & 1) == 0, QRAF_HIP_ERR_INVALID, "output must be 2-byte aligned");
    const uint64_t base = mix64_host(seed ^ mix64_host(stream_id + 0x9E3779B97F4A7C15ULL));
    const double sd = 2.0 * sqrt(8.0 * (65536.0 * 65536.0 - 1.0) / 12.0);
    const float c = (float)((double)stddev / sd);
    const uint64_t nb = (count + QB - 1) / QB;
    hipLaunchKernelGGL(quant_gen_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, mode, src, count, dtype,
                       (uint8_t*)dst, base, c);
    QH_CHECK_HIP(hipGetLastError());
    return QRAF_HIP_OK;
}

int launch_gen_weights(void* dst, uint32_t dtype, uint64_t count, uint64_t seed, uint64_t stream_id, float stddev,
                       hipStream_t s) {
    if (dtype == DT_F32) return launch_quant_gen(2, nullptr, count, dtype, dst, seed, stream_id, stddev, s);
    return launch_quant_gen(1, nullptr, count, dtype, dst, seed, stream_id, stddev, s);
}

int launch_quantize(const float* src, uint64_t count, uint32_t dtype, void* dst, hipStream_t s) {
    return launch_quant_gen(0, src, count, dtype, dst, 0, 0, 0.f, s);
}

}  // namespace qraf_hip

extern "C" {

int qraf_hip_gen_weights_dev(void* dst, uint32_t dtype, uint64_t count, uint64_t seed, uint64_t stream_id,
                             float stddev, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_gen_weights(dst, dtype, count, seed, stream_id, stddev, qraf_hip::as_stream(stream));
}

int qraf_hip_quantize_dev(const float* src, uint64_t count, uint32_t dtype, void* dst, void* stream) {
    qraf_hip::clear_error();
    return qraf_hip::launch_quantize(src, count, dtype, dst, qraf_hip::as_stream(stream));
}

uint64_t qraf_hip_name_hash(const char* name) {  // include/qraf/format.h:136-147
    uint64_t h = 14695981039346656037ULL;
    for (; name && *name; name++) {
        h ^= (uint64_t)(unsigned char)*name;
        h *= 1099511628211ULL;
    }
    return h;
}

}  // extern "C"
