// Shared definitions of the MI355X (gfx950) fast-memory library.
//
// Conventions of every extern "C" entry point in this library:
//   * pointers are device pointers, sizes are element counts;
//   * all work is enqueued on the given hipStream_t, nothing is allocated
//     (temporaries come from a caller-sized workspace);
//   * arguments are validated before any HIP call, so a bad call returns
//     ULM_ERR_INVALID without touching the GPU; the message is kept per
//     thread and read with ulm_last_error();
//   * a launch failure returns ULM_ERR_LAUNCH with the HIP error string.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/ulm_fm.h"

namespace ulm {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---- error reporting (defined in status.cpp)
int fail(int code, const char *fmt, ...);
int check_launch(const char *what);

#define ULM_REQUIRE(cond, ...)                                   \
    do {                                                         \
        if (!(cond)) return ::ulm::fail(ULM_ERR_INVALID, __VA_ARGS__); \
    } while (0)

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---- device helpers

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    bf16 b = static_cast<bf16>(f);   // round to nearest even (v_cvt_pk_bf16_f32)
    return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Loads an element of a float/bf16/fp16 tensor as fp32.
__device__ __forceinline__ float load_as_f32(const void *p, size_t i, int dtype) {
    if (dtype == ULM_F32) return static_cast<const float *>(p)[i];
    if (dtype == ULM_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    return static_cast<float>(static_cast<const _Float16 *>(p)[i]);
}

__device__ __forceinline__ void store_from_f32(void *p, size_t i, int dtype, float v) {
    if (dtype == ULM_F32) static_cast<float *>(p)[i] = v;
    else if (dtype == ULM_BF16) static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
    else static_cast<_Float16 *>(p)[i] = static_cast<_Float16>(v);
}

// ---- scale schedule of the chunked state H = s G. The K-group kernel and the
// producer of its pre-decayed update operand both follow it with the same
// float operations, so the divisor folded into the operand is the one the
// kernel assumes. Walk step k: read-out (k >= 1) renormalises s to 1 when it
// fell below kRenorm; the update then sets s_{k+1} = lam^64 s (or keeps s = 1
// when lam^64 itself is below kRenorm and G is decayed explicitly instead).
constexpr float kRenorm = 0x1p-40f;

__device__ __forceinline__ float state_lam64(float g) { return __expf(g * 64.f); }

// 1 / s_{k+1}, the divisor folded into the update operand of walk step k
__device__ inline float state_inv_scale(float lam64, int k) {
    const bool tiny = lam64 < kRenorm;
    float s = 1.f;
    for (int i = 0; i <= k; ++i) {
        if (i > 0 && !tiny && s < kRenorm) s = 1.f;
        s = tiny ? 1.f : lam64 * s;
    }
    return 1.f / s;
}

inline bool valid_dtype(int dt) { return dt == ULM_F32 || dt == ULM_BF16 || dt == ULM_F16; }

// Generic elementwise helpers (elementwise.hip).
int launch_fill_zero(void *p, size_t bytes, hipStream_t s);
int launch_convert(const void *src, int src_dt, void *dst, int dst_dt, size_t n, hipStream_t s);

}  // namespace ulm
