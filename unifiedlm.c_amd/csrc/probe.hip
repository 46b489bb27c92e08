// Layout probes, built into a test-only library (libulm_probe.so, declared in
// ulm_probe.h), that pin the lane layouts the kernels rely on:
//   * v_mfma_f32_32x32x16_bf16: the operand and accumulator lanes;
//   * ds_read_b64_tr_b16: each lane of a 16-lane group reads 8 bytes; the
//     group's 16 x 4 values are returned transposed;
//   * buffer_load_dwordx4 ... lds: each lane's 16 bytes land in LDS at
//     base + 16 * lane, and out-of-range offsets deliver zeros.
// No counterpart in the reference.
#include "ulm_common.h"

namespace ulm {

// one wave, D (32x32) = A (32x16) B (16x32): lane l holds row l % 32 of A and
// column l % 32 of B, contraction elements 8 (l / 32) .. 8 (l / 32) + 7;
// accumulator register r holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32
__global__ void probe_mfma_kernel(const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, float *__restrict__ d) {
    const int lane = threadIdx.x, lr = lane % 32, lh = lane / 32;
    bf16x8 x, y;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        x[e] = __builtin_bit_cast(bf16, a[lr * 16 + 8 * lh + e]);
        y[e] = __builtin_bit_cast(bf16, b[(8 * lh + e) * 32 + lr]);
    }
    f32x16 acc = {};
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) d[(8 * (r / 4) + 4 * lh + (r % 4)) * 32 + lr] = acc[r];
}

__global__ void probe_tr_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst) {
    __shared__ __align__(16) uint16_t lds[64 * 4];
    const int lane = threadIdx.x;
    for (int i = lane; i < 64 * 4; i += 64) lds[i] = src[i];
    __syncthreads();
    // lane L supplies the address of elements 4L .. 4L+3
    typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
    typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
    bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(lds + 4 * lane));
    // bit-cast the whole vector: extracting single __bf16 lanes and casting
    // each to uint16_t is folded to lane 0 by this compiler
    *reinterpret_cast<u16x4 *>(dst + 4 * lane) = __builtin_bit_cast(u16x4, v);
}

__global__ void probe_dma_kernel(const float *__restrict__ src, int n, const int *__restrict__ offsets,
                                 float *__restrict__ dst) {
    __shared__ __align__(16) float lds[64 * 4];
    const int lane = threadIdx.x;
    for (int i = lane; i < 64 * 4; i += 64) lds[i] = -1.f;
    __syncthreads();
    __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(src), 0, n * 4, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(lds), 16, offsets[lane],
                                             0, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int i = lane; i < 64 * 4; i += 64) dst[i] = lds[i];
}

}  // namespace ulm

using namespace ulm;

extern "C" int ulm_probe_mfma(const uint16_t *a, const uint16_t *b, float *d, void *stream) {
    ULM_REQUIRE(a && b && d, "ulm_probe_mfma: null pointer");
    probe_mfma_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(a, b, d);
    return check_launch("probe_mfma_kernel");
}

extern "C" int ulm_probe_lds_tr(const uint16_t *src, uint16_t *dst, void *stream) {
    ULM_REQUIRE(src && dst, "ulm_probe_lds_tr: null pointer");
    probe_tr_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(src, dst);
    return check_launch("probe_tr_kernel");
}

extern "C" int ulm_probe_lds_dma(const float *src, int n, const int *offsets, float *dst, void *stream) {
    ULM_REQUIRE(src && offsets && dst && n > 0, "ulm_probe_lds_dma: bad arguments");
    probe_dma_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(src, n, offsets, dst);
    return check_launch("probe_dma_kernel");
}
