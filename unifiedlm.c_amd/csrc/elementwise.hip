// Zero fill and dtype conversion used between the chunked kernels. A fill
// kernel rather than hipMemsetAsync keeps the calls safe to capture in a
// HIP graph.
#include "ulm_common.h"

namespace ulm {

__global__ void fill_zero_kernel(uint4 *p, size_t n16, uint8_t *tail, size_t ntail) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t k = i; k < n16; k += stride) p[k] = make_uint4(0, 0, 0, 0);
    if (i < ntail) tail[i] = 0;
}

int launch_fill_zero(void *p, size_t bytes, hipStream_t s) {
    if (bytes == 0) return ULM_OK;
    size_t n16 = bytes / 16;
    size_t ntail = bytes - n16 * 16;
    size_t blocks = (n16 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    fill_zero_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
        static_cast<uint4 *>(p), n16, static_cast<uint8_t *>(p) + n16 * 16, ntail);
    return check_launch("fill_zero_kernel");
}

__global__ void convert_kernel(const void *src, int sdt, void *dst, int ddt, size_t n) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t k = i; k < n; k += stride) store_from_f32(dst, k, ddt, load_as_f32(src, k, sdt));
}

// fp32 -> bf16, four elements per thread and step (16-byte loads, 8-byte stores)
__global__ void convert_f32_bf16x4_kernel(const float4 *__restrict__ src, uint2 *__restrict__ dst, size_t n4) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t k = i; k < n4; k += stride) {
        const float4 v = src[k];
        dst[k] = make_uint2(f32_to_bf16_bits(v.x) | (static_cast<uint32_t>(f32_to_bf16_bits(v.y)) << 16),
                            f32_to_bf16_bits(v.z) | (static_cast<uint32_t>(f32_to_bf16_bits(v.w)) << 16));
    }
}

int launch_convert(const void *src, int src_dt, void *dst, int dst_dt, size_t n, hipStream_t s) {
    if (n == 0) return ULM_OK;
    if (src_dt == ULM_F32 && dst_dt == ULM_BF16 && n % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(dst) % 8 == 0) {
        const size_t n4 = n / 4;
        size_t blocks = (n4 + 255) / 256;
        if (blocks > 16384) blocks = 16384;
        convert_f32_bf16x4_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
            static_cast<const float4 *>(src), static_cast<uint2 *>(dst), n4);
        return check_launch("convert_f32_bf16x4_kernel");
    }
    size_t blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    convert_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(src, src_dt, dst, dst_dt, n);
    return check_launch("convert_kernel");
}

// out[c] = sum_r in[r * ncol + c] over rows r of [r0, r1) for split blockIdx.y
// (rows split into gridDim.y contiguous ranges), written to out[blockIdx.y * ncol + c];
// with out2 given (one split only), columns c >= ncol1 go to out2[c - ncol1] instead.
__global__ __launch_bounds__(256) void column_sum_kernel(const float *__restrict__ in, size_t nrow, size_t ncol,
                                                              float *__restrict__ out, size_t ncol1,
                                                              float *__restrict__ out2) {
    const size_t c = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= ncol) return;
    const size_t per = (nrow + gridDim.y - 1) / gridDim.y;
    const size_t r0 = blockIdx.y * per, r1 = min(nrow, r0 + per);
    // rows added one after another in row order; their loads issued eight at a
    // time, so that the sum does not wait for one load at a time
    float s = 0.f;
    size_t r = r0;
    for (; r + 8 <= r1; r += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = in[(r + k) * ncol + c];
#pragma unroll
        for (int k = 0; k < 8; ++k) s += v[k];
    }
    for (; r < r1; ++r) s += in[r * ncol + c];
    if (out2 && c >= ncol1) out2[c - ncol1] = s;
    else out[blockIdx.y * ncol + c] = s;
}

int launch_column_sum(const float *in, size_t nrow, size_t ncol, float *tmp, int nsplit, float *out, hipStream_t s) {
    const unsigned gx = static_cast<unsigned>((ncol + 256 - 1) / 256);
    column_sum_kernel<<<dim3(gx, nsplit), 256, 0, s>>>(in, nrow, ncol, tmp, ncol, nullptr);
    ULM_TRY(check_launch("column_sum_kernel"));
    column_sum_kernel<<<dim3(gx, 1), 256, 0, s>>>(tmp, nsplit, ncol, out, ncol, nullptr);
    return check_launch("column_sum_kernel");
}

// Column sums of rows [a (ncol1) | b (ncol2)] into out1 (ncol1) and out2 (ncol2),
// in the same fixed order as launch_column_sum; tmp holds nsplit x (ncol1 + ncol2).
int launch_column_sum2(const float *in, size_t nrow, size_t ncol1, size_t ncol2, float *tmp, int nsplit, float *out1,
                       float *out2, hipStream_t s) {
    const size_t ncol = ncol1 + ncol2;
    const unsigned gx = static_cast<unsigned>((ncol + 256 - 1) / 256);
    column_sum_kernel<<<dim3(gx, nsplit), 256, 0, s>>>(in, nrow, ncol, tmp, ncol, nullptr);
    ULM_TRY(check_launch("column_sum_kernel"));
    column_sum_kernel<<<dim3(gx, 1), 256, 0, s>>>(tmp, nsplit, ncol, out1, ncol1, out2);
    return check_launch("column_sum_kernel");
}

}  // namespace ulm
