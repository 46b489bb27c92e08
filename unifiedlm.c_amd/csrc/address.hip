// relu^2 slot address, training form. Replaces UnifiedBlock.code after the
// key GEMM (model.py:70-72, with the fp32 promotion of model.py:26-28):
//
//   z = relu(pre + b)^2,  denom = exp(clamp(log_eps, -10, 10)) + sum_a z,  r = z / denom
//
// and its backward, with rho = sum_a dr_a r_a per row:
//
//   dpre_a = 2 relu(pre_a + b_a) (dr_a - rho) / denom
//   dbias  = sum over rows of dpre,   dlog_eps = -sum_rows rho / denom * exp(log_eps) [inside the clamp]
//
// Layout: one 256-thread block owns a group of rows, each thread a fixed set of
// columns (a = tid + 256 j), so loads are coalesced along the slot index and
// the per-row sums need one block reduction for kRowGroup rows at a time. The
// pass over HBM is bound by bandwidth: fwd moves sizeof(pre) + 4 bytes per
// element, bwd 2*4 + 2*sizeof(pre).
#include "ulm_common.h"

namespace ulm {

constexpr int kRowGroup = 8;     // rows reduced together
constexpr int kFwdRows = 8;      // rows per block, forward
constexpr int kBwdRows = 64;     // rows per block, backward (amortises the dbias partial)

template <typename T> __device__ __forceinline__ float ld(const T *p, size_t i);
template <> __device__ __forceinline__ float ld<float>(const float *p, size_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld<uint16_t>(const uint16_t *p, size_t i) { return bf16_to_f32(p[i]); }
template <> __device__ __forceinline__ float ld<_Float16>(const _Float16 *p, size_t i) { return static_cast<float>(p[i]); }

template <typename T> __device__ __forceinline__ void st(T *p, size_t i, float v);
template <> __device__ __forceinline__ void st<float>(float *p, size_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void st<uint16_t>(uint16_t *p, size_t i, float v) { p[i] = f32_to_bf16_bits(v); }
template <> __device__ __forceinline__ void st<_Float16>(_Float16 *p, size_t i, float v) { p[i] = static_cast<_Float16>(v); }

// Sums kRowGroup per-thread values over the 256-thread block.
__device__ __forceinline__ void block_sum_group(float (&v)[kRowGroup], float (*red)[kRowGroup]) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
#pragma unroll
    for (int i = 0; i < kRowGroup; ++i) v[i] = wave_sum(v[i]);
    __syncthreads();
    if (lane == 0)
        for (int i = 0; i < kRowGroup; ++i) red[wave][i] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRowGroup; ++i) v[i] = red[0][i] + red[1][i] + red[2][i] + red[3][i];
}

__device__ __forceinline__ float eps_of(const float *log_eps) {
    return __expf(fminf(fmaxf(log_eps[0], -10.f), 10.f));
}

template <typename T>
__global__ __launch_bounds__(256) void addr_fwd_kernel(const T *__restrict__ pre, const float *__restrict__ bias,
                                                       const float *__restrict__ log_eps, float *__restrict__ r,
                                                       float *__restrict__ denom, int M, int A) {
    __shared__ float red[4][kRowGroup];
    const float E = eps_of(log_eps);
    const int row0 = blockIdx.x * kFwdRows;
    for (int rg = row0; rg < row0 + kFwdRows && rg < M; rg += kRowGroup) {
        float s[kRowGroup];
#pragma unroll
        for (int i = 0; i < kRowGroup; ++i) {
            s[i] = 0.f;
            const int row = rg + i;
            if (row >= M) continue;
            const size_t base = static_cast<size_t>(row) * A;
            for (int a = threadIdx.x; a < A; a += 256) {
                float p = ld(pre, base + a) + (bias ? bias[a] : 0.f);
                p = p > 0.f ? p : 0.f;
                s[i] += p * p;
            }
        }
        block_sum_group(s, red);
#pragma unroll
        for (int i = 0; i < kRowGroup; ++i) {
            const int row = rg + i;
            if (row >= M) continue;
            const float dn = E + s[i];
            const size_t base = static_cast<size_t>(row) * A;
            for (int a = threadIdx.x; a < A; a += 256) {
                float p = ld(pre, base + a) + (bias ? bias[a] : 0.f);
                p = p > 0.f ? p : 0.f;
                r[base + a] = (p * p) / dn;
            }
            if (threadIdx.x == 0) denom[row] = dn;
        }
    }
}

// Writes dpre and, per block, the partial column sums of dpre (dbias) and the
// partial dlog_eps; addr_reduce_kernel sums the partials in a fixed order.
template <typename T>
__global__ __launch_bounds__(256) void addr_bwd_kernel(const T *__restrict__ pre, const float *__restrict__ bias,
                                                       const float *__restrict__ log_eps, const float *__restrict__ r,
                                                       const float *__restrict__ denom, const float *__restrict__ dr,
                                                       T *__restrict__ dpre, float *__restrict__ dbias_part,
                                                       float *__restrict__ dle_part, int M, int A) {
    extern __shared__ float sdb[];   // A column partials
    __shared__ float red[4][kRowGroup];
    for (int a = threadIdx.x; a < A; a += 256) sdb[a] = 0.f;
    const float E = eps_of(log_eps);
    float dle = 0.f;
    const int row0 = blockIdx.x * kBwdRows;
    for (int rg = row0; rg < row0 + kBwdRows && rg < M; rg += kRowGroup) {
        float rho[kRowGroup];
#pragma unroll
        for (int i = 0; i < kRowGroup; ++i) {
            rho[i] = 0.f;
            const int row = rg + i;
            if (row >= M) continue;
            const size_t base = static_cast<size_t>(row) * A;
            for (int a = threadIdx.x; a < A; a += 256) rho[i] += dr[base + a] * r[base + a];
        }
        block_sum_group(rho, red);
#pragma unroll
        for (int i = 0; i < kRowGroup; ++i) {
            const int row = rg + i;
            if (row >= M) continue;
            const float dn = denom[row];
            const size_t base = static_cast<size_t>(row) * A;
            for (int a = threadIdx.x; a < A; a += 256) {
                float p = ld(pre, base + a) + (bias ? bias[a] : 0.f);
                p = p > 0.f ? p : 0.f;
                const float g = 2.f * p * (dr[base + a] - rho[i]) / dn;
                st(dpre, base + a, g);
                sdb[a] += g;
            }
            dle += -rho[i] / dn;
        }
    }
    __syncthreads();
    for (int a = threadIdx.x; a < A; a += 256) dbias_part[static_cast<size_t>(blockIdx.x) * A + a] = sdb[a];
    if (threadIdx.x == 0) {
        const float le = log_eps[0];
        dle_part[blockIdx.x] = (le > -10.f && le < 10.f) ? dle * E : 0.f;
    }
}

__global__ __launch_bounds__(256) void addr_reduce_kernel(const float *__restrict__ dbias_part,
                                                          const float *__restrict__ dle_part, float *__restrict__ dbias,
                                                          float *__restrict__ dle, int nblk, int A) {
    const int a = blockIdx.x * 256 + threadIdx.x;
    if (dbias && a < A) {
        float s = 0.f;
        for (int k = 0; k < nblk; ++k) s += dbias_part[static_cast<size_t>(k) * A + a];
        dbias[a] = s;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        double s = 0.0;
        for (int k = 0; k < nblk; ++k) s += dle_part[k];
        dle[0] = static_cast<float>(s);
    }
}

}  // namespace ulm

using namespace ulm;

extern "C" int ulm_addr_fwd(const void *pre, int pre_dtype, const float *bias, const float *log_eps, float *r,
                            float *denom, int M, int A, void *stream) {
    ULM_REQUIRE(M > 0 && A > 0, "ulm_addr_fwd: bad sizes M=%d A=%d", M, A);
    ULM_REQUIRE(valid_dtype(pre_dtype), "ulm_addr_fwd: bad pre dtype %d", pre_dtype);
    ULM_REQUIRE(pre && log_eps && r && denom, "ulm_addr_fwd: null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((M + kFwdRows - 1) / kFwdRows);
    if (pre_dtype == ULM_F32)
        addr_fwd_kernel<float><<<grid, 256, 0, s>>>(static_cast<const float *>(pre), bias, log_eps, r, denom, M, A);
    else if (pre_dtype == ULM_BF16)
        addr_fwd_kernel<uint16_t><<<grid, 256, 0, s>>>(static_cast<const uint16_t *>(pre), bias, log_eps, r, denom, M, A);
    else
        addr_fwd_kernel<_Float16><<<grid, 256, 0, s>>>(static_cast<const _Float16 *>(pre), bias, log_eps, r, denom, M, A);
    return check_launch("addr_fwd_kernel");
}

extern "C" size_t ulm_addr_bwd_workspace_bytes(int M, int A) {
    if (M <= 0 || A <= 0) return 0;
    const size_t nblk = (M + kBwdRows - 1) / kBwdRows;
    return align_up(nblk * A * sizeof(float), 256) + align_up(nblk * sizeof(float), 256);
}

extern "C" int ulm_addr_bwd(const void *pre, int pre_dtype, const float *bias, const float *log_eps, const float *r,
                            const float *denom, const float *dr, void *dpre, float *dbias, float *dlog_eps,
                            void *workspace, size_t workspace_bytes, int M, int A, void *stream) {
    ULM_REQUIRE(M > 0 && A > 0, "ulm_addr_bwd: bad sizes M=%d A=%d", M, A);
    ULM_REQUIRE(A <= 16384, "ulm_addr_bwd: A=%d exceeds the LDS column-partial limit 16384", A);
    ULM_REQUIRE(valid_dtype(pre_dtype), "ulm_addr_bwd: bad pre dtype %d", pre_dtype);
    ULM_REQUIRE(pre && log_eps && r && denom && dr && dpre && dlog_eps, "ulm_addr_bwd: null pointer");
    ULM_REQUIRE(!bias || dbias, "ulm_addr_bwd: dbias is required when bias is given");
    ULM_REQUIRE(workspace && workspace_bytes >= ulm_addr_bwd_workspace_bytes(M, A),
                "ulm_addr_bwd: workspace of %zu bytes, need %zu", workspace_bytes, ulm_addr_bwd_workspace_bytes(M, A));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int nblk = (M + kBwdRows - 1) / kBwdRows;
    float *dbias_part = static_cast<float *>(workspace);
    float *dle_part = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                                align_up(static_cast<size_t>(nblk) * A * sizeof(float), 256));
    const size_t lds = static_cast<size_t>(A) * sizeof(float);
    if (lds > 65536) {
        const void *fn = pre_dtype == ULM_F32    ? reinterpret_cast<const void *>(&addr_bwd_kernel<float>)
                         : pre_dtype == ULM_BF16 ? reinterpret_cast<const void *>(&addr_bwd_kernel<uint16_t>)
                                                 : reinterpret_cast<const void *>(&addr_bwd_kernel<_Float16>);
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
            return check_launch("addr_bwd_kernel attribute");
    }
    if (pre_dtype == ULM_F32)
        addr_bwd_kernel<float><<<nblk, 256, lds, s>>>(static_cast<const float *>(pre), bias, log_eps, r, denom, dr,
                                                      static_cast<float *>(dpre), dbias_part, dle_part, M, A);
    else if (pre_dtype == ULM_BF16)
        addr_bwd_kernel<uint16_t><<<nblk, 256, lds, s>>>(static_cast<const uint16_t *>(pre), bias, log_eps, r, denom,
                                                         dr, static_cast<uint16_t *>(dpre), dbias_part, dle_part, M, A);
    else
        addr_bwd_kernel<_Float16><<<nblk, 256, lds, s>>>(static_cast<const _Float16 *>(pre), bias, log_eps, r, denom,
                                                         dr, static_cast<_Float16 *>(dpre), dbias_part, dle_part, M, A);
    int st = check_launch("addr_bwd_kernel");
    if (st) return st;
    addr_reduce_kernel<<<(A + 255) / 256, 256, 0, s>>>(dbias_part, dle_part, bias ? dbias : nullptr, dlog_eps, nblk, A);
    return check_launch("addr_reduce_kernel");
}
