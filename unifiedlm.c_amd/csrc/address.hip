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
// Layout: one wave per row, each lane 4 consecutive slots per step (16-byte
// fp32 and 8-byte 16-bit accesses, coalesced along the slot index), so the
// per-row sums are wave reductions with no block barrier. The pass over HBM is
// bound by bandwidth: fwd moves sizeof(pre) + 4 bytes per element, bwd
// 2*4 + 2*sizeof(pre); each row's second read is served by the cache.
#include "ulm_common.h"

#include <mutex>

namespace ulm {

constexpr int kFwdRowsPerWave = 1;   // 66.7 us at the 110M rows against 74.0 (2), 77.3 (4), 97.0 (8)
constexpr int kBwdRowsPerWave = 8;   // amortises the per-block dbias partial row
constexpr int kAddrWaves = 4;
constexpr int kAddrSplit = 32;       // first-level row ranges of the dbias column sum

// Loads and stores of W consecutive elements (W = 4: one 16-byte fp32 or
// 8-byte 16-bit access; W = 1: scalar, for A % 4 != 0).
template <typename T, int W> struct Vec;
template <int W> struct Vec<float, W> {
    static __device__ __forceinline__ void ld(const float *p, size_t i, float (&v)[W]) {
        if constexpr (W == 4) {
            const float4 x = *reinterpret_cast<const float4 *>(p + i);
            v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
        } else {
            v[0] = p[i];
        }
    }
    static __device__ __forceinline__ void st(float *p, size_t i, const float (&v)[W]) {
        if constexpr (W == 4) *reinterpret_cast<float4 *>(p + i) = make_float4(v[0], v[1], v[2], v[3]);
        else p[i] = v[0];
    }
};
template <int W> struct Vec<uint16_t, W> {
    static __device__ __forceinline__ void ld(const uint16_t *p, size_t i, float (&v)[W]) {
        if constexpr (W == 4) {
            const uint2 x = *reinterpret_cast<const uint2 *>(p + i);
            v[0] = __uint_as_float(x.x << 16), v[1] = __uint_as_float(x.x & 0xffff0000u);
            v[2] = __uint_as_float(x.y << 16), v[3] = __uint_as_float(x.y & 0xffff0000u);
        } else {
            v[0] = bf16_to_f32(p[i]);
        }
    }
    static __device__ __forceinline__ void st(uint16_t *p, size_t i, const float (&v)[W]) {
        if constexpr (W == 4) {
            const uint32_t a = f32_to_bf16_bits(v[0]) | (static_cast<uint32_t>(f32_to_bf16_bits(v[1])) << 16);
            const uint32_t b = f32_to_bf16_bits(v[2]) | (static_cast<uint32_t>(f32_to_bf16_bits(v[3])) << 16);
            *reinterpret_cast<uint2 *>(p + i) = make_uint2(a, b);
        } else {
            p[i] = f32_to_bf16_bits(v[0]);
        }
    }
};
template <int W> struct Vec<_Float16, W> {
    static __device__ __forceinline__ void ld(const _Float16 *p, size_t i, float (&v)[W]) {
#pragma unroll
        for (int k = 0; k < W; ++k) v[k] = static_cast<float>(p[i + k]);
    }
    static __device__ __forceinline__ void st(_Float16 *p, size_t i, const float (&v)[W]) {
#pragma unroll
        for (int k = 0; k < W; ++k) p[i + k] = static_cast<_Float16>(v[k]);
    }
};

__device__ __forceinline__ float eps_of(const float *log_eps) {
    return __expf(fminf(fmaxf(log_eps[0], -10.f), 10.f));
}

// z = relu(pre + bias) for W columns at a
template <typename T, int W>
__device__ __forceinline__ void relu_row(const T *pre, const float *bias, size_t base, int a, float (&p)[W]) {
    Vec<T, W>::ld(pre, base + a, p);
    float b[W];
    if (bias) Vec<float, W>::ld(bias, a, b);
#pragma unroll
    for (int k = 0; k < W; ++k) {
        const float x = p[k] + (bias ? b[k] : 0.f);
        p[k] = x > 0.f ? x : 0.f;
    }
}

// One wave per row: the row sum of z^2 by a wave reduction, then r written
// with the row's second read of pre served by the cache.
template <typename T, int W>
__global__ __launch_bounds__(kAddrWaves * 64) void addr_fwd_kernel(const T *__restrict__ pre,
                                                                   const float *__restrict__ bias,
                                                                   const float *__restrict__ log_eps,
                                                                   float *__restrict__ r, float *__restrict__ denom,
                                                                   int M, int A) {
    const float E = eps_of(log_eps);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int row0 = (blockIdx.x * kAddrWaves + wave) * kFwdRowsPerWave;
    for (int row = row0; row < row0 + kFwdRowsPerWave && row < M; ++row) {
        const size_t base = static_cast<size_t>(row) * A;
        float ss = 0.f;
#pragma unroll 4
        for (int a = W * lane; a < A; a += W * kWave) {
            float p[W];
            relu_row<T, W>(pre, bias, base, a, p);
#pragma unroll
            for (int k = 0; k < W; ++k) ss += p[k] * p[k];
        }
        const float dn = E + wave_sum(ss);
        if (r) {   // null: only the denominators (the block forms r where it reads it)
#pragma unroll 4
            for (int a = W * lane; a < A; a += W * kWave) {
                float p[W];
                relu_row<T, W>(pre, bias, base, a, p);
#pragma unroll
                for (int k = 0; k < W; ++k) p[k] = (p[k] * p[k]) / dn;
                Vec<float, W>::st(r, base + a, p);
            }
        }
        if (lane == 0) denom[row] = dn;
    }
}

// One wave per row: rho = sum_a dr r by a wave reduction, then dpre. Each wave
// keeps its dbias column partials in its own LDS row; the block writes their
// sum as one partial row, and the dlog_eps partial. Without HAS_R, r is formed
// from pre, bias and denom with the forward's operations. With NS > 0 (rows of
// at most NS W 64 slots) the row's relu(pre + b) and dr stay in registers
// between the two passes, so each is read from memory once; with NS = 0 the
// second pass reads them again.
template <typename T, int W, bool HAS_R, int NS = 0>
__global__ __launch_bounds__(kAddrWaves * 64) void addr_bwd_kernel(const T *__restrict__ pre,
                                                                   const float *__restrict__ bias,
                                                                   const float *__restrict__ log_eps,
                                                                   const float *__restrict__ r,
                                                                   const float *__restrict__ denom,
                                                                   const float *__restrict__ dr,
                                                                   T *__restrict__ dpre, float *__restrict__ dbias_part,
                                                                   float *__restrict__ dle_part, int M, int A) {
    extern __shared__ __align__(16) float sdb[];   // [kAddrWaves][A]
    __shared__ float dle_w[kAddrWaves];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    float *const mine = sdb + static_cast<size_t>(wave) * A;
    for (int a = lane; a < A; a += kWave) mine[a] = 0.f;
    const float E = eps_of(log_eps);
    float dle = 0.f;
    const int row0 = (blockIdx.x * kAddrWaves + wave) * kBwdRowsPerWave;
    for (int row = row0; row < row0 + kBwdRowsPerWave && row < M; ++row) {
        const size_t base = static_cast<size_t>(row) * A;
        const float dn = denom[row];
        const float inv = 1.f / dn;
        float rho = 0.f;
        if constexpr (NS > 0) {
            // every load of the row first, unconditional at a clamped slot (a
            // load in a branch is waited for before the branch ends), the
            // slots past A masked to zero after
            float ps[NS][W], xs[NS][W];
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const int a = W * lane + k * W * kWave, ac = a < A ? a : 0;
                relu_row<T, W>(pre, bias, base, ac, ps[k]);
                Vec<float, W>::ld(dr, base + ac, xs[k]);
            }
#pragma unroll
            for (int k = 0; k < NS; ++k)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const bool ok = W * lane + k * W * kWave < A;
                    ps[k][e] = ok ? ps[k][e] : 0.f;
                    xs[k][e] = ok ? xs[k][e] : 0.f;
                }
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                float y[W];
                const int a = W * lane + k * W * kWave;
                if constexpr (HAS_R) {
                    if (a < A) Vec<float, W>::ld(r, base + a, y);
                    else for (int e = 0; e < W; ++e) y[e] = 0.f;
                } else {
#pragma unroll
                    for (int e = 0; e < W; ++e) y[e] = (ps[k][e] * ps[k][e]) * inv;   // as the fast memory's statistics form it
                }
#pragma unroll
                for (int e = 0; e < W; ++e) rho += xs[k][e] * y[e];
            }
            rho = wave_sum(rho);
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const int a = W * lane + k * W * kWave;
                if (a < A) {
                    float acc[W];
                    Vec<float, W>::ld(mine, a, acc);
#pragma unroll
                    for (int e = 0; e < W; ++e) {
                        ps[k][e] = 2.f * ps[k][e] * (xs[k][e] - rho) * inv;
                        acc[e] += ps[k][e];
                    }
                    Vec<T, W>::st(dpre, base + a, ps[k]);
                    Vec<float, W>::st(mine, a, acc);
                }
            }
            dle -= rho * inv;
            continue;
        }
#pragma unroll 4
        for (int a = W * lane; a < A; a += W * kWave) {
            float x[W], y[W];
            Vec<float, W>::ld(dr, base + a, x);
            if constexpr (HAS_R) {
                Vec<float, W>::ld(r, base + a, y);
            } else {
                relu_row<T, W>(pre, bias, base, a, y);
#pragma unroll
                for (int k = 0; k < W; ++k) y[k] = (y[k] * y[k]) * inv;   // as the fast memory's statistics form it
            }
#pragma unroll
            for (int k = 0; k < W; ++k) rho += x[k] * y[k];
        }
        rho = wave_sum(rho);
#pragma unroll 4
        for (int a = W * lane; a < A; a += W * kWave) {
            float p[W], x[W], acc[W];
            relu_row<T, W>(pre, bias, base, a, p);
            Vec<float, W>::ld(dr, base + a, x);
            Vec<float, W>::ld(mine, a, acc);
#pragma unroll
            for (int k = 0; k < W; ++k) {
                p[k] = 2.f * p[k] * (x[k] - rho) * inv;
                acc[k] += p[k];
            }
            Vec<T, W>::st(dpre, base + a, p);
            Vec<float, W>::st(mine, a, acc);
        }
        dle -= rho * inv;
    }
    if (lane == 0) dle_w[wave] = dle;
    __syncthreads();
    for (int a = threadIdx.x; a < A; a += kAddrWaves * kWave) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kAddrWaves; ++w) sum += sdb[static_cast<size_t>(w) * A + a];
        dbias_part[static_cast<size_t>(blockIdx.x) * A + a] = sum;
    }
    if (threadIdx.x == 0) {
        const float le = log_eps[0];
        const float d = dle_w[0] + dle_w[1] + dle_w[2] + dle_w[3];
        dle_part[blockIdx.x] = (le >= -10.f && le <= 10.f) ? d * E : 0.f;   // torch clamp passes the gradient at the bounds
    }
}

// dlog_eps = sum of the per-block partials in a fixed order (lane-strided
// partial sums, then the fixed shuffle tree of one wave)
__global__ __launch_bounds__(64) void addr_dle_kernel(const float *__restrict__ dle_part, float *__restrict__ dle,
                                                      int nblk) {
    double s = 0.0;
    for (int k = threadIdx.x; k < nblk; k += kWave) s += dle_part[k];
    s = wave_sum(s);
    if (threadIdx.x == 0) dle[0] = static_cast<float>(s);
}

int addr_blocks(int M, int rows_per_wave) {
    return (M + kAddrWaves * rows_per_wave - 1) / (kAddrWaves * rows_per_wave);
}

template <typename T>
int launch_addr_fwd(const void *pre, const float *bias, const float *log_eps, float *r, float *denom, int M, int A,
                    hipStream_t s) {
    const int nblk = addr_blocks(M, kFwdRowsPerWave);
    const bool vec = A % 4 == 0 && reinterpret_cast<uintptr_t>(pre) % (4 * sizeof(T)) == 0 &&
                     reinterpret_cast<uintptr_t>(r) % 16 == 0 && reinterpret_cast<uintptr_t>(bias) % 16 == 0;
    if (vec)
        addr_fwd_kernel<T, 4><<<nblk, kAddrWaves * 64, 0, s>>>(static_cast<const T *>(pre), bias, log_eps, r, denom,
                                                               M, A);
    else
        addr_fwd_kernel<T, 1><<<nblk, kAddrWaves * 64, 0, s>>>(static_cast<const T *>(pre), bias, log_eps, r, denom,
                                                               M, A);
    return check_launch("addr_fwd_kernel");
}

template <typename T, int W, bool HAS_R, int NS>
int launch_addr_bwd_ns(const T *pre, const float *bias, const float *log_eps, const float *r, const float *denom,
                       const float *dr, T *dpre, float *dbias_part, float *dle_part, int M, int A, int nblk,
                       size_t lds, hipStream_t s) {
    if (lds > 65536 &&
        hipFuncSetAttribute(reinterpret_cast<const void *>(&addr_bwd_kernel<T, W, HAS_R, NS>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
        return check_launch("addr_bwd_kernel attribute");
    addr_bwd_kernel<T, W, HAS_R, NS><<<nblk, kAddrWaves * 64, lds, s>>>(pre, bias, log_eps, r, denom, dr, dpre,
                                                                        dbias_part, dle_part, M, A);
    return check_launch("addr_bwd_kernel");
}

// rows of up to 16 x 256 slots (W = 4) are kept in registers between the passes
template <typename T, int W, bool HAS_R>
int launch_addr_bwd_kernel(const T *pre, const float *bias, const float *log_eps, const float *r, const float *denom,
                           const float *dr, T *dpre, float *dbias_part, float *dle_part, int M, int A, int nblk,
                           size_t lds, hipStream_t s) {
    if constexpr (W == 4) {
        const int steps = (A + W * kWave - 1) / (W * kWave);
        if (steps <= 4)
            return launch_addr_bwd_ns<T, W, HAS_R, 4>(pre, bias, log_eps, r, denom, dr, dpre, dbias_part, dle_part, M, A,
                                                      nblk, lds, s);
        if (steps <= 8)
            return launch_addr_bwd_ns<T, W, HAS_R, 8>(pre, bias, log_eps, r, denom, dr, dpre, dbias_part, dle_part, M, A,
                                                      nblk, lds, s);
        if (steps <= 12)
            return launch_addr_bwd_ns<T, W, HAS_R, 12>(pre, bias, log_eps, r, denom, dr, dpre, dbias_part, dle_part, M,
                                                       A, nblk, lds, s);
        if (steps <= 16)
            return launch_addr_bwd_ns<T, W, HAS_R, 16>(pre, bias, log_eps, r, denom, dr, dpre, dbias_part, dle_part, M,
                                                       A, nblk, lds, s);
    }
    return launch_addr_bwd_ns<T, W, HAS_R, 0>(pre, bias, log_eps, r, denom, dr, dpre, dbias_part, dle_part, M, A, nblk,
                                              lds, s);
}

template <typename T>
int launch_addr_bwd(const void *pre, const float *bias, const float *log_eps, const float *r, const float *denom,
                    const float *dr, void *dpre, float *dbias_part, float *dle_part, int M, int A, hipStream_t s) {
    const int nblk = addr_blocks(M, kBwdRowsPerWave);
    const size_t lds = static_cast<size_t>(kAddrWaves) * A * sizeof(float);
    const bool vec = A % 4 == 0 && reinterpret_cast<uintptr_t>(pre) % (4 * sizeof(T)) == 0 &&
                     reinterpret_cast<uintptr_t>(dpre) % (4 * sizeof(T)) == 0 &&
                     reinterpret_cast<uintptr_t>(r) % 16 == 0 && reinterpret_cast<uintptr_t>(dr) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(bias) % 16 == 0;
    const T *pt = static_cast<const T *>(pre);
    T *dp = static_cast<T *>(dpre);
    if (vec && r) return launch_addr_bwd_kernel<T, 4, true>(pt, bias, log_eps, r, denom, dr, dp, dbias_part, dle_part, M, A, nblk, lds, s);
    if (vec) return launch_addr_bwd_kernel<T, 4, false>(pt, bias, log_eps, r, denom, dr, dp, dbias_part, dle_part, M, A, nblk, lds, s);
    if (r) return launch_addr_bwd_kernel<T, 1, true>(pt, bias, log_eps, r, denom, dr, dp, dbias_part, dle_part, M, A, nblk, lds, s);
    return launch_addr_bwd_kernel<T, 1, false>(pt, bias, log_eps, r, denom, dr, dp, dbias_part, dle_part, M, A, nblk, lds, s);
}

}  // namespace ulm

using namespace ulm;

extern "C" int ulm_addr_fwd(const void *pre, int pre_dtype, const float *bias, const float *log_eps, float *r,
                            float *denom, int M, int A, void *stream) {
    ULM_REQUIRE(M > 0 && A > 0, "ulm_addr_fwd: bad sizes M=%d A=%d", M, A);
    ULM_REQUIRE(valid_dtype(pre_dtype), "ulm_addr_fwd: bad pre dtype %d", pre_dtype);
    ULM_REQUIRE(pre && log_eps && denom, "ulm_addr_fwd: null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (pre_dtype == ULM_F32) return launch_addr_fwd<float>(pre, bias, log_eps, r, denom, M, A, s);
    if (pre_dtype == ULM_BF16) return launch_addr_fwd<uint16_t>(pre, bias, log_eps, r, denom, M, A, s);
    return launch_addr_fwd<_Float16>(pre, bias, log_eps, r, denom, M, A, s);
}

namespace {

struct AddrWs {
    float *dbias_part, *dle_part, *tmp;
    size_t bytes;
};

AddrWs addr_ws(void *base, int M, int A) {
    const size_t nblk = addr_blocks(M, kBwdRowsPerWave);
    Carver c(base);
    AddrWs w{};
    w.dbias_part = c.take<float>(nblk * A);
    w.dle_part = c.take<float>(nblk);
    w.tmp = c.take<float>(static_cast<size_t>(kAddrSplit) * A);
    w.bytes = c.off;
    return w;
}

}  // namespace

extern "C" size_t ulm_addr_bwd_workspace_bytes(int M, int A) {
    if (M <= 0 || A <= 0) return 0;
    return addr_ws(nullptr, M, A).bytes;
}

namespace {

// The backward's launches on a scratch buffer of ulm_addr_bwd_workspace_bytes
// (arguments checked by the caller). Every scratch word the kernels read was
// written earlier in the same call: nothing needs to start at zero.
int addr_bwd_run(const void *pre, int pre_dtype, const float *bias, const float *log_eps, const float *r,
                 const float *denom, const float *dr, void *dpre, float *dbias, float *dlog_eps, void *scratch_buf,
                 int M, int A, hipStream_t s) {
    const AddrWs ws = addr_ws(scratch_buf, M, A);
    const int nblk = addr_blocks(M, kBwdRowsPerWave);
    int st;
    if (pre_dtype == ULM_F32)
        st = launch_addr_bwd<float>(pre, bias, log_eps, r, denom, dr, dpre, ws.dbias_part, ws.dle_part, M, A, s);
    else if (pre_dtype == ULM_BF16)
        st = launch_addr_bwd<uint16_t>(pre, bias, log_eps, r, denom, dr, dpre, ws.dbias_part, ws.dle_part, M, A, s);
    else
        st = launch_addr_bwd<_Float16>(pre, bias, log_eps, r, denom, dr, dpre, ws.dbias_part, ws.dle_part, M, A, s);
    if (st) return st;
    if (bias) ULM_TRY(launch_column_sum(ws.dbias_part, nblk, A, ws.tmp, kAddrSplit, dbias, s));
    addr_dle_kernel<<<1, 64, 0, s>>>(ws.dle_part, dlog_eps, nblk);
    return check_launch("addr_dle_kernel");
}

}  // namespace

#define ULM_ADDR_BWD_CHECKS(NAME)                                                                                 \
    ULM_REQUIRE(M > 0 && A > 0, NAME ": bad sizes M=%d A=%d", M, A);                                              \
    ULM_REQUIRE(A <= 8192, NAME ": A=%d exceeds the LDS column-partial limit 8192", A);                          \
    ULM_REQUIRE(valid_dtype(pre_dtype), NAME ": bad pre dtype %d", pre_dtype);                                    \
    ULM_REQUIRE(pre && log_eps && denom && dr && dpre && dlog_eps, NAME ": null pointer");                        \
    ULM_REQUIRE(!bias || dbias, NAME ": dbias is required when bias is given")

extern "C" int ulm_addr_bwd(const void *pre, int pre_dtype, const float *bias, const float *log_eps, const float *r,
                            const float *denom, const float *dr, void *dpre, float *dbias, float *dlog_eps,
                            void *workspace, size_t workspace_bytes, int M, int A, void *stream) {
    ULM_ADDR_BWD_CHECKS("ulm_addr_bwd");
    ULM_REQUIRE(workspace && workspace_bytes >= ulm_addr_bwd_workspace_bytes(M, A),
                "ulm_addr_bwd: workspace of %zu bytes, need %zu", workspace_bytes, ulm_addr_bwd_workspace_bytes(M, A));
    return addr_bwd_run(pre, pre_dtype, bias, log_eps, r, denom, dr, dpre, dbias, dlog_eps, workspace, M, A,
                        static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// ulm_addr_bwd without a workspace argument and without any allocation: the
// scratch lives in a fixed device array, one copy per GPU, held until the
// process ends. Its device address is looked up once per device (with that
// device current) and kept; the array's name is never used as an address on
// the host.

namespace {

static __device__ __align__(256) unsigned char scratch[ULM_ADDR_BWD_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void *g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// scratch's device address on the current device, looked up on first use
int scratch_ptr(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return check_launch("hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(ULM_ERR_UNSUPPORTED, "device %d past the %d supported", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
            return check_launch("hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return ULM_OK;
}

}  // namespace

extern "C" int ulm_addr_bwd_noalloc(const void *pre, int pre_dtype, const float *bias, const float *log_eps,
                                    const float *r, const float *denom, const float *dr, void *dpre, float *dbias,
                                    float *dlog_eps, int M, int A, void *stream) {
    ULM_ADDR_BWD_CHECKS("ulm_addr_bwd_noalloc");
    const size_t need = ulm_addr_bwd_workspace_bytes(M, A);
    ULM_REQUIRE(need <= ULM_ADDR_BWD_NOALLOC_SCRATCH_BYTES,
                "ulm_addr_bwd_noalloc: M=%d A=%d needs %zu bytes of scratch, past the %zu of the static array", M, A,
                need, static_cast<size_t>(ULM_ADDR_BWD_NOALLOC_SCRATCH_BYTES));
    void *buf = nullptr;
    ULM_TRY(scratch_ptr(&buf));
    return addr_bwd_run(pre, pre_dtype, bias, log_eps, r, denom, dr, dpre, dbias, dlog_eps, buf, M, A,
                        static_cast<hipStream_t>(stream));
}
