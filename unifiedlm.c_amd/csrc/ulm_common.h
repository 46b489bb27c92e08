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

// Access at a wave-uniform row pointer plus a lane's 32-bit byte offset: the
// row lives in scalar registers and every access of a row segment shares one
// offset VGPR (a global access with a scalar base), instead of each access
// carrying a 64-bit per-lane address (which the compiler otherwise forms by
// hoisting each access's loop-invariant lane part into its own VGPR pair). Empty
// asm statements, which emit no instruction, pin the row to a scalar register
// pair and keep the 32-bit offset opaque at the access, so that instruction
// selection sees "scalar base + zero-extended 32-bit offset". The row must
// therefore be wave-uniform. Callers clamp the row on wave-uniform conditions
// and the offset per lane, and mask the value after.
using gchar = __attribute__((address_space(1))) char;

__device__ __forceinline__ gchar *row_addr(const void *row, uint32_t byte_off) {
    uint64_t v = reinterpret_cast<uint64_t>(row);
    asm("" : "+s"(v));
    asm("" : "+v"(byte_off));
    return reinterpret_cast<gchar *>(v) + byte_off;
}

template <typename T> __device__ __forceinline__ T ld_row(const T *row, uint32_t byte_off) {
    return *reinterpret_cast<const __attribute__((address_space(1))) T *>(row_addr(row, byte_off));
}

template <typename T> __device__ __forceinline__ void st_row(T *row, uint32_t byte_off, T v) {
    *reinterpret_cast<__attribute__((address_space(1))) T *>(row_addr(row, byte_off)) = v;
}

// ---- operand tile layouts of the chunked kernels
//
// A tile is one v_mfma_f32_32x32x16_bf16 operand: 32 rows x 16 contraction
// elements, 1 KB, where lane l = r + 32 h holds row r, elements 8h .. 8h+7, as
// the 16 bytes at 16 l. A wave loads a tile with one fully coalesced 1 KB read.
//
// R layout (rows = positions, contraction = features), of X (B, T, F), F % 16 == 0,
// positions padded with zeros to 64 NT:
//   tile (b, t / 32, f / 16), lane (t % 32) + 32 ((f % 16) / 8), element f % 8.
// Q layout (rows = features in blocks of 32, in the order perm32; contraction =
// the 64 positions of a chunk, in quarters of 16), F % 32 == 0:
//   tile (b, t / 64, f / 32, (t % 64) / 16), lane perm32(f % 32) + 32 ((t % 16) / 8),
//   element t % 8.
// perm32 exchanges bits 2 and 3 of a row index (an involution). Stored in that
// order, the rows of an MFMA accumulator tile read 8 registers at a time form
// the next product's B operand with contraction index 8 h + e <-> row 16 j + 8 h + e.
__host__ __device__ __forceinline__ int perm32(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

constexpr int kTileElems = 512;   // bf16 per tile

// element offset of X[b][t][f] in the R layout (NT chunks, F features)
__host__ __device__ __forceinline__ size_t r_index(int b, int t, int f, int NT, int F) {
    const size_t tile = (static_cast<size_t>(b) * (2 * NT) + t / 32) * (F / 16) + f / 16;
    return tile * kTileElems + ((t % 32) + 32 * ((f % 16) / 8)) * 8 + f % 8;
}
// element offset of X[b][t][f] in the Q layout
__host__ __device__ __forceinline__ size_t q_index(int b, int t, int f, int NT, int F) {
    const size_t tile = ((static_cast<size_t>(b) * NT + t / 64) * (F / 32) + f / 32) * 4 + (t % 64) / 16;
    return tile * kTileElems + (perm32(f % 32) + 32 * ((t % 16) / 8)) * 8 + t % 8;
}
// element offset of P[b][n][i][j] (a 64 x 64 chunk matrix) in tile layout:
//   tile (b, n, i / 32, j / 16), lane (i % 32) + 32 ((j % 16) / 8), element j % 8
__host__ __device__ __forceinline__ size_t p_index(int b, int n, int i, int j, int NT) {
    const size_t tile = ((static_cast<size_t>(b) * NT + n) * 2 + i / 32) * 4 + j / 16;
    return tile * kTileElems + ((i % 32) + 32 * ((j % 16) / 8)) * 8 + j % 8;
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

// The scale s of H = s G in effect at the read-out of walk step k (after the
// renormalisation that step applies; 1 at k = 0 and whenever lam^64 < 2^-40).
__device__ inline float readout_scale(float lam64, int k) {
    if (lam64 < kRenorm) return 1.f;
    float s = 1.f;
    for (int i = 0; i < k; ++i) {
        if (i > 0 && s < kRenorm) s = 1.f;
        s = lam64 * s;
    }
    return (k > 0 && s < kRenorm) ? 1.f : s;
}

inline bool valid_dtype(int dt) { return dt == ULM_F32 || dt == ULM_BF16 || dt == ULM_F16; }

// Generic elementwise helpers (elementwise.hip).
int launch_fill_zero(void *p, size_t bytes, hipStream_t s);
int launch_convert(const void *src, int src_dt, void *dst, int dst_dt, size_t n, hipStream_t s);
// out[c] = sum over the nrow rows of in (nrow x ncol fp32) in a fixed order:
// nsplit contiguous row ranges into tmp (nsplit x ncol), then their sum.
int launch_column_sum(const float *in, size_t nrow, size_t ncol, float *tmp, int nsplit, float *out, hipStream_t s);
// the same over rows [a | b], into two outputs (elementwise.hip)
int launch_column_sum2(const float *in, size_t nrow, size_t ncol1, size_t ncol2, float *tmp, int nsplit, float *out1,
                       float *out2, hipStream_t s);

// Where the statistics kernels take the read address r (B,T,A) from: an fp32
// tensor r, or, when r is null, the block's address inputs, forming
// r = relu(pre + bias)^2 / denom[row] on the fly (model.py:70-72) so that the
// block never writes r.
struct RSrc {
    const float *r = nullptr;
    const void *pre = nullptr;
    int pre_dt = ULM_F32;
    const float *bias = nullptr;
    const float *denom = nullptr;
};

// Carves consecutive 256-byte aligned regions out of a buffer; with a null
// base it only measures.
struct Carver {
    char *base;
    size_t off = 0;
    explicit Carver(void *b) : base(static_cast<char *>(b)) {}
    template <class T>
    T *take(size_t count) {
        T *p = base ? reinterpret_cast<T *>(base + off) : nullptr;
        off += align_up(count * sizeof(T), 256);
        return p;
    }
};

// ---- the bf16 tile copies of a (B, T, X) tensor, X % 32 == 0
//
// One job: the 64 positions of chunk n x 256 features from xw, on 256 threads
// (tid), into the Q layout (raw) and the R layout (xr), either null; the
// layouts are X wide. Every load of the job is issued before its first store.
// The R layout is a re-tiling of the rows, written from registers; the Q
// layout goes through tile (4 x 64 x 36 words of LDS), where thread (feature
// pair fp, position group g) reads positions 8 g .. 8 g + 7 of features 2 fp,
// 2 fp + 1 as 8 words and writes two 16-byte Q chunks. The row stride of 36
// words puts the two position groups of a wave on disjoint banks.
// With raw, the job takes one workgroup barrier (raw is uniform over the
// workgroup); a job with live false takes it too and touches no memory, so
// several jobs can share a workgroup.
constexpr int kCopyBlocks = 4, kCopyStride = 36;
constexpr uint32_t kCopyLds = kCopyBlocks * ULM_CHUNK * kCopyStride * 4;   // bytes of tile per job
using copy_tile_t = uint32_t[ULM_CHUNK][kCopyStride];

__device__ __forceinline__ void tile_copy_bf16(const uint16_t *__restrict__ src, uint16_t *__restrict__ raw,
                                               uint16_t *__restrict__ xr, int T, int X, int NT, int xw, int n,
                                               int b, int tid, bool live, copy_tile_t *tile) {
    constexpr int C = ULM_CHUNK, NB = kCopyBlocks;
    const int i = tid / 4, c = tid % 4, t = n * C + i;
    uint4 v[NB][2];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        const int x0 = xw + k * C;
        // 16 features per thread: with X % 32 == 0 the block's second half may lie past X
        const bool ok = live && t < T && x0 + 16 * c < X;
        const uint4 *p = reinterpret_cast<const uint4 *>(src + (static_cast<size_t>(b) * T + (ok ? t : 0)) * X +
                                                         (ok ? x0 : 0) + 16 * c);
#pragma unroll
        for (int h = 0; h < 2; ++h) v[k][h] = ok ? p[h] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        const int x0 = xw + k * C;
        if (!live || x0 >= X) break;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (xr && x0 + 16 * c < X) *reinterpret_cast<uint4 *>(xr + r_index(b, t, x0 + 16 * c + 8 * h, NT, X)) = v[k][h];
            if (raw) *reinterpret_cast<uint4 *>(&tile[k][i][8 * c + 4 * h]) = v[k][h];
        }
    }
    if (!raw) return;
    __syncthreads();
    if (!live) return;
    const int fp = tid % 32, g = tid / 32;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        const int x0 = xw + k * C;
        if (x0 >= X) break;
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = tile[k][8 * g + j][fp];
        uint32_t e0[4], e1[4];   // features 2 fp and 2 fp + 1, positions in pairs
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            e0[e] = (w[2 * e] & 0xffffu) | (w[2 * e + 1] << 16);
            e1[e] = (w[2 * e] >> 16) | (w[2 * e + 1] & 0xffff0000u);
        }
        const int t0 = n * C + 8 * g;
        if (x0 + 2 * fp >= X) continue;   // the block's second half past X (X % 64 == 32)
        *reinterpret_cast<uint4 *>(raw + q_index(b, t0, x0 + 2 * fp, NT, X)) = make_uint4(e0[0], e0[1], e0[2], e0[3]);
        *reinterpret_cast<uint4 *>(raw + q_index(b, t0, x0 + 2 * fp + 1, NT, X)) =
            make_uint4(e1[0], e1[1], e1[2], e1[3]);
    }
}

}  // namespace ulm

// return a nonzero status from the enclosing function
#define ULM_TRY(x)              \
    do {                        \
        int _st = (x);          \
        if (_st) return _st;    \
    } while (0)
