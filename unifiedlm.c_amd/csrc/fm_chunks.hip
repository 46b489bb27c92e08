// Per-chunk layouts consumed by the K-group chunked kernel (la_kgroup.hip).
//
//  * chunk_transpose: dst[b][n][x][i] = src[b][64n + i][x] as bf16, zero for
//    64n + i >= T: the feature-major copy of each 64-position chunk, so the
//    operands that contract over time load as 16 contiguous bytes (8
//    positions of one feature); optionally also the pre-decayed copy that
//    the chunked kernel's state update consumes.
//  * chunk_scores: per chunk n, with S[i][j] = a_{64n+i} . b_{64n+j},
//      P_lo[i][j] = S[i][j] lam^(i-j)  (j <= i, else 0)   forward walk
//      P_up[i][j] = S[j][i] lam^(j-i)  (j >= i, else 0)   = P_lo^T
//    as bf16. P_lo is the intra-chunk matrix of o = LA(a, b, .) and P_up that
//    of the reversed product with a and b exchanged (LA_rev(b, a, .)), so one
//    pass serves fwd + dv (a = q, b = k) and dq + dk (a = dfast, b = v). This
//    is the _la_attn_kernel product (kernel.py:51-72), computed once per chunk
//    and shared by every value tile.
//  * partial_reduce: out = sum over nK fp32 partial outputs, in out's dtype.
#include "ulm_common.h"

namespace ulm {

namespace chunks {

constexpr int C = ULM_CHUNK;

// grid (ceil(X/64), NT, B), 256 threads: one 64-position x 64-feature tile.
// DEC = 0: raw copy only. DEC = 1 / 2: also the pre-decayed update operand of
// the forward / reversed walk, bf16 hi (+ lo = the rounding remainder):
//   forward  lam^(63-i) x / s_{n+1}          at walk step n
//   reversed lam^i      x / s_{NT-n}         at walk step NT-1-n
// with s the state scale schedule of the chunked kernel (state_inv_scale).
template <int DEC>
__global__ __launch_bounds__(256) void transpose_kernel(const void *__restrict__ src, int sdt, uint16_t *__restrict__ raw,
                                                        uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                        const float *__restrict__ g, int T, int X, int NT) {
    __shared__ uint16_t tile[C][C + 2];
    const int x0 = blockIdx.x * C, n = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    {
        const int i = tid / 4, c0 = (tid % 4) * 16;   // position row i, 16 features
        const int t = n * C + i;
        const bool ok = t < T;
        const size_t row = (static_cast<size_t>(b) * T + (ok ? t : 0)) * X;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int x = x0 + c0 + e;
            tile[i][c0 + e] = (ok && x < X) ? f32_to_bf16_bits(load_as_f32(src, row + x, sdt)) : 0;
        }
    }
    __syncthreads();
    const int xl = tid / 4, i0 = (tid % 4) * 16;   // feature row xl, 16 positions
    const int x = x0 + xl;
    if (x >= X) return;
    const size_t o = ((static_cast<size_t>(b) * NT + n) * X + x) * C + i0;
    if (raw) {
        uint32_t w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            w[e] = static_cast<uint32_t>(tile[i0 + 2 * e][xl]) | (static_cast<uint32_t>(tile[i0 + 2 * e + 1][xl]) << 16);
        uint4 *d = reinterpret_cast<uint4 *>(raw + o);
        d[0] = make_uint4(w[0], w[1], w[2], w[3]);
        d[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
    if (DEC) {
        const float gl = g[0];
        const int step = DEC == 1 ? n : NT - 1 - n;
        const float inv_s = state_inv_scale(state_lam64(gl), step);
        uint32_t wh[8], wl[8];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int i = i0 + e;
            const float f = __expf(gl * static_cast<float>(DEC == 1 ? C - 1 - i : i)) * inv_s;
            const float v = bf16_to_f32(tile[i][xl]) * f;
            const uint16_t h = f32_to_bf16_bits(v);
            const uint16_t l = f32_to_bf16_bits(v - bf16_to_f32(h));
            if (e % 2 == 0) {
                wh[e / 2] = h;
                wl[e / 2] = l;
            } else {
                wh[e / 2] |= static_cast<uint32_t>(h) << 16;
                wl[e / 2] |= static_cast<uint32_t>(l) << 16;
            }
        }
        uint4 *dh = reinterpret_cast<uint4 *>(hi + o);
        dh[0] = make_uint4(wh[0], wh[1], wh[2], wh[3]);
        dh[1] = make_uint4(wh[4], wh[5], wh[6], wh[7]);
        if (lo) {
            uint4 *dl = reinterpret_cast<uint4 *>(lo + o);
            dl[0] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
            dl[1] = make_uint4(wl[4], wl[5], wl[6], wl[7]);
        }
    }
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// grid (NT, B), 256 threads. Wave w owns score tile (mt, nt) = (w/2, w%2) of the
// 64 x 64 chunk, 32 x 32, contracted over all K (K % 8 == 0). Tile (0, 1) is
// strictly above the diagonal: that wave only writes the zero tiles.
__global__ __launch_bounds__(256) void scores_kernel(const uint16_t *__restrict__ A_, const uint16_t *__restrict__ B_,
                                                     const float *__restrict__ g, uint16_t *__restrict__ Plo,
                                                     uint16_t *__restrict__ Pup, int T, int K, int NT) {
    const int n = blockIdx.x, b = blockIdx.y;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int lr = lane % 32, lh = lane / 32;
    const int mt = wave >> 1, nt = wave & 1;
    const size_t tile_off = (static_cast<size_t>(b) * NT + n) * C * C;
    uint16_t *lo = Plo + tile_off, *up = Pup + tile_off;
    if (mt == 0 && nt == 1) {
        // P_lo rows 0..31 x cols 32..63 and P_up rows 32..63 x cols 0..31 are zero
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r / 4) + 4 * lh + (r % 4);
            lo[row * C + 32 + lr] = 0;
            up[(32 + row) * C + lr] = 0;
        }
        return;
    }
    const int ti = n * C + 32 * mt + lr, tj = n * C + 32 * nt + lr;
    const bool oki = ti < T, okj = tj < T;
    const uint16_t *pa = A_ + (static_cast<size_t>(b) * T + (oki ? ti : 0)) * K + 8 * lh;
    const uint16_t *pb = B_ + (static_cast<size_t>(b) * T + (okj ? tj : 0)) * K + 8 * lh;
    const int nks = K / 16;   // full 16-key steps; a trailing 8 keys (K % 16 == 8) taken by lh == 0
    f32x16 acc[4] = {};
    int ks = 0;
    for (; ks + 4 <= nks; ks += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bf16x8 x = oki ? *reinterpret_cast<const bf16x8 *>(pa + 16 * (ks + u)) : bf16x8{};
            const bf16x8 y = okj ? *reinterpret_cast<const bf16x8 *>(pb + 16 * (ks + u)) : bf16x8{};
            acc[u] = mfma(x, y, acc[u]);
        }
    }
    for (; ks < nks; ++ks) {
        const bf16x8 x = oki ? *reinterpret_cast<const bf16x8 *>(pa + 16 * ks) : bf16x8{};
        const bf16x8 y = okj ? *reinterpret_cast<const bf16x8 *>(pb + 16 * ks) : bf16x8{};
        acc[0] = mfma(x, y, acc[0]);
    }
    if (K % 16) {
        const bool tail = lh == 0;
        const bf16x8 x = (oki && tail) ? *reinterpret_cast<const bf16x8 *>(pa + 16 * nks) : bf16x8{};
        const bf16x8 y = (okj && tail) ? *reinterpret_cast<const bf16x8 *>(pb + 16 * nks) : bf16x8{};
        acc[1] = mfma(x, y, acc[1]);
    }
    const float gl = g[0];
    const int j = 32 * nt + lr;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint16_t vals[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int r = 4 * q + m;
            const int i = 32 * mt + 8 * q + 4 * lh + m;
            const float s = acc[0][r] + acc[1][r] + acc[2][r] + acc[3][r];
            const int lag = i - j;
            const float v = lag >= 0 ? s * __expf(gl * static_cast<float>(lag)) : 0.f;
            vals[m] = f32_to_bf16_bits(v);
            lo[i * C + j] = vals[m];
        }
        // P_up[j][i .. i+3] = P_lo[i .. i+3][j]
        const int i0 = 32 * mt + 8 * q + 4 * lh;
        uint2 pk;
        pk.x = static_cast<uint32_t>(vals[0]) | (static_cast<uint32_t>(vals[1]) << 16);
        pk.y = static_cast<uint32_t>(vals[2]) | (static_cast<uint32_t>(vals[3]) << 16);
        *reinterpret_cast<uint2 *>(up + j * C + i0) = pk;
    }
}

// out[i] = sum_k part[k * n + i], written in out's dtype
__global__ __launch_bounds__(256) void partial_reduce_kernel(const float *__restrict__ part, int nK, size_t n,
                                                             void *__restrict__ out, int odt, bool vec) {
    const size_t n4 = vec ? n / 4 : 0;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 s = reinterpret_cast<const float4 *>(part)[i];
        for (int k = 1; k < nK; ++k) {
            const float4 x = reinterpret_cast<const float4 *>(part + k * n)[i];
            s.x += x.x;
            s.y += x.y;
            s.z += x.z;
            s.w += x.w;
        }
        if (odt == ULM_F32) {
            reinterpret_cast<float4 *>(out)[i] = s;
        } else {
            store_from_f32(out, 4 * i + 0, odt, s.x);
            store_from_f32(out, 4 * i + 1, odt, s.y);
            store_from_f32(out, 4 * i + 2, odt, s.z);
            store_from_f32(out, 4 * i + 3, odt, s.w);
        }
    }
    // scalar tail (n % 4)
    for (size_t i = 4 * n4 + static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        float s = 0.f;
        for (int k = 0; k < nK; ++k) s += part[k * n + i];
        store_from_f32(out, i, odt, s);
    }
}

}  // namespace chunks

// raw, hi, lo: (B, NT, X, 64) bf16 or null. decay 0: raw only; 1 / 2: hi (+ lo)
// hold the pre-decayed update operand of the forward / reversed walk.
int launch_chunk_transpose(const void *src, int src_dt, uint16_t *raw, uint16_t *hi, uint16_t *lo, const float *g,
                           int decay, int B, int T, int X, hipStream_t s) {
    if (decay && !(hi && g)) return fail(ULM_ERR_INVALID, "chunk transpose: decayed output needs hi and g");
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    const dim3 grid((X + ULM_CHUNK - 1) / ULM_CHUNK, NT, B);
    if (decay == 1) chunks::transpose_kernel<1><<<grid, 256, 0, s>>>(src, src_dt, raw, hi, lo, g, T, X, NT);
    else if (decay == 2) chunks::transpose_kernel<2><<<grid, 256, 0, s>>>(src, src_dt, raw, hi, lo, g, T, X, NT);
    else chunks::transpose_kernel<0><<<grid, 256, 0, s>>>(src, src_dt, raw, nullptr, nullptr, g, T, X, NT);
    return check_launch("chunk transpose_kernel");
}

int launch_chunk_scores(const uint16_t *a, const uint16_t *b, const float *g, uint16_t *Plo, uint16_t *Pup, int B,
                        int T, int K, hipStream_t s) {
    if (K % 8) return fail(ULM_ERR_UNSUPPORTED, "chunk scores: K=%d is not a multiple of 8", K);
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    chunks::scores_kernel<<<dim3(NT, B), 256, 0, s>>>(a, b, g, Plo, Pup, T, K, NT);
    return check_launch("chunk scores_kernel");
}

int launch_partial_reduce(const float *part, int nK, size_t n, void *out, int odt, hipStream_t s) {
    if (n == 0) return ULM_OK;
    // float4 path when every partial row and the output are 16-byte aligned
    const bool vec = n % 4 == 0 && reinterpret_cast<uintptr_t>(part) % 16 == 0 &&
                     (odt != ULM_F32 || reinterpret_cast<uintptr_t>(out) % 16 == 0);
    size_t blocks = ((vec ? n / 4 : n) + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    chunks::partial_reduce_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(part, nK, n, out, odt, vec);
    return check_launch("partial_reduce_kernel");
}

}  // namespace ulm
