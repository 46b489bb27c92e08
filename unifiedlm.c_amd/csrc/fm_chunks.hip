// Per-chunk layouts consumed by the K-group chunked kernel (la_kgroup.hip).
//
//  * chunk_transpose: the tiled copies of a (B, T, X) tensor that the chunked
//    kernel loads (R and Q layouts of ulm_common.h; positions past T are zero),
//    optionally with the pre-decayed copy its state update consumes.
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

// grid (ceil(X/64), NT, B), 256 threads: one 64-position x 64-feature block of
// X (B, T, X) in any float dtype, rounded to bf16 (X % 32 == 0). Outputs, each
// optional: raw (Q layout), the pre-decayed update operand hi (+ lo, the
// rounding remainder) in the Q layout, and xr (R layout). DEC = 1 / 2 decays
// for the forward / reversed walk:
//   forward  lam^(63-i) x / s_{n+1}          at walk step n
//   reversed lam^i      x / s_{NT-n}         at walk step NT-1-n
// with s the state scale schedule of the chunked kernel (state_inv_scale).
template <int DEC>
__global__ __launch_bounds__(256) void transpose_kernel(const void *__restrict__ src, int sdt, uint16_t *__restrict__ raw,
                                                        uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                        uint16_t *__restrict__ xr, const float *__restrict__ g, int T,
                                                        int X, int NT) {
    __shared__ __align__(16) uint16_t tile[C][C + 8];   // [position][feature]
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
    if (xr) {
        // R layout: 64 positions x 64 features are 8 tiles; thread -> 2 lanes of one tile
        const int tl = tid / 32, mt = tl / 4, tf4 = tl % 4;
        if (x0 + 16 * tf4 < X) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int l = 2 * (tid % 32) + u, row = 32 * mt + l % 32, col = 16 * tf4 + 8 * (l / 32);
                *reinterpret_cast<uint4 *>(xr + r_index(b, n * C + row, x0 + col, NT, X)) =
                    *reinterpret_cast<const uint4 *>(&tile[row][col]);
            }
        }
    }
    // Q layouts: feature xl, positions i0 .. i0+15 = two lanes' 16 bytes
    const int xl = tid / 4, i0 = (tid % 4) * 16;
    const int x = x0 + xl;
    if (x >= X) return;
    if (raw) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = static_cast<uint32_t>(tile[i0 + 8 * h + 2 * e][xl]) |
                       (static_cast<uint32_t>(tile[i0 + 8 * h + 2 * e + 1][xl]) << 16);
            *reinterpret_cast<uint4 *>(raw + q_index(b, n * C + i0 + 8 * h, x, NT, X)) = make_uint4(w[0], w[1], w[2], w[3]);
        }
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
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const size_t o = q_index(b, n * C + i0 + 8 * h, x, NT, X);
            *reinterpret_cast<uint4 *>(hi + o) = make_uint4(wh[4 * h], wh[4 * h + 1], wh[4 * h + 2], wh[4 * h + 3]);
            if (lo) *reinterpret_cast<uint4 *>(lo + o) = make_uint4(wl[4 * h], wl[4 * h + 1], wl[4 * h + 2], wl[4 * h + 3]);
        }
    }
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// grid (NT, B), 256 threads. From a and b in the R layout (K % 16 == 0), wave w
// computes the score tile (mt, nt) = (w/2, w%2) of the 64 x 64 chunk over all K
// (tile (0, 1) lies strictly above the diagonal and is zero in both outputs);
// P_lo and P_up go out in the tile layout (p_index) through an LDS transpose.
__global__ __launch_bounds__(256) void scores_kernel(const uint16_t *__restrict__ aR, const uint16_t *__restrict__ bR,
                                                     const float *__restrict__ g, uint16_t *__restrict__ Plo,
                                                     uint16_t *__restrict__ Pup, int K, int NT) {
    __shared__ __align__(16) uint16_t slo[C][C + 8], sup[C][C + 8];   // [i][j]
    const int n = blockIdx.x, b = blockIdx.y;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int lr = lane % 32, lh = lane / 32;
    const int mt = wave >> 1, nt = wave & 1;
    const int KT = K / 16;   // tiles per R row block
    f32x16 acc[4] = {};
    if (!(mt == 0 && nt == 1)) {
        const uint16_t *pa = aR + ((static_cast<size_t>(b) * (2 * NT) + 2 * n + mt) * KT) * kTileElems + 8 * lane;
        const uint16_t *pb = bR + ((static_cast<size_t>(b) * (2 * NT) + 2 * n + nt) * KT) * kTileElems + 8 * lane;
        int ks = 0;
        for (; ks + 4 <= KT; ks += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                acc[u] = mfma(*reinterpret_cast<const bf16x8 *>(pa + (ks + u) * kTileElems),
                              *reinterpret_cast<const bf16x8 *>(pb + (ks + u) * kTileElems), acc[u]);
        }
        for (; ks < KT; ++ks)
            acc[0] = mfma(*reinterpret_cast<const bf16x8 *>(pa + ks * kTileElems),
                          *reinterpret_cast<const bf16x8 *>(pb + ks * kTileElems), acc[0]);
    }
    const float gl = g[0];
    const int j = 32 * nt + lr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = 32 * mt + 8 * (r / 4) + 4 * lh + (r % 4);
        const float sv = acc[0][r] + acc[1][r] + acc[2][r] + acc[3][r];
        const int lag = i - j;
        const uint16_t v = f32_to_bf16_bits(lag >= 0 ? sv * __expf(gl * static_cast<float>(lag)) : 0.f);
        slo[i][j] = v;   // P_lo[i][j]
        sup[j][i] = v;   // P_up[j][i] = P_lo[i][j]
    }
    __syncthreads();
    // 2 x 8 tiles of 1 KB: thread -> 2 lanes of one tile of each
    const int tl = threadIdx.x / 32, tm = tl / 4, tq = tl % 4;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int l = 2 * (threadIdx.x % 32) + u, i = 32 * tm + l % 32, j0 = 16 * tq + 8 * (l / 32);
        const size_t o = p_index(b, n, i, j0, NT);
        *reinterpret_cast<uint4 *>(Plo + o) = *reinterpret_cast<const uint4 *>(&slo[i][j0]);
        *reinterpret_cast<uint4 *>(Pup + o) = *reinterpret_cast<const uint4 *>(&sup[i][j0]);
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

// Tiled copies of X (B, T, X): raw, hi, lo in the Q layout and xr in the R
// layout, each bf16 or null (X % 32 == 0). decay 0: no hi / lo; 1 / 2: hi (+ lo)
// hold the pre-decayed update operand of the forward / reversed walk.
int launch_chunk_transpose(const void *src, int src_dt, uint16_t *raw, uint16_t *hi, uint16_t *lo, uint16_t *xr,
                           const float *g, int decay, int B, int T, int X, hipStream_t s) {
    if (X % 32) return fail(ULM_ERR_INVALID, "chunk transpose: X=%d is not a multiple of 32", X);
    if (decay && !(hi && g)) return fail(ULM_ERR_INVALID, "chunk transpose: decayed output needs hi and g");
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    const dim3 grid((X + ULM_CHUNK - 1) / ULM_CHUNK, NT, B);
    if (decay == 1) chunks::transpose_kernel<1><<<grid, 256, 0, s>>>(src, src_dt, raw, hi, lo, xr, g, T, X, NT);
    else if (decay == 2) chunks::transpose_kernel<2><<<grid, 256, 0, s>>>(src, src_dt, raw, hi, lo, xr, g, T, X, NT);
    else chunks::transpose_kernel<0><<<grid, 256, 0, s>>>(src, src_dt, raw, nullptr, nullptr, xr, g, T, X, NT);
    return check_launch("chunk transpose_kernel");
}

// a, b in the R layout (K % 16 == 0); P_lo, P_up in the tile layout of p_index.
int launch_chunk_scores(const uint16_t *aR, const uint16_t *bR, const float *g, uint16_t *Plo, uint16_t *Pup, int B,
                        int T, int K, hipStream_t s) {
    if (K % 16) return fail(ULM_ERR_UNSUPPORTED, "chunk scores: K=%d is not a multiple of 16", K);
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    chunks::scores_kernel<<<dim3(NT, B), 256, 0, s>>>(aR, bR, g, Plo, Pup, K, NT);
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
