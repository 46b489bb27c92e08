// Per-chunk layouts consumed by the K-group chunked kernel (la_kgroup.hip).
//
//  * chunk_transpose: the tiled copies of a (B, T, X) tensor that the chunked
//    kernel loads (R and Q layouts of ulm_common.h; positions past T are zero),
//    each optionally with its bf16 rounding remainder.
//  * chunk_scores: per chunk n, with S[i][j] = a_{64n+i} . b_{64n+j},
//      P_lo[i][j] = S[i][j] lam^(i-j) / f_lo(i)  (j <= i, else 0)   forward walk
//      P_up[i][j] = S[j][i] lam^(j-i) / f_up(i)  (j >= i, else 0)   reversed walk
//    as bf16. P_lo is the intra-chunk matrix of o = LA(a, b, .) and P_up that
//    of the reversed product with a and b exchanged (LA_rev(b, a, .)), so one
//    pass serves fwd + dv (a = q, b = k) and dq + dk (a = dfast, b = v). This
//    is the _la_attn_kernel product (kernel.py:51-72), computed once per chunk
//    and shared by every value tile. With `scaled`, f is the chunked kernel's
//    read-out row factor, s lam^(i+1) forward and s lam^(64-i) reversed with s
//    the state scale at that walk step (readout_scale), and the chunked kernel
//    multiplies its summed row i by f once; that keeps every factor below 2^80
//    unless lam^64 < 2^-40, where f = 1. Without `scaled`, f = 1 and P_up is
//    exactly P_lo^T in bf16: the products behind the d/dg identity (dq, dk)
//    need their intra-chunk terms rounded identically on both sides.
//  * partial_reduce: out = sum over nK fp32 partial outputs (plus an optional fp32
//    residual), in out's dtype.
#include "ulm_common.h"

namespace ulm {

namespace chunks {

constexpr int C = ULM_CHUNK;

// grid (ceil(XL/64), NT, B), 256 threads: one 64-position x 64-feature block of
// X (B, T, X) in any float dtype, into layouts XL features wide (XL % 32 == 0,
// X <= XL; features X .. XL-1 are written as zeros). Outputs, each optional:
// raw = bf16(x) (+ raw_lo = bf16(x - raw), the rounding remainder) in the Q
// layout; xr = bf16(x) (+ xr_lo) in the R layout.
__global__ __launch_bounds__(256) void transpose_kernel(const void *__restrict__ src, int sdt, uint16_t *__restrict__ raw,
                                                        uint16_t *__restrict__ raw_lo, uint16_t *__restrict__ xr,
                                                        uint16_t *__restrict__ xr_lo, int T, int X, int XL, int NT) {
    __shared__ float tile[C][C + 1];   // [position][feature]
    const int x0 = blockIdx.x * C, n = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    {
        // position row i, 16 contiguous features; with X % 16 == 0 and a
        // 16-byte aligned source they are wholly in or out and 16-byte aligned
        const int i = tid / 4, c0 = (tid % 4) * 16;
        const int t = n * C + i;
        float vals[16];
        const bool vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 && X % 16 == 0;   // else one element at a time
        if (t < T && x0 + c0 < X && !vec) {
            const size_t o = (static_cast<size_t>(b) * T + t) * X + x0 + c0;
#pragma unroll
            for (int e = 0; e < 16; ++e) vals[e] = x0 + c0 + e < X ? load_as_f32(src, o + e, sdt) : 0.f;
        } else if (t < T && x0 + c0 < X) {
            const size_t o = (static_cast<size_t>(b) * T + t) * X + x0 + c0;
            if (sdt == ULM_F32) {
                const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(src) + o);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 w = p[k];
                    vals[4 * k] = w.x;
                    vals[4 * k + 1] = w.y;
                    vals[4 * k + 2] = w.z;
                    vals[4 * k + 3] = w.w;
                }
            } else {
                const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(src) + o);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const uint4 w = p[k];
                    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        const uint16_t lo16 = static_cast<uint16_t>(ws[h] & 0xffffu), hi16 = static_cast<uint16_t>(ws[h] >> 16);
                        if (sdt == ULM_BF16) {
                            vals[8 * k + 2 * h] = bf16_to_f32(lo16);
                            vals[8 * k + 2 * h + 1] = bf16_to_f32(hi16);
                        } else {
                            vals[8 * k + 2 * h] = static_cast<float>(__builtin_bit_cast(_Float16, lo16));
                            vals[8 * k + 2 * h + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi16));
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) vals[e] = 0.f;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) tile[i][c0 + e] = vals[e];
    }
    __syncthreads();
    if (xr) {
        // R layout: 64 positions x 64 features are 8 tiles; thread -> 2 lanes of one tile
        const int tl = tid / 32, mt = tl / 4, tf4 = tl % 4;
        if (x0 + 16 * tf4 < XL) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int l = 2 * (tid % 32) + u, row = 32 * mt + l % 32, col = 16 * tf4 + 8 * (l / 32);
                uint32_t wh[4], wl[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v0 = tile[row][col + 2 * e], v1 = tile[row][col + 2 * e + 1];
                    const uint16_t h0 = f32_to_bf16_bits(v0), h1 = f32_to_bf16_bits(v1);
                    wh[e] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
                    wl[e] = static_cast<uint32_t>(f32_to_bf16_bits(v0 - bf16_to_f32(h0))) |
                            (static_cast<uint32_t>(f32_to_bf16_bits(v1 - bf16_to_f32(h1))) << 16);
                }
                const size_t o = r_index(b, n * C + row, x0 + col, NT, XL);
                *reinterpret_cast<uint4 *>(xr + o) = make_uint4(wh[0], wh[1], wh[2], wh[3]);
                if (xr_lo) *reinterpret_cast<uint4 *>(xr_lo + o) = make_uint4(wl[0], wl[1], wl[2], wl[3]);
            }
        }
    }
    // Q layouts: feature xl, positions i0 .. i0+15 = two lanes' 16 bytes
    const int xl = tid / 4, i0 = (tid % 4) * 16;
    const int x = x0 + xl;
    if (x >= XL) return;
    if (raw) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t wh[4], wl[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v0 = tile[i0 + 8 * h + 2 * e][xl], v1 = tile[i0 + 8 * h + 2 * e + 1][xl];
                const uint16_t h0 = f32_to_bf16_bits(v0), h1 = f32_to_bf16_bits(v1);
                wh[e] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
                wl[e] = static_cast<uint32_t>(f32_to_bf16_bits(v0 - bf16_to_f32(h0))) |
                        (static_cast<uint32_t>(f32_to_bf16_bits(v1 - bf16_to_f32(h1))) << 16);
            }
            const size_t o = q_index(b, n * C + i0 + 8 * h, x, NT, XL);
            *reinterpret_cast<uint4 *>(raw + o) = make_uint4(wh[0], wh[1], wh[2], wh[3]);
            if (raw_lo) *reinterpret_cast<uint4 *>(raw_lo + o) = make_uint4(wl[0], wl[1], wl[2], wl[3]);
        }
    }
}

// The bf16 case of transpose_kernel with X % 32 == 0 and the layouts X wide:
// grid (ceil(X / 256), NT, B), 256 threads, one tile_copy_bf16 job (64
// positions x 256 features) per workgroup.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ raw,
                                                             uint16_t *__restrict__ xr, int T, int X, int NT) {
    __shared__ __align__(16) copy_tile_t tile[kCopyBlocks];
    tile_copy_bf16(src, raw, xr, T, X, NT, blockIdx.x * kCopyBlocks * C, blockIdx.y, blockIdx.z, threadIdx.x, true,
                   tile);
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// grid (NT, B), 768 threads. From a and b in the R layout (K % 16 == 0), the
// three score tiles (mt, nt) of the 64 x 64 chunk on or below the diagonal,
// (0,0), (1,0), (1,1), are each computed by 4 waves over a quarter of K and
// summed through LDS in a fixed order (tile (0, 1) lies strictly above the
// diagonal and is zero in both outputs). P_lo and P_up go out in the tile
// layout (p_index) through an LDS transpose.
// ALO / BLO: a / b also come with bf16 remainders (a = ah + al, b = bh + bl);
// the product takes ah bh + ah bl + al bh over the parts present.
constexpr int kScoreWaves = 12;

template <bool ALO, bool BLO>
__global__ __launch_bounds__(kScoreWaves * 64) void scores_kernel(const uint16_t *__restrict__ aR,
                                                                  const uint16_t *__restrict__ aL,
                                                                  const uint16_t *__restrict__ bR,
                                                                  const uint16_t *__restrict__ bL,
                                                                  const float *__restrict__ g,
                                                                  uint16_t *__restrict__ Plo,
                                                                  uint16_t *__restrict__ Pup, int K, int NT,
                                                                  int scaled) {
    __shared__ __align__(16) uint16_t slo[C][C + 8], sup[C][C + 8];   // [i][j]
    __shared__ float red[3][3][16][kWave];                             // partials of quarters 1..3
    const int n = blockIdx.x, b = blockIdx.y;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int lr = lane % 32, lh = lane / 32;
    const int tile = wave / 4, kq = wave % 4;
    const int mt = tile == 0 ? 0 : 1, nt = tile == 2 ? 1 : 0;
    const int KT = K / 16;   // tiles per R row block
    const int k0 = (KT * kq) / 4, k1 = (KT * (kq + 1)) / 4;
    // the tile above the diagonal is zero in both outputs
    for (int e = threadIdx.x; e < 32 * 32; e += kScoreWaves * 64) {
        slo[e / 32][32 + e % 32] = 0;
        sup[32 + e / 32][e % 32] = 0;
    }
    f32x16 acc[2] = {};
    {
        const size_t oa = ((static_cast<size_t>(b) * (2 * NT) + 2 * n + mt) * KT) * kTileElems + 8 * lane;
        const size_t ob = ((static_cast<size_t>(b) * (2 * NT) + 2 * n + nt) * KT) * kTileElems + 8 * lane;
        // batches of 8 tile pairs: all loads of a batch in flight before its MFMAs;
        // two accumulators with fixed register indices
        constexpr int NB = 8;
        int ks = k0;
        for (; ks + NB <= k1; ks += NB) {
            bf16x8 x[NB], y[NB], xl[NB], yl[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const size_t t = static_cast<size_t>(ks + u) * kTileElems;
                x[u] = *reinterpret_cast<const bf16x8 *>(aR + oa + t);
                y[u] = *reinterpret_cast<const bf16x8 *>(bR + ob + t);
                if (ALO) xl[u] = *reinterpret_cast<const bf16x8 *>(aL + oa + t);
                if (BLO) yl[u] = *reinterpret_cast<const bf16x8 *>(bL + ob + t);
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                f32x16 &c = acc[u & 1];
                c = mfma(x[u], y[u], c);
                if (BLO) c = mfma(x[u], yl[u], c);
                if (ALO) c = mfma(xl[u], y[u], c);
            }
        }
        for (; ks < k1; ++ks) {
            const size_t t = static_cast<size_t>(ks) * kTileElems;
            const bf16x8 x = *reinterpret_cast<const bf16x8 *>(aR + oa + t);
            const bf16x8 y = *reinterpret_cast<const bf16x8 *>(bR + ob + t);
            acc[0] = mfma(x, y, acc[0]);
            if (BLO) acc[0] = mfma(x, *reinterpret_cast<const bf16x8 *>(bL + ob + t), acc[0]);
            if (ALO) acc[0] = mfma(*reinterpret_cast<const bf16x8 *>(aL + oa + t), y, acc[0]);
        }
    }
    if (kq > 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[tile][kq - 1][r][lane] = acc[0][r] + acc[1][r];
    }
    __syncthreads();
    if (kq == 0) {
        const float gl = g[0];
        const float lam64 = state_lam64(gl);
        const bool tiny = !scaled || lam64 < kRenorm;
        // unless tiny, the read-out row factors s lam^(i+1) (forward) and
        // s lam^(64-i) (reversed) are divided out here and applied after the
        // chunked kernel's cross-wave sum
        const float inv_f = tiny ? 1.f : 1.f / readout_scale(lam64, n);
        const float inv_r = tiny ? 1.f : 1.f / readout_scale(lam64, NT - 1 - n);
        const int j = 32 * nt + lr;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = 32 * mt + 8 * (r / 4) + 4 * lh + (r % 4);
            const float sv = (acc[0][r] + acc[1][r]) + red[tile][0][r][lane] + red[tile][1][r][lane] +
                             red[tile][2][r][lane];
            const bool on = i >= j;
            // P_lo[i][j] = lam^(i-j) S / (s lam^(i+1));  P_up[j][i] = lam^(i-j) S / (s lam^(64-j))
            const float elo = tiny ? static_cast<float>(i - j) : -static_cast<float>(j + 1);
            const float eup = tiny ? static_cast<float>(i - j) : static_cast<float>(i - C);
            slo[i][j] = f32_to_bf16_bits(on ? sv * (__expf(gl * elo) * inv_f) : 0.f);
            sup[j][i] = f32_to_bf16_bits(on ? sv * (__expf(gl * eup) * inv_r) : 0.f);
        }
    }
    __syncthreads();
    // 2 x 8 tiles of 1 KB: the first 256 threads, 2 lanes of one tile of each
    if (threadIdx.x < 256) {
        const int tl = threadIdx.x / 32, tm = tl / 4, tq = tl % 4;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int l = 2 * (threadIdx.x % 32) + u, i = 32 * tm + l % 32, j0 = 16 * tq + 8 * (l / 32);
            const size_t o = p_index(b, n, i, j0, NT);
            *reinterpret_cast<uint4 *>(Plo + o) = *reinterpret_cast<const uint4 *>(&slo[i][j0]);
            *reinterpret_cast<uint4 *>(Pup + o) = *reinterpret_cast<const uint4 *>(&sup[i][j0]);
        }
    }
}

// out[i] = sum_k part[k * n + i], written in out's dtype
__global__ __launch_bounds__(256) void partial_reduce_kernel(const float *__restrict__ part, int nK, size_t n,
                                                             const float *__restrict__ resid,
                                                             void *__restrict__ out, int odt, bool vec) {
    const size_t n4 = vec ? n / 4 : 0;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 s = reinterpret_cast<const float4 *>(part)[i];
        if (resid) {
            const float4 x = reinterpret_cast<const float4 *>(resid)[i];
            s.x += x.x;
            s.y += x.y;
            s.z += x.z;
            s.w += x.w;
        }
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
        float s = part[i] + (resid ? resid[i] : 0.f);
        for (int k = 1; k < nK; ++k) s += part[k * n + i];
        store_from_f32(out, i, odt, s);
    }
}

// The padded-width form of partial_reduce: part holds nK partial (B, Rp, Fp)
// arrays; out (B, R, F) takes, for r < R and f < F, sum_k part[k][b][r][f]
// (+ resid[b][r][f]) in out's dtype. The padding rows and columns are dropped.
__global__ __launch_bounds__(256) void unpad_sum_kernel(const float *__restrict__ part, int nK, int R, int Rp, int F,
                                                        int Fp, size_t n, const float *__restrict__ resid,
                                                        void *__restrict__ out, int odt) {
    const size_t kstride = n / (static_cast<size_t>(R) * F) * Rp * Fp;   // B Rp Fp
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const size_t row = i / F;
        const int f = static_cast<int>(i % F);
        const size_t src = (row / R * Rp + row % R) * Fp + f;
        float s = part[src] + (resid ? resid[i] : 0.f);
        for (int k = 1; k < nK; ++k) s += part[k * kstride + src];
        store_from_f32(out, i, odt, s);
    }
}

}  // namespace chunks

// Tiled copies of X (B, T, X): raw (+ raw_lo) in the Q layout and xr (+ xr_lo)
// in the R layout, each bf16 or null, XL features wide (0: XL = X; XL % 32 ==
// 0 and X <= XL, the features past X zero).
int launch_chunk_transpose(const void *src, int src_dt, uint16_t *raw, uint16_t *raw_lo, uint16_t *xr,
                           uint16_t *xr_lo, int B, int T, int X, hipStream_t s, int XL) {
    if (XL == 0) XL = X;
    if (XL % 32 || X > XL) return fail(ULM_ERR_INVALID, "chunk transpose: layout width %d for X=%d", XL, X);
    if (raw_lo && !raw) return fail(ULM_ERR_INVALID, "chunk transpose: raw_lo needs raw");
    if (xr_lo && !xr) return fail(ULM_ERR_INVALID, "chunk transpose: xr_lo needs xr");
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    if (src_dt == ULM_BF16 && X % 32 == 0 && XL == X && !raw_lo && !xr_lo && reinterpret_cast<uintptr_t>(src) % 16 == 0) {
        const dim3 grid((X + 4 * ULM_CHUNK - 1) / (4 * ULM_CHUNK), NT, B);
        chunks::transpose_bf16_kernel<<<grid, 256, 0, s>>>(static_cast<const uint16_t *>(src), raw, xr, T, X, NT);
        return check_launch("chunk transpose_bf16_kernel");
    }
    const dim3 grid((XL + ULM_CHUNK - 1) / ULM_CHUNK, NT, B);
    chunks::transpose_kernel<<<grid, 256, 0, s>>>(src, src_dt, raw, raw_lo, xr, xr_lo, T, X, XL, NT);
    return check_launch("chunk transpose_kernel");
}

// a, b in the R layout (K % 16 == 0), with optional bf16 remainders aL, bL;
// P_lo, P_up in the tile layout of p_index.
int launch_chunk_scores(const uint16_t *aR, const uint16_t *aL, const uint16_t *bR, const uint16_t *bL, const float *g,
                        uint16_t *Plo, uint16_t *Pup, int B, int T, int K, bool scaled, hipStream_t s) {
    if (K % 16) return fail(ULM_ERR_UNSUPPORTED, "chunk scores: K=%d is not a multiple of 16", K);
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    const dim3 grid(NT, B);
    const int nthreads = chunks::kScoreWaves * kWave;
    if (aL && bL) chunks::scores_kernel<true, true><<<grid, nthreads, 0, s>>>(aR, aL, bR, bL, g, Plo, Pup, K, NT, scaled ? 1 : 0);
    else if (aL) chunks::scores_kernel<true, false><<<grid, nthreads, 0, s>>>(aR, aL, bR, bL, g, Plo, Pup, K, NT, scaled ? 1 : 0);
    else if (bL) chunks::scores_kernel<false, true><<<grid, nthreads, 0, s>>>(aR, aL, bR, bL, g, Plo, Pup, K, NT, scaled ? 1 : 0);
    else chunks::scores_kernel<false, false><<<grid, nthreads, 0, s>>>(aR, aL, bR, bL, g, Plo, Pup, K, NT, scaled ? 1 : 0);
    return check_launch("chunk scores_kernel");
}

// out (B, R, F) = the sum of nK partial (B, Rp, Fp) arrays (+ resid (B, R, F)
// when not null) without their padding, as odt.
int launch_unpad_sum(const float *part, int nK, int B, int R, int Rp, int F, int Fp, void *out, int odt, hipStream_t s,
                     const float *resid) {
    if (R > Rp || F > Fp) return fail(ULM_ERR_INVALID, "unpad sum: %dx%d from %dx%d", R, F, Rp, Fp);
    const size_t n = static_cast<size_t>(B) * R * F;
    if (n == 0) return ULM_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    chunks::unpad_sum_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(part, nK, R, Rp, F, Fp, n, resid, out, odt);
    return check_launch("unpad_sum_kernel");
}

// out = sum of the nK partial rows of part (+ resid when not null), as odt.
int launch_partial_reduce(const float *part, int nK, size_t n, void *out, int odt, hipStream_t s,
                          const float *resid) {
    if (n == 0) return ULM_OK;
    // float4 path when every partial row, the residual and the output are 16-byte aligned
    const bool vec = n % 4 == 0 && reinterpret_cast<uintptr_t>(part) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(resid) % 16 == 0 &&
                     (odt != ULM_F32 || reinterpret_cast<uintptr_t>(out) % 16 == 0);
    size_t blocks = ((vec ? n / 4 : n) + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    chunks::partial_reduce_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(part, nK, n, resid, out, odt, vec);
    return check_launch("partial_reduce_kernel");
}

}  // namespace ulm
