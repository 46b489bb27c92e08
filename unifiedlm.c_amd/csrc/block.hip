// The elementwise ends of UnifiedBlock around its GEMMs and the fast memory,
// fused: RMSNorm + causal depthwise conv in the forward, and in the backward
// their chain rule together with the residual branch.
//
// Forward (model.py:78-79, RMSNorm model.py:31-42, conv model.py:63): per
// position t of batch row b,
//   rstd_t = (mean_d x_t,d^2 + eps)^-1/2,   h_t = (x_t rstd_t) * norm_w,
//   u_t,d  = sum_j conv_w[d, j] h_{t-(Kc-1)+j, d}   (h = 0 before position 0),
// i.e. nn.Conv1d(groups=D, padding=Kc-1) truncated to the first T outputs.
// Backward, with du = dL/du, dhv = dL/dh from the value GEMM, dres = dL/dout
// of the residual x + ...:
//   dh_t  = dhv_t + sum_j conv_w[:, j] du_{t+(Kc-1)-j}
//   dconv_w[d, j] = sum_t du_t,d h_{t-(Kc-1)+j, d},   dnorm_w = sum_t dh_t xn_t
//   dx_t  = dres_t + rstd_t (dxn_t - xn_t <dxn_t, xn_t> / D),  xn = x rstd, dxn = dh norm_w
// The weight gradients are summed per tile of positions into partials and
// then over tiles by a fixed-order column sum (deterministic, no atomics).
#include "ulm_common.h"

namespace ulm {
namespace blk {

constexpr int kThreads = 256;
constexpr int kFwdTP = 32;    // positions per forward workgroup
constexpr int kMaxTaps = 8;   // conv windows are kMaxTaps wide; unused taps are zero
constexpr int kBatch = 8;     // rows whose loads a channel walk issues together

template <typename T> __device__ __forceinline__ float ldf(const T *p, size_t i);
template <> __device__ __forceinline__ float ldf<float>(const float *p, size_t i) { return p[i]; }
template <> __device__ __forceinline__ float ldf<uint16_t>(const uint16_t *p, size_t i) { return bf16_to_f32(p[i]); }
template <> __device__ __forceinline__ float ldf<_Float16>(const _Float16 *p, size_t i) { return static_cast<float>(p[i]); }

template <typename T> __device__ __forceinline__ void stf(T *p, size_t i, float v);
template <> __device__ __forceinline__ void stf<float>(float *p, size_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void stf<uint16_t>(uint16_t *p, size_t i, float v) { p[i] = f32_to_bf16_bits(v); }
template <> __device__ __forceinline__ void stf<_Float16>(_Float16 *p, size_t i, float v) { p[i] = static_cast<_Float16>(v); }

// Loads are unconditional (clamped to a valid index, the value then masked),
// so no load sits in a branch that would wait for it.

// One workgroup per (32 positions, batch row): rstd of the rows t0 - (Kc-1) ..
// t0 + 31, one wave per row, then a channel-parallel walk over those rows with
// h at the last 8 positions in registers (taps right-aligned: wa[8-Kc+j] = cw[j]).
template <typename TX, typename TO>
__global__ __launch_bounds__(kThreads) void norm_conv_fwd_kernel(const TX *__restrict__ x, const float *__restrict__ nw,
                                                                 const float *__restrict__ cw, int Kc, float eps,
                                                                 TO *__restrict__ h, TO *__restrict__ u,
                                                                 float *__restrict__ rstd, int T, int D) {
    constexpr int halo = kMaxTaps - 1;
    __shared__ float rs[kFwdTP + halo];   // rows t0 - halo .. t0 + kFwdTP - 1
    const int t0 = blockIdx.x * kFwdTP;
    const int tfirst = max(0, t0 - (Kc - 1));
    const int tend = min(T, t0 + kFwdTP);
    const size_t row0 = static_cast<size_t>(blockIdx.y) * T;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    for (int i = wave; i < kFwdTP + halo; i += kThreads / kWave) {
        const int t = t0 - halo + i;
        const bool ok = t >= tfirst && t < tend;
        float ss = 0.f;
        if (ok) {
            const TX *xr = x + (row0 + t) * D;
#pragma unroll 4
            for (int d = lane; d < D; d += kWave) {
                const float v = ldf(xr, d);
                ss += v * v;
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) {
            const float r = ok ? rsqrtf(ss / static_cast<float>(D) + eps) : 0.f;
            rs[i] = r;
            if (ok && t >= t0) rstd[row0 + t] = r;
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float wa[kMaxTaps], win[kMaxTaps];   // taps and h at positions t-7 .. t
#pragma unroll
        for (int m = 0; m < kMaxTaps; ++m) {
            const int j = m - (kMaxTaps - Kc);
            wa[m] = j >= 0 ? cw[static_cast<size_t>(d) * Kc + max(j, 0)] : 0.f;
            win[m] = 0.f;
        }
        const float nwd = nw[d];
        // rows in batches of kBatch: the batch's loads are issued together
        for (int tb = tfirst; tb < tend; tb += kBatch) {
            float xv[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) xv[k] = ldf(x, (row0 + min(tb + k, tend - 1)) * D + d);
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int t = tb + k;
                if (t >= tend) break;
                const size_t o = (row0 + t) * D + d;
                const float hv = (xv[k] * rs[t - t0 + halo]) * nwd;
#pragma unroll
                for (int m = 0; m + 1 < kMaxTaps; ++m) win[m] = win[m + 1];
                win[kMaxTaps - 1] = hv;
                if (t >= t0) {
                    float acc = 0.f;
#pragma unroll
                    for (int m = 0; m < kMaxTaps; ++m) acc += wa[m] * win[m];
                    stf(h, o, hv);
                    stf(u, o, acc);
                }
            }
        }
    }
}

// One workgroup per (tile of tp positions, batch row). With the window of du
// anchored at t + Kc - 1, dv[m] = du_{t+Kc-8+m}:
//   dh_t = dhv_t + sum_j cw[j] dv[7-j],   dconv_w[j] += h_t dv[7-j]
// (the second sums du_{s+Kc-1-j} h_s over the tile's own positions s, so no
// earlier rows are read). Dynamic LDS: dh (tp x D fp32), tp x kThreads row-dot
// partials, tp rstd. Partials: pnw (ntiles, D), pcw (ntiles, D, Kc).
template <typename TX, typename TD>
__global__ __launch_bounds__(kThreads) void norm_conv_bwd_kernel(const TX *__restrict__ x,
                                                                 const float *__restrict__ rstd,
                                                                 const float *__restrict__ nw,
                                                                 const float *__restrict__ cw, int Kc,
                                                                 const TD *__restrict__ du,
                                                                 const TD *__restrict__ dhv, const float *dres,
                                                                 float *dx, float *__restrict__ pnw,
                                                                 float *__restrict__ pcw, int T, int D, int tp) {
    extern __shared__ __align__(16) float lds[];
    float *const dh_s = lds;                                      // [tp][D]
    float *const rdot = lds + static_cast<size_t>(tp) * D;        // [tp][kThreads]
    float *const rs = rdot + static_cast<size_t>(tp) * kThreads;  // [tp]
    const int t0 = blockIdx.x * tp;
    const size_t row0 = static_cast<size_t>(blockIdx.y) * T;
    const size_t tile = static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    const int tend = min(T, t0 + tp);
    for (int i = threadIdx.x; i < tp; i += kThreads) rs[i] = t0 + i < T ? rstd[row0 + t0 + i] : 0.f;
    for (int i = 0; i < tp; ++i) rdot[i * kThreads + threadIdx.x] = 0.f;
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float cl[kMaxTaps], dv[kMaxTaps], gcw[kMaxTaps];   // taps left-aligned, du window, dconv_w partials
#pragma unroll
        for (int j = 0; j < kMaxTaps; ++j) {
            cl[j] = j < Kc ? cw[static_cast<size_t>(d) * Kc + min(j, Kc - 1)] : 0.f;
            gcw[j] = 0.f;
        }
        // prime: dv[m + 1] = du at t0 + Kc - 8 + m, rows t0 .. t0 + Kc - 2 only (the rest meet zero taps)
#pragma unroll
        for (int m = 0; m + 1 < kMaxTaps; ++m) {
            const int tu = t0 + Kc - kMaxTaps + m;
            const bool ok = tu >= t0 && tu < T;
            const float v = ldf(du, (row0 + (ok ? tu : t0)) * D + d);
            dv[m + 1] = ok ? v : 0.f;
        }
        dv[0] = 0.f;
        const float nwd = nw[d];
        float gnw = 0.f;
        for (int tb = t0; tb < tend; tb += kBatch) {
            // the batch's loads first: x, the next du and dhv of up to kBatch rows
            float xv[kBatch], nv[kBatch], hv[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int t = min(tb + k, tend - 1), tn = t + Kc - 1;
                const size_t o = (row0 + t) * D + d;
                xv[k] = ldf(x, o);
                nv[k] = ldf(du, (row0 + (tn < T ? tn : t)) * D + d);
                nv[k] = tn < T ? nv[k] : 0.f;
                hv[k] = dhv ? ldf(dhv, o) : 0.f;
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int t = tb + k;
                if (t >= tend) break;
                const float xn = xv[k] * rs[t - t0];
#pragma unroll
                for (int m = 0; m + 1 < kMaxTaps; ++m) dv[m] = dv[m + 1];
                dv[kMaxTaps - 1] = nv[k];
                float dh = hv[k];
                const float ht = xn * nwd;
#pragma unroll
                for (int j = 0; j < kMaxTaps; ++j) {
                    dh += cl[j] * dv[kMaxTaps - 1 - j];
                    gcw[j] += ht * dv[kMaxTaps - 1 - j];
                }
                gnw += dh * xn;
                dh_s[static_cast<size_t>(t - t0) * D + d] = dh;
                rdot[(t - t0) * kThreads + threadIdx.x] += dh * nwd * xn;
            }
        }
        pnw[tile * D + d] = gnw;
#pragma unroll
        for (int j = 0; j < kMaxTaps; ++j)
            if (j < Kc) pcw[(tile * D + d) * Kc + j] = gcw[j];
    }
    __syncthreads();
    // row dots in a fixed order: thread i < tp sums row i
    if (threadIdx.x < tp) {
        float sum = 0.f;
        for (int k = 0; k < kThreads; ++k) sum += rdot[threadIdx.x * kThreads + k];
        rdot[threadIdx.x * kThreads] = sum;
    }
    __syncthreads();
    const float invD = 1.f / static_cast<float>(D);
    for (int t = t0; t < tend; ++t) {
        const float rst = rs[t - t0];
        const float dot = rdot[(t - t0) * kThreads] * invD;
#pragma unroll 4
        for (int d = threadIdx.x; d < D; d += kThreads) {
            const size_t o = (row0 + t) * D + d;
            const float xn = ldf(x, o) * rst;
            const float dxn = dh_s[static_cast<size_t>(t - t0) * D + d] * nw[d];
            const float g = rst * (dxn - xn * dot);
            dx[o] = (dres ? dres[o] : 0.f) + g;
        }
    }
}

// Channel-per-thread backward for D <= kColsMaxD: one workgroup per (kColTP
// positions, batch row) with a thread per channel, which issues all of its
// tile's loads at once (x, dh_v, d_res of the kColTP rows and du of the
// kColTP + 7 rows of its window) and keeps dh, xn in registers, so x is read
// once and no dh buffer is staged. The conv taps are right-aligned, ca[m] =
// cw[Kc-1-m] (zero for m >= Kc), so with du_w[m] = du_{t0+m}:
//   dh_{t0+i} = dhv + sum_m ca[m] du_w[i+m],   g2[m] += h_{t0+i} du_w[i+m],
// and dconv_w[j] is g2[Kc-1-j]. The row dots <dxn, xn> are wave sums, then a
// fixed-order sum over the waves in LDS. Partials: one row per tile,
// [dnorm_w (D) | dconv_w (D, Kc)], summed over tiles by one column sum.
constexpr int kColTP = 16;
constexpr int kColsMaxD = 1024;
constexpr int kColWin = kColTP + kMaxTaps - 1;

template <typename T> __device__ __forceinline__ float ldrow(const T *row, uint32_t d);
template <> __device__ __forceinline__ float ldrow<float>(const float *row, uint32_t d) { return ld_row(row, 4u * d); }
template <> __device__ __forceinline__ float ldrow<uint16_t>(const uint16_t *row, uint32_t d) {
    return bf16_to_f32(ld_row(row, 2u * d));
}
template <> __device__ __forceinline__ float ldrow<_Float16>(const _Float16 *row, uint32_t d) {
    return static_cast<float>(ld_row(row, 2u * d));
}

template <typename TX, typename TD>
__global__ __launch_bounds__(kColsMaxD) void norm_conv_bwd_cols_kernel(
    const TX *__restrict__ x, const float *__restrict__ rstd, const float *__restrict__ nw,
    const float *__restrict__ cw, int Kc, const TD *__restrict__ du, const TD *__restrict__ dhv,
    const float *dres, float *dx, float *__restrict__ pw, int T, int D) {
    __shared__ float part[kColTP][kColsMaxD / kWave];   // per-wave row-dot partials
    __shared__ float dots[kColTP];
    const int d = threadIdx.x, wave = d / kWave, lane = d % kWave, nwave = blockDim.x / kWave;
    const bool vd = d < D;
    const uint32_t dc = vd ? d : 0;
    const int t0 = blockIdx.x * kColTP;
    const size_t row0 = static_cast<size_t>(blockIdx.y) * T;
    const size_t tile = static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    // rows are clamped on wave-uniform conditions, channels per lane; values masked after
    auto urow = [&](int t) { return row0 + static_cast<size_t>(t < T ? t : T - 1); };
    float xv[kColTP], hv[kColTP], rv[kColTP], dv[kColWin], ca[kMaxTaps];
#pragma unroll
    for (int i = 0; i < kColTP; ++i) {
        const int t = t0 + i;
        const bool ok = vd && t < T;
        const size_t r = urow(t);
        const float a = ldrow(x + r * D, dc);
        xv[i] = ok ? a : 0.f;
        const float h = dhv ? ldrow(dhv + r * D, dc) : 0.f;
        hv[i] = ok ? h : 0.f;
        rv[i] = t < T ? rstd[r] : 0.f;
    }
#pragma unroll
    for (int m = 0; m < kColWin; ++m) {
        const int t = t0 + m;
        const bool ok = vd && t < T && m < kColTP + Kc - 1;
        const float v = ldrow(du + urow(t) * D, dc);
        dv[m] = ok ? v : 0.f;
    }
#pragma unroll
    for (int m = 0; m < kMaxTaps; ++m) ca[m] = m < Kc ? cw[static_cast<size_t>(dc) * Kc + (Kc - 1 - m)] : 0.f;
    const float nwd = vd ? nw[dc] : 0.f;
    float g2[kMaxTaps], dh[kColTP], rd[kColTP];
#pragma unroll
    for (int m = 0; m < kMaxTaps; ++m) g2[m] = 0.f;
    float gnw = 0.f;
#pragma unroll
    for (int i = 0; i < kColTP; ++i) {
        const float xn = xv[i] * rv[i];
        const float ht = xn * nwd;
        float a = hv[i];
#pragma unroll
        for (int m = 0; m < kMaxTaps; ++m) {
            a += ca[m] * dv[i + m];
            g2[m] += ht * dv[i + m];
        }
        dh[i] = a;
        gnw += a * xn;
        xv[i] = xn;
        rd[i] = wave_sum(a * nwd * xn);
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < kColTP; ++i) part[i][wave] = rd[i];
    }
    // d_res loads go out before the barrier, with the row sums in flight
    float dr[kColTP];
#pragma unroll
    for (int i = 0; i < kColTP; ++i) {
        const int t = t0 + i;
        const float v = dres ? ld_row(dres + urow(t) * D, 4u * dc) : 0.f;
        dr[i] = (vd && t < T) ? v : 0.f;
    }
    __syncthreads();
    // thread i < kColTP sums row i over the waves in a fixed order
    if (d < kColTP) {
        float dot = 0.f;
        for (int w = 0; w < nwave; ++w) dot += part[d][w];
        dots[d] = dot * (1.f / static_cast<float>(D));
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kColTP; ++i) {
        const int t = t0 + i;
        const float dot = dots[i];
        const float g = rv[i] * (dh[i] * nwd - xv[i] * dot);
        if (vd && t < T) st_row(dx + (row0 + t) * D, 4u * dc, dr[i] + g);
    }
    if (vd) {
        float *const row = pw + tile * D * (Kc + 1);
        row[d] = gnw;
#pragma unroll
        for (int m = 0; m < kMaxTaps; ++m)
            if (m < Kc) row[D + d * Kc + (Kc - 1 - m)] = g2[m];
    }
}

// Channel-per-thread forward for D <= kColsMaxD: one workgroup per
// (kColTP positions, batch row), a thread per channel. Each thread loads x of
// its channel at the tile's kColTP rows and the kMaxTaps - 1 rows before them
// once (halo rows a conv with Kc < kMaxTaps does not reach are clamped onto
// the tile's first row, already loaded); the rows' mean squares are wave sums
// plus a fixed-order sum over the waves in LDS; h and the conv output u
// (taps right-aligned, wa[q] = cw[q - (kMaxTaps - Kc)]) go out from registers.
template <typename TX, typename TO>
__global__ __launch_bounds__(1024) void norm_conv_fwd_cols_kernel(const TX *__restrict__ x,
                                                                  const float *__restrict__ nw,
                                                                  const float *__restrict__ cw, int Kc, float eps,
                                                                  TO *__restrict__ h, TO *__restrict__ u,
                                                                  float *__restrict__ rstd, int T, int D) {
    constexpr int halo = kMaxTaps - 1;
    constexpr int W = kColTP + halo;   // rows t0 - halo .. t0 + kColTP - 1
    __shared__ float part[W][1024 / kWave];
    __shared__ float rs[W];
    const int d = threadIdx.x, wave = d / kWave, lane = d % kWave, nwave = blockDim.x / kWave;
    const bool vd = d < D;
    const uint32_t dc = vd ? d : 0;
    const int t0 = blockIdx.x * kColTP;
    const size_t row0 = static_cast<size_t>(blockIdx.y) * T;
    const int first = kMaxTaps - Kc;   // rows m < first meet zero taps only
    float xv[W];
#pragma unroll
    for (int m = 0; m < W; ++m) {
        const int t = t0 - halo + m;
        const bool used = m >= first && t >= 0 && t < T;   // wave-uniform
        const int tr = used ? t : min(t0, T - 1);
        const float v = ldrow(x + (row0 + tr) * D, dc);
        xv[m] = (used && vd) ? v : 0.f;
    }
#pragma unroll
    for (int m = 0; m < W; ++m) {
        const float ss = wave_sum(xv[m] * xv[m]);
        if (lane == 0) part[m][wave] = ss;
    }
    float wa[kMaxTaps];
#pragma unroll
    for (int q = 0; q < kMaxTaps; ++q) wa[q] = q >= first ? cw[static_cast<size_t>(dc) * Kc + (q - first)] : 0.f;
    const float nwd = vd ? nw[dc] : 0.f;
    __syncthreads();
    // thread m < W sums row m over the waves in a fixed order
    if (d < W) {
        const int t = t0 - halo + d;
        float ss = 0.f;
        for (int w = 0; w < nwave; ++w) ss += part[d][w];
        const bool ok = d >= first && t >= 0 && t < T;
        const float r = ok ? rsqrtf(ss * (1.f / static_cast<float>(D)) + eps) : 0.f;
        rs[d] = r;
        if (d >= halo && t < T) rstd[row0 + t] = r;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < W; ++m) xv[m] = (xv[m] * rs[m]) * nwd;   // h
#pragma unroll
    for (int i = 0; i < kColTP; ++i) {
        const int t = t0 + i;
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < kMaxTaps; ++q) acc += wa[q] * xv[i + q];
        if (vd && t < T) {
            const size_t o = (row0 + t) * D + d;
            stf(h, o, xv[halo + i]);
            stf(u, o, acc);
        }
    }
}

constexpr int kSplit = 32;   // first-level row ranges of the weight-gradient sums

constexpr size_t kBwdLds = 80 * 1024;   // two backward workgroups per CU (160 KiB of LDS)

size_t bwd_lds_bytes(int tp, int D, int) {
    return (static_cast<size_t>(tp) * D + static_cast<size_t>(tp) * kThreads + tp) * 4;
}

// positions per backward workgroup: kColTP for the channel-per-thread kernel
// (D <= kColsMaxD), else the largest of 16, 8, 4, 2, 1 whose LDS fits kBwdLds
int bwd_tile(int D, int Kc) {
    if (D <= kColsMaxD) return kColTP;
    for (int tp = 16; tp >= 1; tp /= 2)
        if (bwd_lds_bytes(tp, D, Kc) <= kBwdLds) return tp;
    return 0;
}

struct BwdWs {
    float *pnw, *pcw, *tmp;
    size_t bytes;
};

BwdWs bwd_layout(void *base, int B, int T, int D, int Kc) {
    const int tp = bwd_tile(D, Kc);
    const size_t ntile = tp ? static_cast<size_t>(B) * ((T + tp - 1) / tp) : 0;
    Carver c(base);
    BwdWs w{};
    w.pnw = c.take<float>(ntile * D);
    w.pcw = c.take<float>(ntile * D * Kc);
    w.tmp = c.take<float>(static_cast<size_t>(kSplit) * D * (Kc + 1));
    w.bytes = c.off;
    return w;
}

template <typename TX, typename TO>
int launch_fwd(const void *x, const float *nw, const float *cw, int Kc, float eps, void *h, void *u, float *rstd, int B,
               int T, int D, hipStream_t s) {
    if (D <= kColsMaxD) {
        const int nth = (D + kWave - 1) / kWave * kWave;
        norm_conv_fwd_cols_kernel<TX, TO><<<dim3((T + kColTP - 1) / kColTP, B), nth, 0, s>>>(
            static_cast<const TX *>(x), nw, cw, Kc, eps, static_cast<TO *>(h), static_cast<TO *>(u), rstd, T, D);
        return check_launch("norm_conv_fwd_cols_kernel");
    }
    const dim3 grid((T + kFwdTP - 1) / kFwdTP, B);
    norm_conv_fwd_kernel<TX, TO><<<grid, kThreads, 0, s>>>(static_cast<const TX *>(x), nw, cw, Kc, eps,
                                                           static_cast<TO *>(h), static_cast<TO *>(u), rstd, T, D);
    return check_launch("norm_conv_fwd_kernel");
}

template <typename TX, typename TD>
int launch_bwd(const void *x, const float *rstd, const float *nw, const float *cw, int Kc, const void *du,
               const void *dhv, const float *dres, float *dx, float *dnw, float *dcw, void *workspace, int B, int T,
               int D, hipStream_t s) {
    const int tp = bwd_tile(D, Kc);
    const BwdWs ws = bwd_layout(workspace, B, T, D, Kc);
    const int ntx = (T + tp - 1) / tp;
    const size_t ntile = static_cast<size_t>(B) * ntx;
    if (D <= kColsMaxD) {
        const int nth = (D + kWave - 1) / kWave * kWave;
        norm_conv_bwd_cols_kernel<TX, TD><<<dim3(ntx, B), nth, 0, s>>>(
            static_cast<const TX *>(x), rstd, nw, cw, Kc, static_cast<const TD *>(du), static_cast<const TD *>(dhv),
            dres, dx, ws.pnw, T, D);
        ULM_TRY(check_launch("norm_conv_bwd_cols_kernel"));
        // pnw and pcw are carved back to back: their span holds ntile rows of D (Kc + 1)
        return launch_column_sum2(ws.pnw, ntile, D, static_cast<size_t>(D) * Kc, ws.tmp, kSplit, dnw, dcw, s);
    }
    const size_t lds = bwd_lds_bytes(tp, D, Kc);
    static bool attr_done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return check_launch("hipGetDevice");
    if (!attr_done[dev]) {
        const void *fn = reinterpret_cast<const void *>(&norm_conv_bwd_kernel<TX, TD>);
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kBwdLds)) !=
            hipSuccess)
            return check_launch("norm_conv_bwd_kernel attribute");
        attr_done[dev] = true;
    }
    norm_conv_bwd_kernel<TX, TD><<<dim3(ntx, B), kThreads, lds, s>>>(
        static_cast<const TX *>(x), rstd, nw, cw, Kc, static_cast<const TD *>(du), static_cast<const TD *>(dhv), dres,
        dx, ws.pnw, ws.pcw, T, D, tp);
    ULM_TRY(check_launch("norm_conv_bwd_kernel"));
    ULM_TRY(launch_column_sum(ws.pnw, ntile, D, ws.tmp, kSplit, dnw, s));
    return launch_column_sum(ws.pcw, ntile, static_cast<size_t>(D) * Kc, ws.tmp, kSplit, dcw, s);
}

// The block's fast-memory parameters from their logs (model.py:75, 84):
// g = -exp(log_rate), w = exp(clamp(log_w, lo, hi)); and the chain rule back,
// d log_rate = dg g, d log_w = dw w where lo <= log_w <= hi, else 0 (the
// gradient torch's clamp passes).
__global__ __launch_bounds__(256) void params_fwd_kernel(const float *__restrict__ log_rate,
                                                         const float *__restrict__ log_w, float lo, float hi, int A,
                                                         float *__restrict__ g, float *__restrict__ w) {
    const int a = blockIdx.x * 256 + threadIdx.x;
    if (a < A) w[a] = expf(fminf(fmaxf(log_w[a], lo), hi));
    if (a == 0) g[0] = -expf(log_rate[0]);
}

__global__ __launch_bounds__(256) void params_bwd_kernel(const float *__restrict__ log_rate,
                                                         const float *__restrict__ log_w, float lo, float hi,
                                                         const float *__restrict__ dg, const float *__restrict__ dw,
                                                         int A, float *__restrict__ dlog_rate,
                                                         float *__restrict__ dlog_w) {
    const int a = blockIdx.x * 256 + threadIdx.x;
    if (a < A) {
        const float x = log_w[a];
        const float wa = expf(fminf(fmaxf(x, lo), hi));
        dlog_w[a] = (x >= lo && x <= hi) ? dw[a] * wa : 0.f;
    }
    if (a == 0) dlog_rate[0] = dg[0] * -expf(log_rate[0]);
}

// Calls f.template operator()<T>() with T the element type of dtype dt.
template <class F>
int with_type(int dt, F &&f) {
    switch (dt) {
    case ULM_F32: return f(float{});
    case ULM_BF16: return f(uint16_t{});
    case ULM_F16: return f(_Float16{});
    }
    return fail(ULM_ERR_INVALID, "bad dtype %d", dt);
}

}  // namespace blk
}  // namespace ulm

using namespace ulm;

namespace {

bool x_dtype_ok(int dt) { return dt == ULM_F32 || dt == ULM_BF16; }

}  // namespace

extern "C" int ulm_norm_conv_fwd(const void *x, int x_dtype, const float *norm_w, const float *conv_w, int Kc,
                                 float norm_eps, void *h, int h_dtype, void *u, int u_dtype, float *rstd, int B, int T,
                                 int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && D > 0, "ulm_norm_conv_fwd: bad sizes B=%d T=%d D=%d", B, T, D);
    ULM_REQUIRE(Kc >= 1 && Kc <= blk::kMaxTaps, "ulm_norm_conv_fwd: Kc=%d outside 1..%d", Kc, blk::kMaxTaps);
    ULM_REQUIRE(x_dtype_ok(x_dtype) && valid_dtype(h_dtype) && h_dtype == u_dtype,
                "ulm_norm_conv_fwd: bad dtypes x %d, h %d, u %d (h and u share one)", x_dtype, h_dtype, u_dtype);
    ULM_REQUIRE(x && norm_w && conv_w && h && u && rstd, "ulm_norm_conv_fwd: null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    return blk::with_type(x_dtype, [&](auto tx) {
        return blk::with_type(h_dtype, [&](auto to) {
            return blk::launch_fwd<decltype(tx), decltype(to)>(x, norm_w, conv_w, Kc, norm_eps, h, u, rstd, B, T, D, s);
        });
    });
}

extern "C" size_t ulm_norm_conv_bwd_workspace_bytes(int B, int T, int D, int Kc) {
    if (B <= 0 || T <= 0 || D <= 0 || Kc < 1 || Kc > blk::kMaxTaps || !blk::bwd_tile(D, Kc)) return 0;
    return blk::bwd_layout(nullptr, B, T, D, Kc).bytes;
}

extern "C" int ulm_norm_conv_bwd(const void *x, int x_dtype, const float *rstd, const float *norm_w,
                                 const float *conv_w, int Kc, const void *du, int du_dtype, const void *dhv,
                                 int dhv_dtype, const float *dres, float *dx, float *dnorm_w, float *dconv_w,
                                 void *workspace, size_t workspace_bytes, int B, int T, int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && D > 0, "ulm_norm_conv_bwd: bad sizes B=%d T=%d D=%d", B, T, D);
    ULM_REQUIRE(Kc >= 1 && Kc <= blk::kMaxTaps, "ulm_norm_conv_bwd: Kc=%d outside 1..%d", Kc, blk::kMaxTaps);
    ULM_REQUIRE(blk::bwd_tile(D, Kc) > 0, "ulm_norm_conv_bwd: D=%d too large", D);
    ULM_REQUIRE(x_dtype_ok(x_dtype) && valid_dtype(du_dtype) && (!dhv || dhv_dtype == du_dtype),
                "ulm_norm_conv_bwd: bad dtypes x %d, du %d, dhv %d (du and dhv share one)", x_dtype, du_dtype,
                dhv_dtype);
    ULM_REQUIRE(x && rstd && norm_w && conv_w && du && dx && dnorm_w && dconv_w && workspace,
                "ulm_norm_conv_bwd: null pointer");
    const size_t need = ulm_norm_conv_bwd_workspace_bytes(B, T, D, Kc);
    ULM_REQUIRE(workspace_bytes >= need, "ulm_norm_conv_bwd: workspace of %zu bytes, need %zu", workspace_bytes, need);
    hipStream_t s = static_cast<hipStream_t>(stream);
    return blk::with_type(x_dtype, [&](auto tx) {
        return blk::with_type(du_dtype, [&](auto td) {
            return blk::launch_bwd<decltype(tx), decltype(td)>(x, rstd, norm_w, conv_w, Kc, du, dhv, dres, dx,
                                                              dnorm_w, dconv_w, workspace, B, T, D, s);
        });
    });
}

extern "C" int ulm_block_params(const float *log_rate, const float *log_w, float log_w_min, float log_w_max, int A,
                                float *g, float *w, void *stream) {
    ULM_REQUIRE(A > 0, "ulm_block_params: bad size A=%d", A);
    ULM_REQUIRE(log_rate && log_w && g && w, "ulm_block_params: null pointer");
    ULM_REQUIRE(log_w_min <= log_w_max, "ulm_block_params: empty clamp range [%g, %g]", log_w_min, log_w_max);
    blk::params_fwd_kernel<<<(A + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(log_rate, log_w, log_w_min,
                                                                                           log_w_max, A, g, w);
    return check_launch("params_fwd_kernel");
}

extern "C" int ulm_block_params_bwd(const float *log_rate, const float *log_w, float log_w_min, float log_w_max,
                                    const float *dg, const float *dw, int A, float *dlog_rate, float *dlog_w,
                                    void *stream) {
    ULM_REQUIRE(A > 0, "ulm_block_params_bwd: bad size A=%d", A);
    ULM_REQUIRE(log_rate && log_w && dg && dw && dlog_rate && dlog_w, "ulm_block_params_bwd: null pointer");
    ULM_REQUIRE(log_w_min <= log_w_max, "ulm_block_params_bwd: empty clamp range [%g, %g]", log_w_min, log_w_max);
    blk::params_bwd_kernel<<<(A + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(
        log_rate, log_w, log_w_min, log_w_max, dg, dw, A, dlog_rate, dlog_w);
    return check_launch("params_bwd_kernel");
}

extern "C" int ulm_cast(const void *src, int src_dtype, void *dst, int dst_dtype, size_t n, void *stream) {
    ULM_REQUIRE(valid_dtype(src_dtype) && valid_dtype(dst_dtype), "ulm_cast: bad dtype %d/%d", src_dtype, dst_dtype);
    ULM_REQUIRE(n == 0 || (src && dst), "ulm_cast: null pointer");
    return launch_convert(src, src_dtype, dst, dst_dtype, n, static_cast<hipStream_t>(stream));
}
