// Batched recurrent decode of one UnifiedBlock for N sequences and one position.
//
// Replaces UnifiedBlock.step (model.py:96-111) and its C mirror run.c:193-265.
// Per block and position the caller runs:
//   ulm_decode_pre   RMSNorm + causal depthwise conv window       (model.py:99-102)
//   pre = u K^T, v = h Wv^T                                        (library GEMMs)
//   ulm_decode_addr  relu^2 address, c update, q = r / c, w*q      (model.py:103-108)
//   ymu = (w*q) mu^T                                               (library GEMM)
//   ulm_decode_state S <- lam S + v r_prev^T, y = S q, out         (model.py:107-111)
//
// HBM layout: S is (N, D, A) fp32 with the slot index fastest, one row of A
// floats per (sequence, feature), like run.c's U[l][i][a] (run.c:38-41). The
// state kernel streams every row exactly once per token (read + write), which
// is the whole of the path's HBM traffic at large N: 8*A*D bytes per sequence.
#include "ulm_common.h"

namespace ulm {

// Sum over a 256-thread block; every thread gets the result.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
    v = wave_sum(v);
    int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void decode_pre_kernel(const float *__restrict__ x, const float *__restrict__ nw,
                                                         const float *__restrict__ cw, float *__restrict__ buf,
                                                         float *__restrict__ h, float *__restrict__ u, int D, int Kc,
                                                         float eps) {
    __shared__ float red[4];
    const size_t n = blockIdx.x;
    const float *xr = x + n * D;
    float ss = 0.f;
    for (int d = threadIdx.x; d < D; d += 256) ss += xr[d] * xr[d];
    ss = block_sum_256(ss, red);
    const float inv = rsqrtf(ss / static_cast<float>(D) + eps);
    const int kw = Kc - 1;
    for (int d = threadIdx.x; d < D; d += 256) {
        const float hd = (xr[d] * inv) * nw[d];
        float *st = buf + (n * D + d) * kw;
        const float *w = cw + static_cast<size_t>(d) * Kc;
        float ud = 0.f;
        for (int j = 0; j < kw; ++j) ud += w[j] * st[j];
        ud += w[kw] * hd;
        for (int j = 0; j + 1 < kw; ++j) st[j] = st[j + 1];
        if (kw > 0) st[kw - 1] = hd;
        h[n * D + d] = hd;
        u[n * D + d] = ud;
    }
}

__global__ __launch_bounds__(256) void decode_addr_kernel(const float *__restrict__ pre, const float *__restrict__ bias,
                                                          const float *__restrict__ log_eps, const float *__restrict__ w,
                                                          const float *__restrict__ g, const float *__restrict__ r_prev,
                                                          float *__restrict__ c, float *__restrict__ r,
                                                          float *__restrict__ q, float *__restrict__ wq, int A) {
    __shared__ float red[4];
    const size_t row = static_cast<size_t>(blockIdx.x) * A;
    float s = 0.f;
    for (int a = threadIdx.x; a < A; a += 256) {
        float p = pre[row + a] + (bias ? bias[a] : 0.f);
        p = p > 0.f ? p : 0.f;
        s += p * p;
    }
    s = block_sum_256(s, red);
    const float denom = __expf(fminf(fmaxf(log_eps[0], -10.f), 10.f)) + s;
    const float lam = __expf(g[0]);
    for (int a = threadIdx.x; a < A; a += 256) {
        float p = pre[row + a] + (bias ? bias[a] : 0.f);
        p = p > 0.f ? p : 0.f;
        const float ra = (p * p) / denom;
        const float cn = lam * c[row + a] + (1.f - lam) * w[a] + r_prev[row + a];
        const float qa = ra / cn;
        c[row + a] = cn;
        r[row + a] = ra;
        q[row + a] = qa;
        wq[row + a] = w[a] * qa;
    }
}

constexpr int kStateRows = 4;    // rows (features) per block, one per wave
constexpr int kMaxPending = 16;  // write terms a deferred state holds at most
constexpr int kRowChunk = 12;    // 16-byte loads per lane in flight per row: 3072 slots in one pass

// S[n, d, :] <- lam S + v[n, d] r_prev[n, :];  out[n, d] = x + S[n, d, :] . q[n, :] + ymu.
// q and r_prev of the block's sequence are staged once in LDS; each wave
// streams one whole row with 16-byte accesses, all of a pass's loads issued
// before any of its stores (kRowChunk per lane: at A = 3072 the row's 12 KB
// in flight at once), and reduces its dot product with cross-lane shuffles.
template <bool VEC4>
__global__ __launch_bounds__(256) void decode_state_kernel(float *__restrict__ S, const float *__restrict__ v,
                                                           const float *__restrict__ r_prev, const float *__restrict__ q,
                                                           const float *__restrict__ g, const float *__restrict__ x,
                                                           const float *__restrict__ ymu, float *__restrict__ out, int D,
                                                           int A) {
    extern __shared__ float smem[];
    float *sq = smem;
    float *srp = smem + A;
    const size_t n = blockIdx.x;
    for (int a = threadIdx.x; a < A; a += 256) {
        sq[a] = q[n * A + a];
        srp[a] = r_prev[n * A + a];
    }
    __syncthreads();
    const float lam = __expf(g[0]);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int d = blockIdx.y * kStateRows + wave;
    if (d >= D) return;
    float *Sr = S + (n * D + d) * static_cast<size_t>(A);
    const float vd = v[n * D + d];
    float acc = 0.f;
    if (VEC4) {
        // S is touched once per token: non-temporal 16-byte loads and stores
        // keep it from evicting the staged and reused data in the caches
        const int A4 = A / 4;
        f32x4 *S4 = reinterpret_cast<f32x4 *>(Sr);
        const f32x4 *q4 = reinterpret_cast<const f32x4 *>(sq);
        const f32x4 *p4 = reinterpret_cast<const f32x4 *>(srp);
        for (int base = 0; base < A4; base += kWave * kRowChunk) {
            f32x4 sv[kRowChunk];
#pragma unroll
            for (int k = 0; k < kRowChunk; ++k) {
                const int j = base + lane + kWave * k;
                sv[k] = j < A4 ? __builtin_nontemporal_load(S4 + j) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int k = 0; k < kRowChunk; ++k) {
                const int j = base + lane + kWave * k;
                if (j < A4) {
                    const f32x4 rp = p4[j], qq = q4[j];
                    const f32x4 s = lam * sv[k] + vd * rp;
                    __builtin_nontemporal_store(s, S4 + j);
                    acc += s[0] * qq[0] + s[1] * qq[1] + s[2] * qq[2] + s[3] * qq[3];
                }
            }
        }
    } else {
        for (int a = lane; a < A; a += kWave) {
            const float s = lam * Sr[a] + vd * srp[a];
            Sr[a] = s;
            acc += s * sq[a];
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) out[n * D + d] = x[n * D + d] + acc + ymu[n * D + d];
}

// decode_addr with 16-byte accesses, A % 4 == 0 and A <= 1024 R4: pre (+ bias)
// is read once and its relu^2 kept in registers across the row sum. With pr
// (a deferred state's pending keys, (mslot + 1, N, A) at least), r_prev is also
// appended as term mslot, and with cj the terms' read-out weights
// cj[j][n] = pr_j[n, :] . q[n, :], j = 0 .. mslot, are formed from the q in registers.
template <int R4>
__global__ __launch_bounds__(256) void decode_addr_vec_kernel(const float *__restrict__ pre, const float *__restrict__ bias,
                                                              const float *__restrict__ log_eps, const float *__restrict__ w,
                                                              const float *__restrict__ g, const float *__restrict__ r_prev,
                                                              float *__restrict__ c, float *__restrict__ r,
                                                              float *__restrict__ q, float *__restrict__ wq, int A,
                                                              float *__restrict__ pr = nullptr, int mslot = 0,
                                                              float *__restrict__ cj = nullptr, int N = 0) {
    __shared__ float red[4];
    const size_t row = static_cast<size_t>(blockIdx.x) * A;
    const int A4 = A / 4;
    const f32x4 *p4 = reinterpret_cast<const f32x4 *>(pre + row);
    const f32x4 *b4 = reinterpret_cast<const f32x4 *>(bias);
    // every load unconditional at a clamped index and selected after, so that
    // a loop's loads are in flight together (a load under a condition is
    // waited for before the condition ends)
    f32x4 z[R4], bz[R4];
#pragma unroll
    for (int k = 0; k < R4; ++k) {
        const int j = threadIdx.x + 256 * k, jc = j < A4 ? j : 0;
        z[k] = p4[jc];
        bz[k] = bias ? b4[jc] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < R4; ++k) {
        const bool ok = threadIdx.x + 256 * k < A4;
        f32x4 p = z[k] + bz[k];
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = ok && p[e] > 0.f ? p[e] * p[e] : 0.f;
        z[k] = p;
        s += (p[0] + p[1]) + (p[2] + p[3]);
    }
    s = block_sum_256(s, red);
    const float idn = 1.f / (__expf(fminf(fmaxf(log_eps[0], -10.f), 10.f)) + s);
    const float lam = __expf(g[0]);
    const f32x4 *w4 = reinterpret_cast<const f32x4 *>(w);
    const f32x4 *rp4 = reinterpret_cast<const f32x4 *>(r_prev + row);
    f32x4 *c4 = reinterpret_cast<f32x4 *>(c + row);
    f32x4 qk[R4], wv[R4], rpv[R4], cv[R4];
#pragma unroll
    for (int k = 0; k < R4; ++k) {
        const int j = threadIdx.x + 256 * k, jc = j < A4 ? j : 0;
        wv[k] = w4[jc];
        rpv[k] = rp4[jc];
        cv[k] = c4[jc];
    }
#pragma unroll
    for (int k = 0; k < R4; ++k) {
        const int j = threadIdx.x + 256 * k;
        qk[k] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (j >= A4) continue;
        const f32x4 wa = wv[k], rp = rpv[k], cn = lam * cv[k] + (1.f - lam) * wa + rp;
        const f32x4 ra = z[k] * idn;
        f32x4 qa;
#pragma unroll
        for (int e = 0; e < 4; ++e) qa[e] = ra[e] / cn[e];
        c4[j] = cn;
        reinterpret_cast<f32x4 *>(r + row)[j] = ra;
        reinterpret_cast<f32x4 *>(q + row)[j] = qa;
        reinterpret_cast<f32x4 *>(wq + row)[j] = wa * qa;
        if (pr) reinterpret_cast<f32x4 *>(pr + static_cast<size_t>(mslot) * N * A + row)[j] = rp;
        qk[k] = qa;
    }
    if (!cj) return;
    // the pending terms' weights pr_t . q, t = 0 .. mslot: each thread's partial
    // dots of every term, then one exchange for all of them. The term just
    // appended is read back from the store above by the same lanes, so it
    // needs no barrier.
    __shared__ float part[4][kMaxPending];
    const size_t n = blockIdx.x;
    float dt[kMaxPending];
#pragma unroll
    for (int t = 0; t < kMaxPending; ++t) dt[t] = 0.f;
    // terms in groups of 4, each group's loads unconditional (terms past the
    // slot clamped to it and selected away), so a group's loads are in flight
    // together; the groups past the slot are skipped
#pragma unroll
    for (int t0 = 0; t0 < kMaxPending; t0 += 4) {
        if (t0 > mslot) break;
        f32x4 pk[4][R4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int t = min(t0 + u, mslot);
            const f32x4 *p4 = reinterpret_cast<const f32x4 *>(pr + static_cast<size_t>(t) * N * A + row);
#pragma unroll
            for (int k = 0; k < R4; ++k) {
                const int j = threadIdx.x + 256 * k;
                pk[u][k] = p4[j < A4 ? j : 0];   // clamped load; selected away past A
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int k = 0; k < R4; ++k) {
                const f32x4 v = pk[u][k] * qk[k];
                const bool ok = threadIdx.x + 256 * k < A4 && t0 + u <= mslot;
                dt[t0 + u] += ok ? (v[0] + v[1]) + (v[2] + v[3]) : 0.f;
            }
    }
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
#pragma unroll
    for (int t = 0; t < kMaxPending; ++t) {
        if (t > mslot) break;
        const float v = wave_sum(dt[t]);
        if (lane == 0) part[wave][t] = v;
    }
    __syncthreads();
    if (threadIdx.x <= mslot)
        cj[static_cast<size_t>(threadIdx.x) * N + n] =
            (part[0][threadIdx.x] + part[1][threadIdx.x]) + (part[2][threadIdx.x] + part[3][threadIdx.x]);
}

// ---- Deferred state write-back. The state is kept as S_base plus the m most
// recent write terms (v_j, rp_j), j = 0 (oldest) .. m - 1, of m <= J pending
// positions:
//   S_t = lam^m S_base + sum_j lam^(m-1-j) v_j rp_j^T,
//   y_t = S_t q = lam^m (S_base q) + sum_j lam^(m-1-j) v_j (rp_j . q).
// A position with m < J only reads S_base (decode_read_kernel); the position
// that fills the J-th term writes S_t back as the new S_base (decode_flush_kernel).
// Per J positions the state moves J reads and one write instead of J of each.

// cj[j][n] = rp_j[n, :] . q[n, :] for the m pending terms; one block per sequence
__global__ __launch_bounds__(256) void decode_dots_kernel(const float *__restrict__ pr, const float *__restrict__ q,
                                                          float *__restrict__ cj, int m, int N, int A) {
    __shared__ float red[4];
    const size_t n = blockIdx.x;
    for (int j = 0; j < m; ++j) {
        const float *p = pr + (static_cast<size_t>(j) * N + n) * A;
        float s = 0.f;
        for (int a = threadIdx.x; a < A; a += 256) s += p[a] * q[n * A + a];
        s = block_sum_256(s, red);
        if (threadIdx.x == 0) cj[static_cast<size_t>(j) * N + n] = s;
    }
}

constexpr int kReadRowsPerWave = 4;

// Read-only position: out[n, d] = x + lam^m (S_base[n, d, :] . q) + sum_j lam^(m-1-j)
// pv_j[n, d] cj[j][n] + ymu. Each lane keeps its CH 16-byte slices of q in
// registers for all of its wave's rows and streams each row with all of the
// row's loads in flight (A % 4 == 0, A <= 256 CH).
template <int CH>
__global__ __launch_bounds__(256) void decode_read_kernel(const float *__restrict__ S, const float *__restrict__ pv,
                                                          const float *__restrict__ cj, int m,
                                                          const float *__restrict__ q, const float *__restrict__ g,
                                                          const float *__restrict__ x, const float *__restrict__ ymu,
                                                          float *__restrict__ out, int N, int D, int A) {
    const size_t n = blockIdx.x;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int A4 = A / 4;
    const f32x4 *q4 = reinterpret_cast<const f32x4 *>(q + n * A);
    f32x4 qv[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const int j = lane + kWave * k;
        qv[k] = j < A4 ? q4[j] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float lam = __expf(g[0]);
    float lm = 1.f;
    for (int j = 0; j < m; ++j) lm *= lam;
    // lane j < m carries term j: its weight lam^(m-1-j) cj[j][n]; the term's
    // v_j[n, d] joins the row's wave sum
    const int jt = lane < m ? lane : 0;
    float cw = cj[static_cast<size_t>(jt) * N + n];
    for (int e = jt + 1; e < m; ++e) cw *= lam;
    cw = lane < m ? cw : 0.f;
    const int d0 = (blockIdx.y * 4 + wave) * kReadRowsPerWave;
    for (int r = 0; r < kReadRowsPerWave; ++r) {
        const int d = d0 + r;
        if (d >= D) break;
        const f32x4 *S4 = reinterpret_cast<const f32x4 *>(S + (n * D + d) * static_cast<size_t>(A));
        f32x4 sv[CH];
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int j = lane + kWave * k;
            sv[k] = __builtin_nontemporal_load(S4 + (j < A4 ? j : 0));
        }
        const float pvl = pv[(static_cast<size_t>(jt) * N + n) * D + d];
        // the row's loads all go out before its arithmetic (interleaved by the
        // scheduler, each load waited for the one before it)
        __builtin_amdgcn_sched_barrier(0);
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const f32x4 t = sv[k] * qv[k];   // q is zero past A
            acc += (t[0] + t[1]) + (t[2] + t[3]);
        }
        acc = wave_sum(lm * acc + cw * pvl);
        if (lane == 0) out[n * D + d] = x[n * D + d] + acc + ymu[n * D + d];
    }
}

constexpr int kFlushRows = 64;   // rows (features) per workgroup
// rows whose loads a lane has in flight at once: 8 where the registers allow
// (12 waves, 168 VGPRs), else 4
template <int MAXW> constexpr int flush_batch() { return MAXW <= 12 ? 8 : 4; }

// Flush position: S_base[n, d, :] <- lam^m S_base + sum_j lam^(m-1-j) pv_j[n, d] rp_j[n, :],
// out[n, d] = x + S_base . q + ymu. Column-strip layout: wave w of the
// workgroup owns slots 256 w .. 256 w + 255 (one 16-byte slice per lane) of
// kFlushRows rows of one sequence, and keeps its slices of the m pending keys
// and of q in registers for all of them; the per-row coefficients
// lam^(m-1-j) pv_j[n, d] are uniform over the wave. Each lane streams its
// slice of a batch of rows at a time (loads first), and the rows' dot
// products are summed over the waves through LDS in a fixed order.
// A <= 64 MAXW (MAXW waves at most), A % 4 == 0; MAXW = 12 (A <= 3072) allows
// 168 VGPRs per lane, where the 16 key slices fit without spills.
template <int MAXW>
__global__ __launch_bounds__(MAXW * 64) void decode_flush_kernel(float *__restrict__ S, const float *__restrict__ pv,
                                                            const float *__restrict__ pr, int m,
                                                            const float *__restrict__ q, const float *__restrict__ g,
                                                            const float *__restrict__ x, const float *__restrict__ ymu,
                                                            float *__restrict__ out, int N, int D, int A) {
    __shared__ float part[16][kFlushRows];
    __shared__ float spv[kMaxPending][kFlushRows];   // the block's rows' pending values
    const size_t n = blockIdx.x;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, nw = blockDim.x / kWave;
    const int d0 = blockIdx.y * kFlushRows;
    for (int k = threadIdx.x; k < kMaxPending * kFlushRows; k += blockDim.x) {
        const int j = k / kFlushRows, d = min(d0 + k % kFlushRows, D - 1);
        spv[j][k % kFlushRows] = j < m ? pv[(static_cast<size_t>(j) * N + n) * D + d] : 0.f;
    }
    const int A4 = A / 4, i = wave * kWave + lane;   // this lane's 16-byte slice of every row
    const bool ok = i < A4;
    const int ic = ok ? i : 0;
    f32x4 rp[kMaxPending];
#pragma unroll
    for (int j = 0; j < kMaxPending; ++j)
        rp[j] = reinterpret_cast<const f32x4 *>(pr + (static_cast<size_t>(j < m ? j : 0) * N + n) * A)[ic];
    const f32x4 qv = reinterpret_cast<const f32x4 *>(q + n * A)[ic];
    const float lam = __expf(g[0]);
    float lm = 1.f;
    for (int j = 0; j < m; ++j) lm *= lam;
    __syncthreads();
    for (int b = 0; b < kFlushRows; b += flush_batch<MAXW>()) {
        f32x4 sv[flush_batch<MAXW>()];
#pragma unroll
        for (int u = 0; u < flush_batch<MAXW>(); ++u) {
            const int d = min(d0 + b + u, D - 1);   // rows past D: a clamped load, nothing stored
            sv[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(S + (n * D + d) * static_cast<size_t>(A)) + ic);
        }
        __builtin_amdgcn_sched_barrier(0);   // the batch's loads before its arithmetic
#pragma unroll
        for (int u = 0; u < flush_batch<MAXW>(); ++u) {
            const int d = d0 + b + u;
            float cf[kMaxPending];
            float pw = 1.f;
#pragma unroll
            for (int j = kMaxPending - 1; j >= 0; --j) {
                cf[j] = j < m ? pw * spv[j][b + u] : 0.f;
                if (j < m) pw *= lam;
            }
            f32x4 t = lm * sv[u];
#pragma unroll
            for (int j = 0; j < kMaxPending; ++j) t += cf[j] * rp[j];
            if (ok && d < D)
                __builtin_nontemporal_store(t, reinterpret_cast<f32x4 *>(S + (n * D + d) * static_cast<size_t>(A)) + i);
            const f32x4 pq = t * qv;
            float acc = ok ? (pq[0] + pq[1]) + (pq[2] + pq[3]) : 0.f;
            acc = wave_sum(acc);
            if (lane == 0) part[wave][b + u] = acc;
        }
    }
    __syncthreads();
    if (threadIdx.x < kFlushRows) {
        const int d = d0 + threadIdx.x;
        if (d < D) {
            float y = 0.f;
            for (int w2 = 0; w2 < nw; ++w2) y += part[w2][threadIdx.x];
            out[n * D + d] = x[n * D + d] + y + ymu[n * D + d];
        }
    }
}

}  // namespace ulm

using namespace ulm;

extern "C" int ulm_decode_pre(const float *x, const float *norm_w, const float *conv_w, float *conv_buf, float *h,
                              float *u, int N, int D, int Kc, float norm_eps, void *stream) {
    ULM_REQUIRE(N > 0 && D > 0 && Kc >= 1, "ulm_decode_pre: bad sizes N=%d D=%d Kc=%d", N, D, Kc);
    ULM_REQUIRE(x && norm_w && conv_w && h && u && (Kc == 1 || conv_buf), "ulm_decode_pre: null pointer");
    decode_pre_kernel<<<dim3(N), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(x, norm_w, conv_w, conv_buf, h, u,
                                                                                   D, Kc, norm_eps);
    return check_launch("decode_pre_kernel");
}

extern "C" int ulm_decode_addr(const float *pre, const float *bias, const float *log_eps, const float *w,
                               const float *g, const float *r_prev, float *c, float *r, float *q, float *wq, int N,
                               int A, void *stream) {
    ULM_REQUIRE(N > 0 && A > 0, "ulm_decode_addr: bad sizes N=%d A=%d", N, A);
    ULM_REQUIRE(pre && log_eps && w && g && r_prev && c && r && q && wq, "ulm_decode_addr: null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    bool aligned = A % 4 == 0;
    for (const void *t : {static_cast<const void *>(pre), static_cast<const void *>(bias), static_cast<const void *>(w),
                          static_cast<const void *>(r_prev), static_cast<const void *>(c), static_cast<const void *>(r),
                          static_cast<const void *>(q), static_cast<const void *>(wq)})
        aligned = aligned && reinterpret_cast<uintptr_t>(t) % 16 == 0;
    const int r4 = (A / 4 + 255) / 256;
    if (aligned && r4 <= 4) {
        switch (r4) {
        case 1: decode_addr_vec_kernel<1><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A); break;
        case 2: decode_addr_vec_kernel<2><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A); break;
        case 3: decode_addr_vec_kernel<3><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A); break;
        default: decode_addr_vec_kernel<4><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A); break;
        }
        return check_launch("decode_addr_vec_kernel");
    }
    decode_addr_kernel<<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A);
    return check_launch("decode_addr_kernel");
}

extern "C" int ulm_decode_state(float *S, const float *v, const float *r_prev, const float *q, const float *g,
                                const float *x, const float *ymu, float *out, int N, int D, int A, void *stream) {
    ULM_REQUIRE(N > 0 && D > 0 && A > 0, "ulm_decode_state: bad sizes N=%d D=%d A=%d", N, D, A);
    ULM_REQUIRE(A <= 8192, "ulm_decode_state: A=%d exceeds the LDS staging limit 8192", A);
    ULM_REQUIRE(S && v && r_prev && q && g && x && ymu && out, "ulm_decode_state: null pointer");
    const dim3 grid(N, (D + kStateRows - 1) / kStateRows);
    const size_t lds = 2 * static_cast<size_t>(A) * sizeof(float);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = (A % 4 == 0) && (reinterpret_cast<uintptr_t>(S) % 16 == 0);
    if (vec)
        decode_state_kernel<true><<<grid, dim3(256), lds, s>>>(S, v, r_prev, q, g, x, ymu, out, D, A);
    else
        decode_state_kernel<false><<<grid, dim3(256), lds, s>>>(S, v, r_prev, q, g, x, ymu, out, D, A);
    return check_launch("decode_state_kernel");
}

namespace {
// the per-lane 16-byte slice count of a row of A slots: 4, 8, 12 or 16 (A <= 4096), else 0
int deferred_chunks(int A) {
    const int ch = (A / 4 + kWave - 1) / kWave;
    return ch <= 4 ? 4 : ch <= 8 ? 8 : ch <= 12 ? 12 : ch <= 16 ? 16 : 0;
}
bool aligned16(std::initializer_list<const void *> ps) {
    for (const void *p : ps)
        if (reinterpret_cast<uintptr_t>(p) % 16) return false;
    return true;
}
}  // namespace

extern "C" int ulm_decode_max_pending(void) { return kMaxPending; }

extern "C" int ulm_decode_dots(const float *pr, const float *q, float *cj, int m, int N, int A, void *stream) {
    ULM_REQUIRE(N > 0 && A > 0 && m >= 1 && m <= kMaxPending, "ulm_decode_dots: bad sizes N=%d A=%d m=%d", N, A, m);
    ULM_REQUIRE(pr && q && cj, "ulm_decode_dots: null pointer");
    decode_dots_kernel<<<dim3(N), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(pr, q, cj, m, N, A);
    return check_launch("decode_dots_kernel");
}

extern "C" int ulm_decode_read(const float *S, const float *pv, const float *cj, int m, const float *q, const float *g,
                               const float *x, const float *ymu, float *out, int N, int D, int A, void *stream) {
    ULM_REQUIRE(N > 0 && D > 0 && A > 0 && m >= 1 && m <= kMaxPending, "ulm_decode_read: bad sizes N=%d D=%d A=%d m=%d",
                N, D, A, m);
    ULM_REQUIRE(A % 4 == 0 && deferred_chunks(A) > 0, "ulm_decode_read: A=%d must be a multiple of 4 and at most 4096",
                A);
    ULM_REQUIRE(S && pv && cj && q && g && x && ymu && out, "ulm_decode_read: null pointer");
    ULM_REQUIRE(aligned16({S, q}), "ulm_decode_read: S and q must be 16-byte aligned");
    const dim3 grid(N, (D + 4 * kReadRowsPerWave - 1) / (4 * kReadRowsPerWave));
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (deferred_chunks(A)) {
    case 4: decode_read_kernel<4><<<grid, dim3(256), 0, s>>>(S, pv, cj, m, q, g, x, ymu, out, N, D, A); break;
    case 8: decode_read_kernel<8><<<grid, dim3(256), 0, s>>>(S, pv, cj, m, q, g, x, ymu, out, N, D, A); break;
    case 12: decode_read_kernel<12><<<grid, dim3(256), 0, s>>>(S, pv, cj, m, q, g, x, ymu, out, N, D, A); break;
    default: decode_read_kernel<16><<<grid, dim3(256), 0, s>>>(S, pv, cj, m, q, g, x, ymu, out, N, D, A); break;
    }
    return check_launch("decode_read_kernel");
}

extern "C" int ulm_decode_flush(float *S, const float *pv, const float *pr, int m, const float *q, const float *g,
                                const float *x, const float *ymu, float *out, int N, int D, int A, void *stream) {
    ULM_REQUIRE(N > 0 && D > 0 && A > 0 && m >= 1 && m <= kMaxPending,
                "ulm_decode_flush: bad sizes N=%d D=%d A=%d m=%d", N, D, A, m);
    ULM_REQUIRE(A % 4 == 0 && deferred_chunks(A) > 0, "ulm_decode_flush: A=%d must be a multiple of 4 and at most 4096",
                A);
    ULM_REQUIRE(S && pv && pr && q && g && x && ymu && out, "ulm_decode_flush: null pointer");
    ULM_REQUIRE(aligned16({S, q, pr}), "ulm_decode_flush: S, q and the pending keys must be 16-byte aligned");
    const int waves = (A / 4 + kWave - 1) / kWave;   // one 256-slot strip per wave
    const dim3 grid(N, (D + kFlushRows - 1) / kFlushRows);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (waves <= 12)
        decode_flush_kernel<12><<<grid, dim3(waves * kWave), 0, s>>>(S, pv, pr, m, q, g, x, ymu, out, N, D, A);
    else
        decode_flush_kernel<16><<<grid, dim3(waves * kWave), 0, s>>>(S, pv, pr, m, q, g, x, ymu, out, N, D, A);
    return check_launch("decode_flush_kernel");
}

extern "C" int ulm_decode_addr_deferred(const float *pre, const float *bias, const float *log_eps, const float *w,
                                        const float *g, const float *r_prev, float *c, float *r, float *q, float *wq,
                                        float *pr, int mslot, float *cj, int N, int A, void *stream) {
    ULM_REQUIRE(N > 0 && A > 0 && mslot >= 0 && mslot < kMaxPending,
                "ulm_decode_addr_deferred: bad sizes N=%d A=%d slot=%d", N, A, mslot);
    ULM_REQUIRE(pre && log_eps && w && g && r_prev && c && r && q && wq && pr, "ulm_decode_addr_deferred: null pointer");
    const int r4 = (A / 4 + 255) / 256;
    ULM_REQUIRE(A % 4 == 0 && r4 <= 4, "ulm_decode_addr_deferred: A=%d must be a multiple of 4 and at most 4096", A);
    ULM_REQUIRE(aligned16({pre, bias, w, r_prev, c, r, q, wq, pr}),
                "ulm_decode_addr_deferred: every vector must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (r4) {
    case 1: decode_addr_vec_kernel<1><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A, pr, mslot, cj, N); break;
    case 2: decode_addr_vec_kernel<2><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A, pr, mslot, cj, N); break;
    case 3: decode_addr_vec_kernel<3><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A, pr, mslot, cj, N); break;
    default: decode_addr_vec_kernel<4><<<dim3(N), dim3(256), 0, s>>>(pre, bias, log_eps, w, g, r_prev, c, r, q, wq, A, pr, mslot, cj, N); break;
    }
    return check_launch("decode_addr_vec_kernel");
}
