// Per-slot statistics of the fast memory: the decayed evidence scan and its
// backward. Replaces _fwd_stats_kernel / _bwd_stats_kernel (kernel.py:104-180).
//
// Forward, per batch row and slot a:
//   k_t = r_{t-1} (k_0 = 0),  n_t = lam n_{t-1} + k_t,  c_t = w_a + n_t,  q_t = r_t / c_t
// Backward (kernel.py:142-178), walking time in reverse:
//   dq = dq_f + dq_out, dr_t = dq_t / c_t + dkt_{t+1}, dc = -dq q / c,
//   dkc_t = dc_t + lam dkc_{t+1}, dkt = dk_f + dkc, dw = sum_t dc,
//   dg = sum_t (t - tau) [q dq_f + dc (c - w) - k dk_f - k dkc]_t   (any tau; tau = (T-1)/2)
//   with the bf16 copies of q and k in the dq_f and dk_f terms (the values the
//   chunked products used), so the pair terms cancel exactly between the sums.
// The block's read-out x + mu(w q) (model.py:85) is served by two options: the
// forward can write w q in the GEMM's dtype instead of q, and the backward can
// take d(w q) for dq_out, adding w d(w q) to dq and sum_t q d(w q) to dw.
//
// Thread layout: a 256-thread block owns 64 slots of one batch row; thread
// (slot s, segment j) holds 16 consecutive positions of each 64-position chunk,
// so every global access is a 256-byte row segment. A chunk is scanned in
// registers per segment and the four segments are joined through LDS
// (carry_j = lam^16 carry_{j-1} + total_{j-1}). Instead of the full c tensor
// the forward saves n at every chunk start (B x ceil(T/64) x A); the backward
// rebuilds c inside each chunk from it.
#include "ulm_common.h"

namespace ulm {

constexpr int kSeg = 16;      // positions per thread segment
constexpr int kSlots = 64;    // slots per block

__device__ __forceinline__ float pow_int(float x, int e) {
    float r = 1.f;
    for (int i = 0; i < e; ++i) r *= x;
    return r;
}

// Sources of r for the kernels below (RSrc). raw(row, ac, A) loads the stored
// element of row `row` (wave-uniform, clamped by the caller to a valid row) at
// slot `ac` (clamped per lane); make() turns it into r with the slot and
// position constants and the validity mask. Keeping the two apart lets a kernel
// issue a chunk's loads ahead of the arithmetic that waits on them; at() does
// both. Loads are unconditional and masked after, so none waits in a branch.
struct RTensor {
    const float *r;
    using raw_t = float;
    __device__ __forceinline__ float slot_const(int) const { return 0.f; }
    static constexpr bool kRowConst = false;
    __device__ __forceinline__ float row_raw(size_t, bool) const { return 1.f; }
    __device__ __forceinline__ raw_t raw(size_t row, uint32_t ac, int A) const { return ld_row(r + row * A, 4u * ac); }
    __device__ __forceinline__ float make(raw_t v, float, float, bool ok) const { return ok ? v : 0.f; }
    __device__ __forceinline__ float at(size_t row, uint32_t ac, int A, float b, float inv, bool ok) const {
        return make(raw(row, ac, A), b, inv, ok);
    }
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(uint16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }

// r = relu(pre + bias)^2 * (1 / denom[row]); addr_bwd_kernel forms r with the
// same operations, so every kernel of the block sees the same r. The
// reciprocal depends on the position only, which is uniform over a wave (its
// lanes are 64 slots), so it is formed once per position from row_raw.
template <typename TP>
struct RAddr {
    const TP *pre;
    const float *bias, *denom;
    using raw_t = TP;
    __device__ __forceinline__ float slot_const(int a) const { return bias ? bias[a] : 0.f; }
    static constexpr bool kRowConst = true;
    __device__ __forceinline__ float row_raw(size_t row, bool tok) const { return denom[tok ? row : 0]; }
    __device__ __forceinline__ raw_t raw(size_t row, uint32_t ac, int A) const {
        return ld_row(pre + row * A, static_cast<uint32_t>(sizeof(TP)) * ac);
    }
    __device__ __forceinline__ float make(raw_t v, float b, float inv, bool ok) const {
        float p = to_f32(v) + b;
        p = p > 0.f ? p : 0.f;
        const float r = (p * p) * inv;
        return ok ? r : 0.f;
    }
    __device__ __forceinline__ float at(size_t row, uint32_t ac, int A, float b, float inv, bool ok) const {
        return make(raw(row, ac, A), b, inv, ok);
    }
};

// The per-position constants of a thread segment (positions t0 .. t0+15 and
// t0 - 1): lane l < 16 loads position t0 + l, lane 16 position t0 - 1, and
// v_readlane hands each value to the whole wave. seg_row_raw loads the
// denominators, seg_inv turns them into the factors make() takes.
template <class RS>
__device__ __forceinline__ float seg_row_raw(const RS &rs, size_t row_t0, int t0, int T, int lane) {
    if constexpr (RS::kRowConst) {
        const int tl = lane < kSeg ? t0 + lane : t0 - 1;
        return rs.row_raw(row_t0 + (tl - t0), tl >= 0 && tl < T);
    } else {
        return 1.f;
    }
}

template <class RS> __device__ __forceinline__ float seg_inv(float d) {
    if constexpr (RS::kRowConst) return 1.f / d;
    else return 1.f;
}

__device__ __forceinline__ float lane_value(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Row b T + t of a (B, T, ...) tensor when 0 <= t < T, else row 0: the clamp
// depends on wave-uniform values only, so the row stays in scalar registers.
__device__ __forceinline__ size_t urow(size_t b, int t, int T) { return (t >= 0 && t < T) ? b * T + t : 0; }

// Calls f(source) with the RTensor or RAddr<T> that src describes.
template <class F>
int with_rsrc(const RSrc &src, F &&f) {
    if (src.r) return f(RTensor{src.r});
    if (!src.pre || !src.denom) return fail(ULM_ERR_INVALID, "stats: neither r nor the address inputs given");
    switch (src.pre_dt) {
    case ULM_F32: return f(RAddr<float>{static_cast<const float *>(src.pre), src.bias, src.denom});
    case ULM_BF16: return f(RAddr<uint16_t>{static_cast<const uint16_t *>(src.pre), src.bias, src.denom});
    case ULM_F16: return f(RAddr<_Float16>{static_cast<const _Float16 *>(src.pre), src.bias, src.denom});
    }
    return fail(ULM_ERR_INVALID, "stats: bad pre dtype %d", src.pre_dt);
}

// Outputs besides n_ckpt (each may be null): q (fp32); qw = w q in qw_dt; q16n, k16n natural bf16
// copies; qR, kR in the R layout and qQ, kQ in the Q layout (the products'
// operand tiles, AL slots wide: AL % 32 == 0, A <= AL <= the grid's slots);
// c_last = c at position T-1 (B, A), the decode state after the sequence.
// Positions past T and slots past A are zero in R and Q.
// QW: the dtype of the w q output (-1 none, else a ulm_dtype); HAS_Q: the fp32 q output.
template <class RS, int QW, bool HAS_Q>
__global__ __launch_bounds__(256) void fwd_stats_kernel(RS rs, const float *__restrict__ w,
                                                        const float *__restrict__ g, float *__restrict__ q,
                                                        void *__restrict__ qw, int qw_dt,
                                                        uint16_t *__restrict__ q16n, uint16_t *__restrict__ k16n,
                                                        uint16_t *__restrict__ qR, uint16_t *__restrict__ kR,
                                                        uint16_t *__restrict__ qQ, uint16_t *__restrict__ kQ,
                                                        float *__restrict__ nck, float *__restrict__ c_last, int T,
                                                        int A, int AL, int NT) {
    __shared__ float tot[4][kSlots];
    __shared__ __align__(16) uint16_t sq[ULM_CHUNK][kSlots + 8], sk[ULM_CHUNK][kSlots + 8];   // [position][slot]
    const int s = threadIdx.x % kSlots;
    const int j = __builtin_amdgcn_readfirstlane(threadIdx.x / kSlots);   // wave-uniform (kSlots = wave size)
    const int a0 = blockIdx.x * kSlots;
    const int a = a0 + s;
    const bool va = a < A;
    const uint32_t ac = va ? a : 0;   // the lane's slot, clamped for loads
    const int b = blockIdx.y;
    const size_t bs = blockIdx.y;
    const float lam = __expf(g[0]);
    const float lam16 = pow_int(lam, kSeg);
    const float wa = va ? w[a] : 1.f;
    const float rb = va ? rs.slot_const(a) : 0.f;   // the slot's key bias when r is formed here
    float carry = 0.f;   // n at the position before the chunk
    // the stored elements of a chunk's positions t0 .. t0+15 and t0 - 1, and
    // their denominators, loaded two chunks ahead into alternating buffers
    typename RS::raw_t pv[2][kSeg + 1];
    float pd[2];
    auto fetch = [&](int n, int u) {
        const int t0 = n * ULM_CHUNK + j * kSeg;
        pd[u] = seg_row_raw(rs, bs * T + t0, t0, T, s);
#pragma unroll
        for (int i = 0; i < kSeg; ++i) pv[u][i] = rs.raw(urow(bs, t0 + i, T), ac, A);
        pv[u][kSeg] = rs.raw(urow(bs, t0 - 1, T), ac, A);
    };
    fetch(0, 0);
    if (NT > 1) fetch(1, 1);
    auto chunk = [&](int n, int u) {
        const int t0 = n * ULM_CHUNK + j * kSeg;
        const float seg_c = seg_inv<RS>(pd[u]);
        float rv[kSeg], kv[kSeg], nl[kSeg];
#pragma unroll
        for (int i = 0; i < kSeg; ++i) rv[i] = rs.make(pv[u][i], rb, lane_value(seg_c, i), va && t0 + i < T);
        kv[0] = rs.make(pv[u][kSeg], rb, lane_value(seg_c, kSeg), va && t0 >= 1 && t0 - 1 < T);
        if (n + 2 < NT) fetch(n + 2, u);
#pragma unroll
        for (int i = 1; i < kSeg; ++i) kv[i] = rv[i - 1];
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
            acc = lam * acc + kv[i];
            nl[i] = acc;
        }
        tot[j][s] = acc;
        __syncthreads();
        float cj = carry;
        for (int m = 0; m < j; ++m) cj = lam16 * cj + tot[m][s];
        float pw = lam;
        uint32_t qpk[kSeg / 2], kpk[kSeg / 2];   // bf16 pairs of this thread's 16 positions
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
            const int t = t0 + i;
            const float ct = wa + (pw * cj + nl[i]);
            pw *= lam;
            uint16_t qb = 0, kb = 0;   // positions past T are zero in the tiled copies
            if (va && t < T) {
                const size_t ro = (bs * T + t) * A;   // wave-uniform row offset
                const float qt = rv[i] / ct;
                if (c_last && t == T - 1) c_last[bs * A + a] = ct;
                qb = f32_to_bf16_bits(qt);
                kb = f32_to_bf16_bits(kv[i]);
                if constexpr (HAS_Q) st_row(q + ro, 4u * ac, qt);
                if constexpr (QW == ULM_F32) st_row(static_cast<float *>(qw) + ro, 4u * ac, qt * wa);
                if constexpr (QW == ULM_BF16) st_row(static_cast<uint16_t *>(qw) + ro, 2u * ac, f32_to_bf16_bits(qt * wa));
                if constexpr (QW == ULM_F16) st_row(static_cast<_Float16 *>(qw) + ro, 2u * ac, static_cast<_Float16>(qt * wa));
                if (q16n) {
                    st_row(q16n + ro, 2u * ac, qb);
                    st_row(k16n + ro, 2u * ac, kb);
                }
            }
            sq[j * kSeg + i][s] = qb;
            sk[j * kSeg + i][s] = kb;
            if (i % 2 == 0) {
                qpk[i / 2] = qb;
                kpk[i / 2] = kb;
            } else {
                qpk[i / 2] |= static_cast<uint32_t>(qb) << 16;
                kpk[i / 2] |= static_cast<uint32_t>(kb) << 16;
            }
        }
        if ((qQ || kQ) && a < AL) {
            // Q layout: this thread's positions 16 j .. 16 j + 15 of slot a are two lanes' 16 bytes
            // (qQ is null where no backward follows, as in a prefill)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const size_t o = q_index(b, n * ULM_CHUNK + kSeg * j + 8 * h, a, NT, AL);
                if (qQ) *reinterpret_cast<uint4 *>(qQ + o) = make_uint4(qpk[4 * h], qpk[4 * h + 1], qpk[4 * h + 2], qpk[4 * h + 3]);
                if (kQ) *reinterpret_cast<uint4 *>(kQ + o) = make_uint4(kpk[4 * h], kpk[4 * h + 1], kpk[4 * h + 2], kpk[4 * h + 3]);
            }
        }
        if (j == 0 && va) nck[(bs * NT + n) * A + a] = carry;
        float nc = carry;
        for (int m = 0; m < 4; ++m) nc = lam16 * nc + tot[m][s];
        carry = nc;
        __syncthreads();   // sq, sk complete; tot free for the next chunk
        if (qR) {
            // R layout: the block's 64 positions x 64 slots are 8 tiles; thread -> 2 lanes of one tile
            const int tl = threadIdx.x / 32, mt = tl / 4, tf4 = tl % 4;
            if (a0 + 16 * tf4 < AL) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int l = 2 * (threadIdx.x % 32) + u, row = 32 * mt + l % 32, col = 16 * tf4 + 8 * (l / 32);
                    const size_t o = r_index(b, n * ULM_CHUNK + row, a0 + col, NT, AL);
                    *reinterpret_cast<uint4 *>(qR + o) = *reinterpret_cast<const uint4 *>(&sq[row][col]);
                    *reinterpret_cast<uint4 *>(kR + o) = *reinterpret_cast<const uint4 *>(&sk[row][col]);
                }
            }
        }
        __syncthreads();   // sq, sk read before the next chunk writes them
    };
    for (int n = 0; n < NT; n += 2) {
        chunk(n, 0);
        if (n + 1 < NT) chunk(n + 1, 1);
    }
}

// The extra gradient of q, by template so that every load is a plain one:
// XQ = 0 none, 1 dq_out fp32, 2/3/4 d(w q) as fp32/bf16/fp16.
template <int XQ>
__device__ __forceinline__ float load_xq(const void *p, size_t ro, uint32_t ac) {
    if constexpr (XQ == 1 || XQ == 2) return ld_row(static_cast<const float *>(p) + ro, 4u * ac);
    else if constexpr (XQ == 3) return bf16_to_f32(ld_row(static_cast<const uint16_t *>(p) + ro, 2u * ac));
    else if constexpr (XQ == 4) return static_cast<float>(ld_row(static_cast<const _Float16 *>(p) + ro, 2u * ac));
    else return 0.f;
}

template <int XQ, class RS>
__global__ __launch_bounds__(256) void bwd_stats_kernel(const float *__restrict__ dqf, const void *__restrict__ xq,
                                                        RS rs,
                                                        const float *__restrict__ nck, const float *__restrict__ w,
                                                        const float *__restrict__ g, const float *__restrict__ dkf,
                                                        float *__restrict__ dr, float *__restrict__ dw_part,
                                                        double *__restrict__ dg_part, int T, int A, int NT,
                                                        int fast_dg) {
    __shared__ float tot[4][kSlots];
    __shared__ float first_dkt[4][kSlots];
    __shared__ float dw_sh[4][kSlots];
    __shared__ double dg_sh[4];
    const int s = threadIdx.x % kSlots;
    const int j = __builtin_amdgcn_readfirstlane(threadIdx.x / kSlots);   // wave-uniform (kSlots = wave size)
    const int a = blockIdx.x * kSlots + s;
    const bool va = a < A;
    const uint32_t ac = va ? a : 0;   // the lane's slot, clamped for loads
    const size_t b = blockIdx.y;
    const float lam = __expf(g[0]);
    const float lam16 = pow_int(lam, kSeg);
    const float wa = va ? w[a] : 1.f;
    const float rb = va ? rs.slot_const(a) : 0.f;   // the slot's key bias when r is formed here
    const double tau = 0.5 * (T - 1);
    float dkc_next = 0.f;   // dkc at the first position after the chunk
    float dkt_next = 0.f;   // dkt at the first position after the chunk
    float dw_acc = 0.f;
    double dg_acc = 0.0;
    for (int n = NT - 1; n >= 0; --n) {
        const int t0 = n * ULM_CHUNK + j * kSeg;
        const float seg_c = seg_inv<RS>(seg_row_raw(rs, b * T + t0, t0, T, s));
        // xv: the extra gradient of q (dq_out or d(w q), by XQ); dq is formed
        // from dqfv and xv where q is, so neither outlives the reverse scan
        float rv[kSeg], kv[kSeg], cv[kSeg], dqc[kSeg], dqfv[kSeg], xv[kSeg], dkfv[kSeg];
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
            const int t = t0 + i;
            const bool ok = va && t < T;
            const size_t ro = urow(b, t, T) * A;   // wave-uniform row offset
            rv[i] = rs.at(urow(b, t, T), ac, A, rb, lane_value(seg_c, i), ok);
            // unconditional loads at the clamped row and slot keep the waits and
            // the 16-bit conversions out of a branch; dk_f is loaded with the
            // rest so that all of the chunk's reads are in flight together
            const float f = ld_row(dqf + ro, 4u * ac);
            dqfv[i] = ok ? f : 0.f;
            const float x = XQ != 0 ? load_xq<XQ>(xq, ro, ac) : 0.f;
            xv[i] = ok ? x : 0.f;
            const float fk = ld_row(dkf + ro, 4u * ac);
            dkfv[i] = ok ? fk : 0.f;
        }
        kv[0] = rs.at(urow(b, t0 - 1, T), ac, A, rb, lane_value(seg_c, kSeg), va && t0 >= 1 && t0 - 1 < T);
#pragma unroll
        for (int i = 1; i < kSeg; ++i) kv[i] = rv[i - 1];
        // rebuild n (hence c) inside the chunk from its checkpoint
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
            acc = lam * acc + kv[i];
            cv[i] = acc;
        }
        tot[j][s] = acc;
        __syncthreads();
        float cj = va ? nck[(b * NT + n) * A + a] : 0.f;
        for (int m = 0; m < j; ++m) cj = lam16 * cj + tot[m][s];
        __syncthreads();
        float pw = lam;
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
            cv[i] = wa + (pw * cj + cv[i]);
            pw *= lam;
        }
        // dc and its reverse decayed scan. The dw terms and the q-side dg terms
        // are summed here, where q is formed, and dq / c is kept for dr, so c,
        // dq_f, the extra gradient and dc die with this loop (positions past T
        // contribute exact zeros to every term).
        float rl[kSeg];
        float racc = 0.f;
        // dg weights position t0 + i by (t0 - tau) + i: sums of e and i e per segment
        double e0 = 0.0, e1 = 0.0;
#pragma unroll
        for (int i = kSeg - 1; i >= 0; --i) {
            // q = r / c, recomputed with the forward's operations (c is rebuilt
            // exactly from its checkpoint), so q is not read back from HBM
            // q with the forward's exact division; the two gradient quotients
            // by c take the hardware reciprocal (about 1 ulp), a third of the
            // instructions of a correctly rounded division each
            const float qt = rv[i] / cv[i];
            const float ic = __builtin_amdgcn_rcpf(cv[i]);
            const float dq = dqfv[i] + (XQ == 1 ? xv[i] : wa * xv[i]);
            const float dc = -(dq * qt) * ic;
            dqc[i] = dq * ic;
            racc = dc + lam * racc;
            rl[i] = racc;
            dw_acc += dc;
            if constexpr (XQ >= 2) dw_acc += qt * xv[i];
            // The fast-read terms take the bf16 q and k that the dq and dk
            // products contracted with, so each (t, s) pair enters both sums
            // with the same value and the position weights cancel to t - s.
            const float q16 = bf16_to_f32(f32_to_bf16_bits(qt));
            const double e = static_cast<double>((fast_dg ? q16 * dqfv[i] : 0.f) + dc * (cv[i] - wa));
            e0 += e;
            e1 += i * e;
        }
        // finish the q-side sums here: left to the compiler, they sink past the
        // barriers and keep q, dq_f, the extra gradient, dc and c alive through
        // the final phase
        asm volatile("" : "+v"(e0), "+v"(e1), "+v"(dw_acc));
        tot[j][s] = racc;
        __syncthreads();
        float rj = dkc_next;
        for (int m = 3; m > j; --m) rj = tot[m][s] + lam16 * rj;
        float dkcv[kSeg];   // dkt = dkfv + dkcv
        float pr = lam;   // lam^(16-i) for i = 15 .. 0
#pragma unroll
        for (int i = kSeg - 1; i >= 0; --i) {
            dkcv[i] = rl[i] + pr * rj;
            pr *= lam;
        }
        first_dkt[j][s] = dkfv[0] + dkcv[0];
        if (j == 0) tot[0][s] = rl[0] + pow_int(lam, kSeg) * rj;   // dkc at chunk start (rl[0] + lam^16 r_0)
        __syncthreads();
        const float after = (j == 3) ? dkt_next : first_dkt[j + 1][s];
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
            const int t = t0 + i;
            const float nxt = (i + 1 < kSeg) ? dkfv[i + 1] + dkcv[i + 1] : after;
            if (va && t < T) st_row(dr + (b * T + t) * A, 4u * ac, dqc[i] + nxt);
            const float k16 = bf16_to_f32(f32_to_bf16_bits(kv[i]));
            const double e = static_cast<double>((fast_dg ? k16 * dkfv[i] : 0.f) + kv[i] * dkcv[i]);
            e0 -= e;
            e1 -= i * e;
        }
        dg_acc += (static_cast<double>(t0) - tau) * e0 + e1;
        dkc_next = tot[0][s];
        dkt_next = first_dkt[0][s];
        __syncthreads();
    }
    dw_sh[j][s] = dw_acc;
    dg_acc = wave_sum(dg_acc);
    if (threadIdx.x % kWave == 0) dg_sh[threadIdx.x / kWave] = dg_acc;
    __syncthreads();
    if (j == 0 && va) dw_part[b * A + a] = dw_sh[0][s] + dw_sh[1][s] + dw_sh[2][s] + dw_sh[3][s];
    if (threadIdx.x == 0) dg_part[b * gridDim.x + blockIdx.x] = dg_sh[0] + dg_sh[1] + dg_sh[2] + dg_sh[3];
}

// dw[a] = sum_b dw_part[b, a]; dg = sum of all dg partials (those of the
// statistics and, when given, nextra more). Every sum runs in a fixed order
// (thread-strided partial sums, then a fixed shuffle tree), so the result does
// not depend on scheduling.
__global__ __launch_bounds__(256) void stats_reduce_kernel(const float *__restrict__ dw_part,
                                                           const double *__restrict__ dg_part,
                                                           const double *__restrict__ dg_extra, float *__restrict__ dw,
                                                           float *__restrict__ dg, int B, int A, int ndg, int nextra) {
    __shared__ double red[4];
    const int a = blockIdx.x * 256 + threadIdx.x;
    if (a < A) {
        float s = 0.f;
        for (int b = 0; b < B; ++b) s += dw_part[static_cast<size_t>(b) * A + a];
        dw[a] = s;
    }
    if (blockIdx.x == 0) {
        double s = 0.0;
        for (int k = threadIdx.x; k < ndg; k += 256) s += dg_part[k];
        for (int k = threadIdx.x; k < nextra; k += 256) s += dg_extra[k];
        s = wave_sum(s);
        if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = s;
        __syncthreads();
        if (threadIdx.x == 0) dg[0] = static_cast<float>((red[0] + red[1]) + (red[2] + red[3]));
    }
}

// q16n, k16n: natural bf16 copies (both or neither); qR, kR, qQ, kQ: tiled
// copies AL slots wide (0: AL = A; AL % 32 == 0, the slots past A zero).
int launch_fwd_stats(const RSrc &src, const float *w, const float *g, float *q, uint16_t *q16n, uint16_t *k16n,
                     uint16_t *qR, uint16_t *kR, uint16_t *qQ, uint16_t *kQ, float *nck, float *c_last, int B, int T,
                     int A, hipStream_t s, void *qw, int qw_dt, int AL) {
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    if ((q16n == nullptr) != (k16n == nullptr)) return fail(ULM_ERR_INVALID, "fwd stats: q16n and k16n go together");
    // the tiled copies: kQ always, qR and kR together (the chunked products'
    // R layout), qQ when a backward follows
    const bool tiled = qR || kR || qQ || kQ;
    if (AL == 0) AL = A;
    // the grid's blocks of kSlots slots cover the layout's padding slots too
    if (tiled && !(kQ && (qR != nullptr) == (kR != nullptr) && AL % 32 == 0 && A <= AL &&
                   AL <= (A + kSlots - 1) / kSlots * kSlots))
        return fail(ULM_ERR_INVALID, "fwd stats: tiled copies need kQ, qR with kR, and a layout width %d for A=%d", AL, A);
    if (qw && !valid_dtype(qw_dt)) return fail(ULM_ERR_INVALID, "fwd stats: bad w q dtype %d", qw_dt);
    const int qwk = qw ? qw_dt : -1;
    return with_rsrc(src, [&](auto rs) {
        using RS = decltype(rs);
        const dim3 grid((A + kSlots - 1) / kSlots, B);
#define ULM_FWD_STATS(QWK, HQ)                                                                                    \
    fwd_stats_kernel<RS, QWK, HQ><<<grid, 256, 0, s>>>(rs, w, g, q, qw, qw_dt, q16n, k16n, qR, kR, qQ, kQ, nck,   \
                                                       c_last, T, A, AL, NT)
        if (q) {
            switch (qwk) {
            case ULM_F32: ULM_FWD_STATS(ULM_F32, true); break;
            case ULM_BF16: ULM_FWD_STATS(ULM_BF16, true); break;
            case ULM_F16: ULM_FWD_STATS(ULM_F16, true); break;
            default: ULM_FWD_STATS(-1, true); break;
            }
        } else {
            switch (qwk) {
            case ULM_F32: ULM_FWD_STATS(ULM_F32, false); break;
            case ULM_BF16: ULM_FWD_STATS(ULM_BF16, false); break;
            case ULM_F16: ULM_FWD_STATS(ULM_F16, false); break;
            default: ULM_FWD_STATS(-1, false); break;
            }
        }
#undef ULM_FWD_STATS
        return check_launch("fwd_stats_kernel");
    });
}

size_t bwd_stats_partial_bytes(int B, int A) {
    const size_t nb = (A + kSlots - 1) / kSlots;
    return align_up(static_cast<size_t>(B) * A * sizeof(float), 256) + align_up(B * nb * sizeof(double), 256);
}

// dg_extra: nextra more partials of dg (the block-pair products' fast-read
// part); when given, the dq_f / dk_f terms of the positional identity are left
// out here (fast_dg = 0), since those partials hold that part already.
int launch_bwd_stats(const float *dqf, const float *dqo, const RSrc &src, const float *nck,
                     const float *w, const float *g, const float *dkf, float *dr, float *dw, float *dg, void *part,
                     int B, int T, int A, hipStream_t s, const void *dqw, int dqw_dt, const double *dg_extra,
                     int nextra) {
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    const int nb = (A + kSlots - 1) / kSlots;
    float *dw_part = static_cast<float *>(part);
    double *dg_part = reinterpret_cast<double *>(static_cast<char *>(part) +
                                                 align_up(static_cast<size_t>(B) * A * sizeof(float), 256));
    const int xq = dqw ? 2 + dqw_dt : (dqo ? 1 : 0);   // ULM_F32, ULM_BF16, ULM_F16 = 0, 1, 2
    const void *xp = dqw ? dqw : static_cast<const void *>(dqo);
    if (dqw && dqo) return fail(ULM_ERR_INVALID, "bwd stats: dq_out and d(w q) are exclusive");
    if (xq < 0 || xq > 4) return fail(ULM_ERR_INVALID, "bwd stats: bad d(w q) dtype %d", dqw_dt);
    const int fast_dg = dg_extra ? 0 : 1;
    ULM_TRY(with_rsrc(src, [&](auto rs) {
        using RS = decltype(rs);
        const dim3 grid(nb, B);
        switch (xq) {
        case 0: bwd_stats_kernel<0, RS><<<grid, 256, 0, s>>>(dqf, xp, rs, nck, w, g, dkf, dr, dw_part, dg_part, T, A, NT, fast_dg); break;
        case 1: bwd_stats_kernel<1, RS><<<grid, 256, 0, s>>>(dqf, xp, rs, nck, w, g, dkf, dr, dw_part, dg_part, T, A, NT, fast_dg); break;
        case 2: bwd_stats_kernel<2, RS><<<grid, 256, 0, s>>>(dqf, xp, rs, nck, w, g, dkf, dr, dw_part, dg_part, T, A, NT, fast_dg); break;
        case 3: bwd_stats_kernel<3, RS><<<grid, 256, 0, s>>>(dqf, xp, rs, nck, w, g, dkf, dr, dw_part, dg_part, T, A, NT, fast_dg); break;
        default: bwd_stats_kernel<4, RS><<<grid, 256, 0, s>>>(dqf, xp, rs, nck, w, g, dkf, dr, dw_part, dg_part, T, A, NT, fast_dg); break;
        }
        return ULM_OK;
    }));
    int st = check_launch("bwd_stats_kernel");
    if (st) return st;
    stats_reduce_kernel<<<(A + 255) / 256, 256, 0, s>>>(dw_part, dg_part, dg_extra, dw, dg, B, A, B * nb,
                                                        dg_extra ? nextra : 0);
    return check_launch("stats_reduce_kernel");
}

}  // namespace ulm
