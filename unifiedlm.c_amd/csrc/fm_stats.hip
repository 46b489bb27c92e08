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
//
// Sequence segments: a workgroup scans the chunks of one segment of
// kSegChunks chunks (1024 positions), so that a long sequence over few batch
// rows still spreads over the CUs. The values carried into a segment come
// from a totals pass over the segments that precede it (forward) or follow it
// (backward), folded by each workgroup in a fixed order. The segment length
// is fixed, so a row's arithmetic does not depend on the batch size; a
// sequence of one segment has no totals pass and nothing carried in.
#include "ulm_common.h"

#include <type_traits>

namespace ulm {

constexpr int kSeg = 16;      // positions per thread segment
constexpr int kSlots = 64;    // slots per block
constexpr int kSegChunks = 16;                   // chunks per sequence segment
constexpr int kSegLen = kSegChunks * ULM_CHUNK;  // positions per sequence segment

int stat_segments(int T) {
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    return (NT + kSegChunks - 1) / kSegChunks;
}

__device__ __forceinline__ float pow_int(float x, int e) {
    float r = 1.f;
    for (int i = 0; i < e; ++i) r *= x;
    return r;
}
// x^(2^k) by k squarings
__device__ __forceinline__ float pow_2k(float x, int k) {
    for (int i = 0; i < k; ++i) x *= x;
    return x;
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

// The forward's segment totals: tot[b][j][a], for the segments j < S - 1, is n
// at the last position of segment j with n = 0 before the segment
// (n_t = lam n_{t-1} + k_t). A workgroup of 16 waves takes 64 slots of one
// segment, wave w its chunk w: each lane walks the chunk's 64 positions in
// order, 16 loads in flight, and the chunks join as
// (((p_0 lam^64 + p_1) lam^64 + p_2) ...) lam^64 + p_15.
template <class RS>
__global__ __launch_bounds__(1024) void fwd_segtot_kernel(RS rs, const float *__restrict__ g,
                                                          float *__restrict__ tot, int T, int A, int S) {
    __shared__ float part[kSegChunks][kSlots];
    const int s = threadIdx.x % kSlots;
    const int u = __builtin_amdgcn_readfirstlane(threadIdx.x / kSlots);   // the wave's chunk in the segment
    const int a = blockIdx.x * kSlots + s;
    const bool va = a < A;
    const uint32_t ac = va ? a : 0;
    const size_t b = blockIdx.y;
    const int j = blockIdx.z;
    const float lam = __expf(g[0]);
    const float rb = va ? rs.slot_const(a) : 0.f;
    const int t0 = j * kSegLen + u * ULM_CHUNK;
    float n = 0.f;
    for (int i0 = 0; i0 < ULM_CHUNK; i0 += kSeg) {
        float kv[kSeg];
#pragma unroll
        for (int i = 0; i < kSeg; ++i) {
            const int t = t0 + i0 + i - 1;   // k at position t + 1 is r at t
            const bool tok = t >= 0 && t < T;
            const float inv = seg_inv<RS>(rs.row_raw(urow(b, t, T), tok));
            kv[i] = rs.at(urow(b, t, T), ac, A, rb, inv, va && tok);
        }
#pragma unroll
        for (int i = 0; i < kSeg; ++i) n = lam * n + kv[i];
    }
    part[u][s] = n;
    __syncthreads();
    if (u == 0 && va) {
        const float l64 = pow_2k(lam, 6);   // lam^64
        float acc = part[0][s];
        for (int m = 1; m < kSegChunks; ++m) acc = l64 * acc + part[m][s];
        tot[(b * S + j) * A + a] = acc;
    }
}

// Outputs besides n_ckpt (each may be null): q (fp32); qw = w q in qw_dt; q16n, k16n natural bf16
// copies; qR, kR in the R layout and qQ, kQ in the Q layout (the products'
// operand tiles, AL slots wide: AL % 32 == 0, A <= AL <= the grid's slots);
// c_last = c at position T-1 (B, A), the decode state after the sequence.
// Positions past T and slots past A are zero in R and Q. With kq_decay, kQ
// holds the keys decayed to position T-1, k_t lam^(T-1-t) (the operand of the
// decode state as one product over positions).
// segtot: the segment totals of sequences past one segment (see above).
// QW: the dtype of the w q output (-1 none, else a ulm_dtype); HAS_Q: the fp32 q output.
template <class RS, int QW, bool HAS_Q>
__global__ __launch_bounds__(256) void fwd_stats_kernel(RS rs, const float *__restrict__ w,
                                                        const float *__restrict__ g, float *__restrict__ q,
                                                        void *__restrict__ qw, int qw_dt,
                                                        uint16_t *__restrict__ q16n, uint16_t *__restrict__ k16n,
                                                        uint16_t *__restrict__ qR, uint16_t *__restrict__ kR,
                                                        uint16_t *__restrict__ qQ, uint16_t *__restrict__ kQ,
                                                        float *__restrict__ nck, float *__restrict__ c_last, int T,
                                                        int A, int AL, int NT, const float *__restrict__ segtot,
                                                        int S, int kq_decay) {
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
    const float lg = g[0];
    const float lam = __expf(lg);
    const float lam16 = pow_int(lam, kSeg);
    const float wa = va ? w[a] : 1.f;
    const float rb = va ? rs.slot_const(a) : 0.f;   // the slot's key bias when r is formed here
    // this workgroup's sequence segment: chunks n0 .. n1 - 1, n carried in from
    // the totals of the segments before it
    const int seg = blockIdx.z;
    const int n0 = seg * kSegChunks, n1 = min(NT, n0 + kSegChunks);
    float carry = 0.f;   // n at the position before the chunk
    if (seg > 0) {
        const float lamL = pow_2k(lam, 10);   // lam^1024, across one segment
        for (int i = 0; i < seg; ++i) carry = lamL * carry + (va ? segtot[(bs * S + i) * A + a] : 0.f);
    }
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
    fetch(n0, 0);
    if (n0 + 1 < n1) fetch(n0 + 1, 1);
    auto chunk = [&](int n, int u) {
        const int t0 = n * ULM_CHUNK + j * kSeg;
        const float seg_c = seg_inv<RS>(pd[u]);
        float rv[kSeg], kv[kSeg], nl[kSeg];
#pragma unroll
        for (int i = 0; i < kSeg; ++i) rv[i] = rs.make(pv[u][i], rb, lane_value(seg_c, i), va && t0 + i < T);
        kv[0] = rs.make(pv[u][kSeg], rb, lane_value(seg_c, kSeg), va && t0 >= 1 && t0 - 1 < T);
        if (n + 2 < n1) fetch(n + 2, u);
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
            uint16_t qb = 0, kb = 0, kqb = 0;   // positions past T are zero in the tiled copies
            if (va && t < T) {
                const size_t ro = (bs * T + t) * A;   // wave-uniform row offset
                const float qt = rv[i] / ct;
                if (c_last && t == T - 1) c_last[bs * A + a] = ct;
                qb = f32_to_bf16_bits(qt);
                kb = f32_to_bf16_bits(kv[i]);
                // kq_decay: the Q-layout keys decayed to T - 1, k_t lam^(T-1-t)
                kqb = kq_decay ? f32_to_bf16_bits(kv[i] * __expf(lg * static_cast<float>(T - 1 - t))) : kb;
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
                kpk[i / 2] = kqb;
            } else {
                qpk[i / 2] |= static_cast<uint32_t>(qb) << 16;
                kpk[i / 2] |= static_cast<uint32_t>(kqb) << 16;
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
    for (int n = n0; n < n1; n += 2) {
        chunk(n, 0);
        if (n + 1 < n1) chunk(n + 1, 1);
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

// The backward's segment totals: tot[b][j][a], for the segments j >= 1, is
// the sum over the segment's positions t of lam^(t - t_j) dc_t (t_j its first
// position): dkc at t_j with nothing carried in from later positions. A
// workgroup of 16 waves takes 64 slots of one segment, wave w its chunk w:
// each lane rebuilds n from the chunk's checkpoint and walks the chunk's 64
// positions in order with the operations of bwd_stats_kernel for c, q and dc;
// the chunks join as p_0 + lam^64 (p_1 + lam^64 (p_2 + ... + lam^64 p_15)).
template <int XQ, class RS>
__global__ __launch_bounds__(1024) void bwd_segtot_kernel(const float *__restrict__ dqf, const void *__restrict__ xq,
                                                          RS rs, const float *__restrict__ nck,
                                                          const float *__restrict__ w, const float *__restrict__ g,
                                                          float *__restrict__ tot, int T, int A, int NT, int S) {
    __shared__ float part[kSegChunks][kSlots];
    const int s = threadIdx.x % kSlots;
    const int u = __builtin_amdgcn_readfirstlane(threadIdx.x / kSlots);   // the wave's chunk in the segment
    const int a = blockIdx.x * kSlots + s;
    const bool va = a < A;
    const uint32_t ac = va ? a : 0;
    const size_t b = blockIdx.y;
    const int j = blockIdx.z + 1;
    const float lam = __expf(g[0]);
    const float wa = va ? w[a] : 1.f;
    const float rb = va ? rs.slot_const(a) : 0.f;
    float R = 0.f, pw = 1.f;   // pw = lam^(t - the chunk's first position)
    // the wave's chunk, none past the sequence (written as a loop: this
    // compiler rejects the uniform row addresses below under an if)
    const int c0 = j * kSegChunks + u;
    for (int c = c0; c < min(NT, c0 + 1); ++c) {
        float n = va ? nck[(b * NT + c) * A + a] : 0.f;
        for (int i0 = 0; i0 < ULM_CHUNK; i0 += kSeg) {
            const int tb = c * ULM_CHUNK + i0;
            // every load of the 16 positions is issued before any arithmetic
            // (the barrier keeps the scheduler from interleaving them, which
            // left one load in flight at a time)
            typename RS::raw_t pv[kSeg + 1];
            float pd[kSeg + 1], fv[kSeg], xv[kSeg];
#pragma unroll
            for (int i = 0; i <= kSeg; ++i) {
                const int t = tb + i - 1;   // pv[i]: position tb + i - 1
                pd[i] = rs.row_raw(urow(b, t, T), t >= 0 && t < T);
                pv[i] = rs.raw(urow(b, t, T), ac, A);
            }
#pragma unroll
            for (int i = 0; i < kSeg; ++i) {
                const size_t ro = urow(b, tb + i, T) * A;
                fv[i] = ld_row(dqf + ro, 4u * ac);
                xv[i] = XQ != 0 ? load_xq<XQ>(xq, ro, ac) : 0.f;
            }
            __builtin_amdgcn_sched_barrier(0);
            float rv[kSeg + 1], dqv[kSeg];
#pragma unroll
            for (int i = 0; i <= kSeg; ++i) {
                const int t = tb + i - 1;
                rv[i] = rs.make(pv[i], rb, seg_inv<RS>(pd[i]), va && t >= 0 && t < T);
            }
#pragma unroll
            for (int i = 0; i < kSeg; ++i) {
                const float dq = fv[i] + (XQ == 1 ? xv[i] : wa * xv[i]);
                dqv[i] = va && tb + i < T ? dq : 0.f;
            }
#pragma unroll
            for (int i = 0; i < kSeg; ++i) {
                n = lam * n + rv[i];
                const float ct = wa + n;
                const float qt = rv[i + 1] / ct;
                const float dc = -(dqv[i] * qt) * __builtin_amdgcn_rcpf(ct);
                R += pw * dc;
                pw *= lam;
            }
        }
    }
    part[u][s] = R;
    __syncthreads();
    if (u == 0 && va) {
        const float l64 = pow_2k(lam, 6);   // lam^64
        float acc = part[kSegChunks - 1][s];
        for (int m = kSegChunks - 2; m >= 0; --m) acc = part[m][s] + l64 * acc;
        tot[(b * S + j) * A + a] = acc;
    }
}

template <int XQ, class RS>
__global__ __launch_bounds__(256) void bwd_stats_kernel(const float *__restrict__ dqf, const void *__restrict__ xq,
                                                        RS rs,
                                                        const float *__restrict__ nck, const float *__restrict__ w,
                                                        const float *__restrict__ g, const float *__restrict__ dkf,
                                                        float *__restrict__ dr, float *__restrict__ dw_part,
                                                        double *__restrict__ dg_part, int T, int A, int NT,
                                                        int fast_dg, const float *__restrict__ segtot, int S) {
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
    // this workgroup's sequence segment: chunks n1 - 1 down to n0, dkc carried
    // in from the totals of the segments after it
    const int seg = blockIdx.z;
    const int n0 = seg * kSegChunks, n1 = min(NT, n0 + kSegChunks);
    float dkc_next = 0.f;   // dkc at the first position after the chunk
    float dkt_next = 0.f;   // dkt at the first position after the chunk
    if (seg + 1 < S) {
        const float lamL = pow_2k(lam, 10);   // lam^1024, across one segment
        float d = 0.f;
        for (int i = S - 1; i > seg; --i) d = (va ? segtot[(b * S + i) * A + a] : 0.f) + lamL * d;
        dkc_next = d;
        // the next segment's first position is inside the sequence
        dkt_next = va ? ld_row(dkf + (b * T + n1 * ULM_CHUNK) * A, 4u * ac) + d : 0.f;
    }
    float dw_acc = 0.f;
    double dg_acc = 0.0;
    for (int n = n1 - 1; n >= n0; --n) {
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
    const size_t pr = static_cast<size_t>(seg) * gridDim.y + b;   // partial row (segment, batch row)
    if (j == 0 && va) dw_part[pr * A + a] = dw_sh[0][s] + dw_sh[1][s] + dw_sh[2][s] + dw_sh[3][s];
    if (threadIdx.x == 0) dg_part[pr * gridDim.x + blockIdx.x] = dg_sh[0] + dg_sh[1] + dg_sh[2] + dg_sh[3];
}

// dw[a] = sum over the B partial rows (segment, batch row) of dw_part[row][a];
// dg = the sum of all dg partials (those of the statistics and, when given,
// nextra more). Every sum runs in a fixed order (thread-strided partial sums,
// then a fixed shuffle tree), so the result does not depend on scheduling.
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
                     int A, hipStream_t s, void *qw, int qw_dt, int AL, float *segtot, int kq_decay) {
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    const int S = stat_segments(T);
    if ((q16n == nullptr) != (k16n == nullptr)) return fail(ULM_ERR_INVALID, "fwd stats: q16n and k16n go together");
    if (S > 1 && !segtot) return fail(ULM_ERR_INVALID, "fwd stats: %d sequence segments need their totals array", S);
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
        if (S > 1) {
            fwd_segtot_kernel<RS><<<dim3((A + kSlots - 1) / kSlots, B, S - 1), 1024, 0, s>>>(rs, g, segtot, T, A, S);
            ULM_TRY(check_launch("fwd_segtot_kernel"));
        }
        const dim3 grid((A + kSlots - 1) / kSlots, B, S);
#define ULM_FWD_STATS(QWK, HQ)                                                                                    \
    fwd_stats_kernel<RS, QWK, HQ><<<grid, 256, 0, s>>>(rs, w, g, q, qw, qw_dt, q16n, k16n, qR, kR, qQ, kQ, nck,   \
                                                       c_last, T, A, AL, NT, segtot, S, kq_decay)
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

// The forward's segment totals (none for a sequence of one segment).
size_t fwd_stats_segtot_bytes(int B, int T, int A) {
    const int S = stat_segments(T);
    return S > 1 ? align_up(static_cast<size_t>(B) * S * A * sizeof(float), 256) : 0;
}

// The backward's partial sums: dw per (segment, batch row, slot), dg per
// (segment, batch row, slot block), then the segment totals.
size_t bwd_stats_partial_bytes(int B, int T, int A) {
    const size_t nb = (A + kSlots - 1) / kSlots, rows = static_cast<size_t>(B) * stat_segments(T);
    return align_up(rows * A * sizeof(float), 256) + align_up(rows * nb * sizeof(double), 256) +
           fwd_stats_segtot_bytes(B, T, A);
}

// dg_extra: nextra more partials of dg (the block-pair products' fast-read
// part); when given, the dq_f / dk_f terms of the positional identity are left
// out here (fast_dg = 0), since those partials hold that part already.
int launch_bwd_stats(const float *dqf, const float *dqo, const RSrc &src, const float *nck,
                     const float *w, const float *g, const float *dkf, float *dr, float *dw, float *dg, void *part,
                     int B, int T, int A, hipStream_t s, const void *dqw, int dqw_dt, const double *dg_extra,
                     int nextra) {
    const int NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    const int nb = (A + kSlots - 1) / kSlots, S = stat_segments(T);
    const size_t rows = static_cast<size_t>(B) * S;   // partial rows: (segment, batch row)
    float *dw_part = static_cast<float *>(part);
    double *dg_part = reinterpret_cast<double *>(static_cast<char *>(part) + align_up(rows * A * sizeof(float), 256));
    float *segtot = reinterpret_cast<float *>(reinterpret_cast<char *>(dg_part) +
                                              align_up(rows * nb * sizeof(double), 256));
    const int xq = dqw ? 2 + dqw_dt : (dqo ? 1 : 0);   // ULM_F32, ULM_BF16, ULM_F16 = 0, 1, 2
    const void *xp = dqw ? dqw : static_cast<const void *>(dqo);
    if (dqw && dqo) return fail(ULM_ERR_INVALID, "bwd stats: dq_out and d(w q) are exclusive");
    if (xq < 0 || xq > 4) return fail(ULM_ERR_INVALID, "bwd stats: bad d(w q) dtype %d", dqw_dt);
    const int fast_dg = dg_extra ? 0 : 1;
    ULM_TRY(with_rsrc(src, [&](auto rs) {
        using RS = decltype(rs);
        const dim3 tgrid(nb, B, S - 1), grid(nb, B, S);
        auto run = [&](auto xk) {
            constexpr int XQ = decltype(xk)::value;
            if (S > 1) {
                bwd_segtot_kernel<XQ, RS><<<tgrid, 1024, 0, s>>>(dqf, xp, rs, nck, w, g, segtot, T, A, NT, S);
                ULM_TRY(check_launch("bwd_segtot_kernel"));
            }
            bwd_stats_kernel<XQ, RS><<<grid, 256, 0, s>>>(dqf, xp, rs, nck, w, g, dkf, dr, dw_part, dg_part, T, A, NT,
                                                          fast_dg, segtot, S);
            return check_launch("bwd_stats_kernel");
        };
        switch (xq) {
        case 0: return run(std::integral_constant<int, 0>{});
        case 1: return run(std::integral_constant<int, 1>{});
        case 2: return run(std::integral_constant<int, 2>{});
        case 3: return run(std::integral_constant<int, 3>{});
        default: return run(std::integral_constant<int, 4>{});
        }
    }));
    stats_reduce_kernel<<<(A + 255) / 256, 256, 0, s>>>(dw_part, dg_part, dg_extra, dw, dg, static_cast<int>(rows), A,
                                                        static_cast<int>(rows) * nb, dg_extra ? nextra : 0);
    return check_launch("stats_reduce_kernel");
}

}  // namespace ulm
