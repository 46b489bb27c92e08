// K-group chunked linear attention for K % 32 == 0 and V % 32 == 0,
//
//   o_t = sum_{s<=t} lam^(t-s) (a_t . b_s) c_s        (s >= t for the reversed walk)
//
// the product behind every call of `_la` (kernel.py:183-196), with the fp32
// chunk state held in registers for the whole walk instead of being written
// out per chunk (the reference stores it to HBM in bf16, kernel.py:38).
//
// Workgroup = (batch row b, key group of up to 24 blocks of 32 keys, 64 value
// columns), 4 waves. Wave w holds the state of key blocks w, w+4, ... (up to
// 6) of the group x 64 columns (192 fp32 registers per lane) and walks the
// chunks; per chunk n (positions 64n .. 64n+63):
//   read-out  O_w  = diag(s lam^(i+1)) a_n[:, keys_w] bf16(G_w)
//   intra     O_w += P_n[:, 16w:16w+16] c_n[16w:16w+16, :]     (key group 0 only)
//   exchange  O = sum_w O_w through LDS; wave w stores rows 16w .. 16w+15
//   update    G_w += b_n[:, keys_w]^T (lam^(63-j) c_n[j] / s')
// Every operand is one 16-byte global load per lane:
//   a in its natural layout (B, T, K); b and c in the chunk-transposed layout
//   (B, NT, K|V, 64) of chunk_transpose; P (B, NT, 64, 64) from chunk_scores.
// The rows of a 32-key state block are held in the order key(rho) = rho with
// bits 2 and 3 exchanged. In that order the accumulator layout of
// v_mfma_f32_32x32x16_bf16 (lane l, register r -> row 8(r/4) + 4(l/32) + r%4,
// column l%32), taken 8 registers at a time (h = 0, 1), is the B operand of
// the read-out with contraction index 8(l/32) + e <-> key 16h + 8(l/32) + e,
// so the matching A operand is 8 consecutive keys of one row of a.
//
// Reversed walk: chunks are visited n = NT-1 .. 0 over the same forward-chunk
// layouts, and inside a chunk the decays mirror: read-out row i takes
// lam^(64-i), update position j takes lam^j, the intra matrix is the upper
// triangular P_up. Positions past T are zero in b, c and P, so padding the
// last chunk changes no lag.
//
// State scaling: H = s G with a wave-uniform scalar s, so the per-chunk decay
// lam^64 folds into s; G is rescaled (s = 1) only when s would fall below
// 2^-40. SPLIT carries the decayed update operand as a bf16 hi + lo pair
// (twice the update MFMAs), exact to fp32 accumulation for bf16 inputs.
//
// With more than one key group, group k writes its partial output to
// out + k*B*T*V (fp32), summed afterwards by partial_reduce.
#include "ulm_common.h"

#include <algorithm>

namespace ulm {

// launch timer of fm_chunk.hip
int la_timer_begin(hipStream_t s);
int la_timer_end(hipStream_t s);

namespace kgrp {

constexpr int C = ULM_CHUNK;
constexpr int WAVES = 8;                    // two per SIMD
constexpr int MAX_MH = 3;                   // key blocks per wave, at most
constexpr int GROUP_BLOCKS = WAVES * MAX_MH;   // 24 blocks = 768 keys per workgroup
constexpr int VT = 64;                      // value columns per workgroup
constexpr int OPITCH = C + 4;               // floats per column of the exchange buffer
constexpr int OBUF = WAVES * VT * OPITCH;   // floats of the exchange buffer
constexpr int LDS_BYTES = OBUF * 4;
constexpr int ROWS_PER_WAVE = C / WAVES;    // output rows each wave reduces and stores
constexpr uint32_t OOB = 0x80000000u;       // buffer offset past every range: the load returns zeros

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// Raw buffer over `bytes` bytes at base; offsets at or past `bytes` read as zero.
__device__ __forceinline__ rsrc_t rsrc(const void *base, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}
// 16 bytes at byte offset `off` (the range check applies to this offset)
__device__ __forceinline__ bf16x8 bld(rsrc_t rs, uint32_t off) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0));
}
__device__ __forceinline__ float uniform(float x) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}
__device__ __forceinline__ uint32_t uniform(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }
// own LDS traffic done, then meet the other waves
__device__ __forceinline__ void sync_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// MH: key blocks per wave (blocks past the group's end read as zero). SPLIT: the
// update operand comes as bf16 hi + lo (UA, UAlo); ASPLIT: the read-out operand
// as hi + lo (A_, Alo).
template <int MH, bool REV, bool SPLIT, bool ASPLIT>
__global__ __launch_bounds__(WAVES * 64, 1) void la_kgroup_kernel(const uint16_t *__restrict__ A_,
                                                                  const uint16_t *__restrict__ Alo,
                                                                  const uint16_t *__restrict__ UA,
                                                                  const uint16_t *__restrict__ UAlo,
                                                                  const uint16_t *__restrict__ UB,
                                                                  const uint16_t *__restrict__ CR,
                                                                  const uint16_t *__restrict__ P,
                                                                  const float *__restrict__ g, float *__restrict__ out,
                                                                  int Btot, int T, int K, int V, int NT, int nKG, int bpg,
                                                                  int nVT, int total) {
    extern __shared__ __align__(16) float obuf[];   // [WAVES][VT][OPITCH]

    int tile = blockIdx.x;
    if (total % 8 == 0) tile = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;   // XCD-local tiles
    const int vt = tile % nVT;
    const int kgi = (tile / nVT) % nKG;
    const int b = tile / (nVT * nKG);
    const int v0 = vt * VT;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave, lr = lane % 32, lh = lane / 32;

    // this wave's key blocks: blk0 + wave + WAVES mh (valid while < blk1)
    const int blk0 = kgi * bpg;
    const int blk1 = min(K / 32, blk0 + bpg);
    const bool nt1 = v0 + 32 < V;   // the second 32-column tile lies inside V (the first always does)
    const bool intra = kgi == 0;
    const int iq = wave % 4, imt = wave / 4;   // intra-chunk share: position quarter iq of row half imt

    // ---- read-out row factors lam^(i+1) (lam^(64-i) reversed), i = 32 mt + 8 q + 4 lh + m
    const float gl = g[0];
    float upart[2][4];   // uniform part
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            upart[mt][q] = uniform(__expf(gl * static_cast<float>(REV ? 32 * (1 - mt) + 8 * (3 - q) : 32 * mt + 8 * q)));
    float rrow[4];       // lane part
#pragma unroll
    for (int m = 0; m < 4; ++m) rrow[m] = __expf(gl * static_cast<float>(REV ? 8 - 4 * lh - m : 1 + 4 * lh + m));
    const float lam64 = state_lam64(gl);
    const bool tiny = lam64 < kRenorm;

    // ---- operand buffers, one batch row each (tile layouts of ulm_common.h);
    // byte offset of a tile load = 16 lane + a uniform tile offset
    const int KT16 = K / 16, KT32 = K / 32, VT32 = V / 32;
    const size_t rowA = static_cast<size_t>(2 * NT) * KT16 * kTileElems;    // R layout
    const size_t rowU = static_cast<size_t>(NT) * KT32 * 4 * kTileElems;    // Q layout, keys
    const size_t rowB = static_cast<size_t>(NT) * VT32 * 4 * kTileElems;    // Q layout, values
    const size_t rowP = static_cast<size_t>(NT) * 8 * kTileElems;           // score tiles
    const rsrc_t ra = rsrc(A_ + b * rowA, rowA * 2);
    const rsrc_t ral = rsrc((ASPLIT ? Alo : A_) + b * rowA, rowA * 2);
    const rsrc_t rua = rsrc(UA + b * rowU, rowU * 2);
    const rsrc_t rul = rsrc((SPLIT ? UAlo : UA) + b * rowU, rowU * 2);
    const rsrc_t rub = rsrc(UB + b * rowB, rowB * 2);
    const rsrc_t rcr = rsrc(CR + b * rowB, rowB * 2);
    const rsrc_t rp = rsrc(P + b * rowP, rowP * 2);
    constexpr uint32_t TB = kTileElems * 2;   // bytes per tile
    const uint32_t lane16 = static_cast<uint32_t>(lane * 16);
    uint32_t ub_lane[2], cr_lane[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        ub_lane[nt] = (nt == 0 || nt1) ? lane16 + nt * 4 * TB : OOB;
        cr_lane[nt] = (nt == 0 || nt1) ? lane16 + nt * 4 * TB + iq * TB : OOB;
    }
    const uint32_t p_lane = lane16 + (imt * 4 + iq) * TB;
    // uniform key-block offsets (bytes) into a rows and into the update operand; OOB past the group
    uint32_t a_blk[MH], u_blk[MH];
#pragma unroll
    for (int mh = 0; mh < MH; ++mh) {
        const int blk = blk0 + wave + WAVES * mh;
        a_blk[mh] = uniform(blk < blk1 ? static_cast<uint32_t>(2 * blk) * TB : OOB);
        u_blk[mh] = uniform(blk < blk1 ? static_cast<uint32_t>(4 * blk) * TB : OOB);
    }
    float *out_k = out + static_cast<size_t>(kgi) * Btot * T * V;

    f32x16 G[MH][2];
#pragma unroll
    for (int mh = 0; mh < MH; ++mh)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) G[mh][nt][r] = 0.f;
    float s_state = 1.f;

    for (int step = 0; step < NT; ++step) {
        const int n = REV ? NT - 1 - step : step;
        const uint32_t cb = uniform(static_cast<uint32_t>(n * VT32 + v0 / 32) * 4 * TB);   // this chunk's value tiles

        // ---- rescaling of G around the read-out (rarely): renormalisation
        // (G *= s, s = 1) before, when s fell below 2^-40, or, when lam^64 itself
        // is below that, the decay G *= lam^64 after.
        const bool readout = step > 0;
        if (readout && !tiny && s_state < kRenorm) {
#pragma unroll
            for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) G[mh][nt][r] *= s_state;
            s_state = 1.f;
        }

        // ---- read-out of H = s G, one 32-row half at a time, plus this wave's
        // share of the intra-chunk product; both halves go to the exchange buffer.
        f32x16 O[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int r = 0; r < 16; ++r) O[mt][nt][r] = 0.f;
            if (readout) {
#pragma unroll
                for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                    for (int hb = 0; hb < 2; ++hb) {
                        const uint32_t aoff = lane16 + uniform(static_cast<uint32_t>((2 * n + mt) * KT16) * TB) +
                                              a_blk[mh] + hb * TB;
                        const bf16x8 aop = bld(ra, aoff);
                        const bf16x8 aol = ASPLIT ? bld(ral, aoff) : bf16x8{};
                        bf16x8 gop[2];
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                            for (int e = 0; e < 8; ++e) gop[nt][e] = static_cast<bf16>(G[mh][nt][8 * hb + e]);
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt) {
                            O[mt][nt] = mfma(aop, gop[nt], O[mt][nt]);
                            if (ASPLIT) O[mt][nt] = mfma(aol, gop[nt], O[mt][nt]);
                        }
                    }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float f = s_state * upart[mt][q];
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const float sc = f * rrow[m];
                        O[mt][0][4 * q + m] *= sc;
                        O[mt][1][4 * q + m] *= sc;
                    }
                }
            }
        }
        if (intra) {
            const bf16x8 pq = bld(rp, p_lane + uniform(static_cast<uint32_t>(n * 8) * TB));
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const bf16x8 ci = bld(rcr, cr_lane[nt] + cb);
                if (imt == 0) O[0][nt] = mfma(pq, ci, O[0][nt]);
                else O[1][nt] = mfma(pq, ci, O[1][nt]);
            }
        }
        if (readout && tiny) {
#pragma unroll
            for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) G[mh][nt][r] *= lam64;
        }
        s_state = tiny ? 1.f : lam64 * s_state;   // scale after this chunk's update

        // every wave has finished reducing the previous chunk's partials
        if (step > 0) sync_lds();
        {
            float *ob = obuf + wave * (VT * OPITCH);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        f32x4 x;
#pragma unroll
                        for (int m = 0; m < 4; ++m) x[m] = O[mt][nt][4 * q + m];
                        *reinterpret_cast<f32x4 *>(ob + (32 * nt + lr) * OPITCH + 32 * mt + 8 * q + 4 * lh) = x;
                    }
        }

        // ---- state update G += UA^T UB (the decay and 1/s are inside the stored
        // operand); the lo part of a split operand in a second pass
        if (step + 1 < NT) {
            bf16x8 ub[2][4];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) ub[nt][ks] = bld(rub, ub_lane[nt] + cb + ks * TB);
            const uint32_t urow = uniform(static_cast<uint32_t>(n * KT32) * 4 * TB);
#pragma unroll
            for (int pass = 0; pass < (SPLIT ? 2 : 1); ++pass) {
                const rsrc_t ru = pass ? rul : rua;
#pragma unroll
                for (int mh = 0; mh < MH; ++mh) {
                    bf16x8 bop[4];
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) bop[ks] = bld(ru, lane16 + urow + u_blk[mh] + ks * TB);
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt) G[mh][nt] = mfma(bop[ks], ub[nt][ks], G[mh][nt]);
                }
            }
        }

        // ---- exchange: wave w sums rows 8w .. 8w+7 of the eight partials, lane = column
        sync_lds();
        {
            const float *rb = obuf + lane * OPITCH + ROWS_PER_WAVE * wave;
            f32x4 acc[2];
#pragma unroll
            for (int q4 = 0; q4 < 2; ++q4) acc[q4] = *reinterpret_cast<const f32x4 *>(rb + 4 * q4);
#pragma unroll
            for (int w2 = 1; w2 < WAVES; ++w2)
#pragma unroll
                for (int q4 = 0; q4 < 2; ++q4) acc[q4] += *reinterpret_cast<const f32x4 *>(rb + w2 * (VT * OPITCH) + 4 * q4);
            // value tiles hold their 32 columns in the order perm32
            const int col = v0 + 32 * (lane / 32) + perm32(lane % 32);
            if (col < V) {
                float *dst = out_k + (static_cast<size_t>(b) * T + n * C + ROWS_PER_WAVE * wave) * V + col;
#pragma unroll
                for (int q4 = 0; q4 < 2; ++q4)
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        if (n * C + ROWS_PER_WAVE * wave + 4 * q4 + m < T) dst[static_cast<size_t>(4 * q4 + m) * V] = acc[q4][m];
            }
        }
    }
}

template <int MH, bool REV, bool SPLIT, bool ASPLIT>
int launch(const uint16_t *a, const uint16_t *alo, const uint16_t *ua, const uint16_t *ualo, const uint16_t *ub,
           const uint16_t *cr, const uint16_t *P, const float *g, float *out, int B, int T, int K, int V, int nKG,
           int bpg, hipStream_t s) {
    const int NT = (T + C - 1) / C;
    const int nVT = (V + VT - 1) / VT;
    const long long total = static_cast<long long>(B) * nKG * nVT;
    static bool attr_done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return check_launch("hipGetDevice");
    if (!attr_done[dev]) {
        const void *fn = reinterpret_cast<const void *>(&la_kgroup_kernel<MH, REV, SPLIT, ASPLIT>);
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES) != hipSuccess)
            return check_launch("la_kgroup_kernel attribute");
        attr_done[dev] = true;
    }
    int st = la_timer_begin(s);
    if (st) return st;
    la_kgroup_kernel<MH, REV, SPLIT, ASPLIT><<<dim3(static_cast<unsigned>(total)), WAVES * kWave, LDS_BYTES, s>>>(
        a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, NT, nKG, bpg, nVT, static_cast<int>(total));
    st = check_launch("la_kgroup_kernel");
    if (st) return st;
    return la_timer_end(s);
}

template <int MH>
int launch_mh(const uint16_t *a, const uint16_t *alo, const uint16_t *ua, const uint16_t *ualo, const uint16_t *ub,
              const uint16_t *cr, const uint16_t *P, const float *g, float *out, int B, int T, int K, int V, int nKG,
              int bpg, bool reverse, hipStream_t s) {
    const int sel = (reverse ? 4 : 0) + (ualo ? 2 : 0) + (alo ? 1 : 0);
    switch (sel) {
    case 0: return launch<MH, false, false, false>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    case 1: return launch<MH, false, false, true>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    case 2: return launch<MH, false, true, false>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    case 3: return launch<MH, false, true, true>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    case 4: return launch<MH, true, false, false>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    case 5: return launch<MH, true, false, true>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    case 6: return launch<MH, true, true, false>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    default: return launch<MH, true, true, true>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, s);
    }
}

}  // namespace kgrp

// Number of key groups (fp32 partial outputs) the K-group kernel produces for K keys.
int la_kgroup_groups(int K) {
    const int nb = K / 32;
    return (nb + kgrp::GROUP_BLOCKS - 1) / kgrp::GROUP_BLOCKS;
}

bool la_kgroup_supported(int B, int T, int K, int V) {
    if (B <= 0 || T <= 0 || K <= 0 || V <= 0 || K % 32 || V % 32) return false;
    const long long total = static_cast<long long>(B) * la_kgroup_groups(K) * ((V + kgrp::VT - 1) / kgrp::VT);
    // 32-bit buffer offsets: with every per-row operand region below 1 GB, a
    // lane offset plus a uniform offset plus the out-of-range marker (2^31)
    // stays below 2^32, so masked loads never wrap back into range
    const long long NT = (T + ULM_CHUNK - 1) / ULM_CHUNK;
    const long long rowmax = std::max({static_cast<long long>(T) * K, NT * K * ULM_CHUNK, NT * V * ULM_CHUNK}) * 2;
    return total <= 0x7fffffffLL && rowmax < (1LL << 30);
}

// Operands (bf16 tiles, ulm_common.h): a (+ alo) in the R layout; ua (+ ualo)
// and ub, cr in the Q layout. The update adds ua^T ub (+ ualo^T ub); one of ua
// / ub carries the decay and 1/s of the state scale schedule (chunk_transpose).
// The read-out contracts a (+ alo) with the state. cr is the raw c of the
// intra-chunk product; P is P_lo (forward) or P_up (reverse) of chunk_scores.
// out: la_kgroup_groups(K) x (B, T, V) fp32, fully written (no accumulation).
int launch_la_kgroup(const uint16_t *a, const uint16_t *alo, const uint16_t *ua, const uint16_t *ualo,
                     const uint16_t *ub, const uint16_t *cr, const uint16_t *P, const float *g, float *out, int B,
                     int T, int K, int V, bool reverse, hipStream_t s) {
    if (!la_kgroup_supported(B, T, K, V))
        return fail(ULM_ERR_UNSUPPORTED, "K-group kernel: B=%d T=%d K=%d V=%d unsupported", B, T, K, V);
    const int nKG = la_kgroup_groups(K);
    const int nb = K / 32;
    const int bpg = (nb + nKG - 1) / nKG;   // <= 24 blocks, so at most 3 per wave
    const int mh = (bpg + kgrp::WAVES - 1) / kgrp::WAVES;
    switch (mh) {
    case 1: return kgrp::launch_mh<1>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, reverse, s);
    case 2: return kgrp::launch_mh<2>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, reverse, s);
    default: return kgrp::launch_mh<3>(a, alo, ua, ualo, ub, cr, P, g, out, B, T, K, V, nKG, bpg, reverse, s);
    }
}

}  // namespace ulm
