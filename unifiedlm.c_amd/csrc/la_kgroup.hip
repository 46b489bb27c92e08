// K-group chunked linear attention for K % 32 == 0 and V % 32 == 0,
//
//   o_t = sum_{s<=t} lam^(t-s) (a_t . b_s) c_s        (s >= t for the reversed walk)
//
// the product behind every call of `_la` (kernel.py:183-196), with the fp32
// chunk state held in registers for the whole walk instead of being written
// out per chunk (the reference stores it to HBM in bf16, kernel.py:38).
//
// Workgroup = (batch row b, key group of up to 24 blocks of 32 keys, 64 value
// columns), 8 waves, two per SIMD. Wave w holds the state of key blocks w,
// w+8, w+16 of the group x 64 columns (MH <= 3 blocks, 32 fp32 registers per
// block and 32-column tile) and walks the chunks; per chunk n (positions
// 64n .. 64n+63), with s the state scale after the previous update:
//   read-out  O_w  = a_n[:, keys_w] bf16(G_w)
//   intra     O_w += P_n[rows_w, 16 iq_w : 16 iq_w + 16] c_n[16 iq_w : 16 iq_w + 16, :]
//             (key group 0 only; wave w takes one of the 2 x 4 row-half x
//             position-quarter blocks of the 64 x 64 product)
//   exchange  O = diag(s lam^(i+1)) sum_w O_w through LDS; wave w stores rows
//             8w .. 8w+7
// The row factor s lam^(i+1) of the read-out is applied once, after the sum,
// when chunk_scores has divided it out of P (pscaled). Otherwise, and whenever
// lam^64 < 2^-40, the kernel scales the read-out rows of every partial instead
// and P carries no factor.
//   update    G_w += b_n[:, keys_w]^T (lam^(63-j) c_n[j] / s')
// The decayed update operand is made here, once per workgroup: wave w loads
// tile w of the chunk's eight raw c tiles (two 32-column tiles x four
// 16-position quarters), multiplies position j by lam^(63-j) / s' (s' the scale
// after this update) and stages the bf16 result, with its rounding remainder
// when UBSPLIT, and the raw tile for the intra product in LDS. Every wave then
// reads the eight staged tiles from LDS instead of global memory.
//
// Operands are bf16 tiles of 32 rows x 16 contraction elements (ulm_common.h):
// a in the R layout, b and c in the Q layout, P from chunk_scores. Every tile
// load is one 16-byte buffer load per lane; offsets past a buffer's range read
// as zero, which covers keys past the group and a missing second value tile.
//
// Pipelining: the read-out operand of chunk n+1 and the raw c tile of chunk
// n+1 are loaded before the update of chunk n; half of the update operand b_n
// is loaded right after the read-out of chunk n, before the exchange of chunk
// n-1's partials, and the other half after it. Every load therefore has the
// barrier, LDS exchange and MFMA work of a phase to arrive in.
//
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
// 2^-40 (state_inv_scale gives the same schedule on the host side).
//
// Precision: UBSPLIT adds the bf16 rounding remainder of the decayed c as a
// second update pass (exact to fp32 accumulation when b is bf16). FULL takes
// the inputs that are not bf16 as hi + lo pairs where given: the read-out
// operand (alo), the update operand (ualo, one more pass against the hi part
// of c) and c itself (clo, summed before the decay).
//
// With more than one key group, group k writes its partial output to
// out + k*B*T*V (fp32), summed afterwards by partial_reduce.
#include "ulm_common.h"

#include <algorithm>

namespace ulm {

// launch timer of fm_chunk.hip
int la_timer_begin(hipStream_t s, int tag);
int la_timer_end(hipStream_t s);

namespace kgrp {

constexpr int C = ULM_CHUNK;
constexpr int WAVES = 8;                       // two per SIMD
constexpr int MAX_MH = 3;                      // key blocks per wave, at most
constexpr int GROUP_BLOCKS = WAVES * MAX_MH;   // 24 blocks = 768 keys per workgroup
constexpr int VT = 64;                         // value columns per workgroup
constexpr int ROWS_PER_WAVE = C / WAVES;       // output rows each wave reduces and stores
// k-steps of the update operand b_n loaded before the previous chunk's
// exchange (so in flight during it); the rest follow it. More measured slower.
constexpr int UA_EARLY = 2;
constexpr uint32_t TB = kTileElems * 2;        // bytes per operand tile
constexpr uint32_t OOB = 0x80000000u;          // buffer offset past every range: the load returns zeros
// LDS: the staged c tiles (decayed hi, decayed lo, raw: eight 1 KB tiles
// each), then the exchange buffer, one 64-column x 64-row fp32 partial per
// wave, column-major with a pitch of 68 floats (the 16-byte row quads of
// consecutive columns land on distinct banks). Everything a wave addresses in
// a phase is one lane-dependent base plus immediate offsets below 64 KB.
constexpr uint32_t UB_HI = 0;                          // byte offsets
constexpr uint32_t UB_LO = UB_HI + 8 * TB;
constexpr uint32_t C_RAW = UB_LO + 8 * TB;
constexpr uint32_t XBUF = C_RAW + 8 * TB;
constexpr int OPITCH = C + 4;                          // floats per column of a partial
constexpr int XPART = VT * OPITCH;                     // floats per partial
constexpr uint32_t LDS_BYTES = XBUF + WAVES * XPART * 4;   // 163840, the whole LDS of a CU

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
// keep the scheduler from moving instructions across this point
__device__ __forceinline__ void phase() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ bf16x8 lds_tile(const char *lds, uint32_t off) {
    return *reinterpret_cast<const bf16x8 *>(lds + off);
}

// MH: key blocks per wave (blocks past the group's end read as zero).
template <int MH, bool REV, bool UBSPLIT, bool FULL>
__global__ __launch_bounds__(WAVES * 64, 1) void la_kgroup_kernel(const uint16_t *__restrict__ A_,
                                                                  const uint16_t *__restrict__ Alo,
                                                                  const uint16_t *__restrict__ UA,
                                                                  const uint16_t *__restrict__ UAlo,
                                                                  const uint16_t *__restrict__ Cq,
                                                                  const uint16_t *__restrict__ Clo,
                                                                  const uint16_t *__restrict__ P, int pscaled,
                                                                  const float *__restrict__ g, float *__restrict__ out,
                                                                  float *__restrict__ state,
                                                                  int Btot, int T, int K, int V, int NT, int nKG, int bpg,
                                                                  int nVT, int total) {
    extern __shared__ __align__(16) float lds_f[];   // staged c tiles, then the exchange partials
    char *const lds = reinterpret_cast<char *>(lds_f);
    float *const xbuf = reinterpret_cast<float *>(lds + XBUF);

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
    const bool has_alo = FULL && Alo != nullptr;
    const bool has_ualo = FULL && UAlo != nullptr;
    const bool has_clo = FULL && Clo != nullptr;

    const float gl = g[0];
    const float lam64 = uniform(state_lam64(gl));
    const bool tiny = lam64 < kRenorm;
    // final state (forward walk only): the last chunk's update also runs, with
    // its decay taken relative to position T-1 (Tl positions of that chunk)
    const bool want_state = !REV && state != nullptr;
    const int Tl = T - (NT - 1) * C;
    const float lamTl = uniform(__expf(gl * static_cast<float>(Tl)));
    const bool rows_here = tiny || !pscaled;   // read-out rows scaled per partial
    // row factor lam^(i+1) (lam^(64-i) reversed) of exchange row i = 8 wave
    // (uniform), and the ratio between consecutive rows
    const float xrow0 = uniform(__expf(gl * static_cast<float>(REV ? C - ROWS_PER_WAVE * wave : ROWS_PER_WAVE * wave + 1)));
    const float xstep = uniform(__expf(REV ? -gl : gl));
    // state scale after the update of walk step st, from the one after step st-1
    auto scale_after = [&](float s_prev, int st) {
        const float s = (st > 0 && !tiny && s_prev < kRenorm) ? 1.f : s_prev;
        return tiny ? 1.f : lam64 * s;
    };

    // ---- operand buffers, one batch row each (tile layouts of ulm_common.h);
    // byte offset of a tile load = 16 lane + a uniform tile offset
    const int KT16 = K / 16, KT32 = K / 32, VT32 = V / 32;
    const size_t rowA = static_cast<size_t>(2 * NT) * KT16 * kTileElems;    // R layout
    const size_t rowU = static_cast<size_t>(NT) * KT32 * 4 * kTileElems;    // Q layout, keys
    const size_t rowC = static_cast<size_t>(NT) * VT32 * 4 * kTileElems;    // Q layout, values
    const size_t rowP = static_cast<size_t>(NT) * 8 * kTileElems;           // score tiles
    const rsrc_t ra = rsrc(A_ + b * rowA, rowA * 2);
    const rsrc_t ral = rsrc((has_alo ? Alo : A_) + b * rowA, rowA * 2);
    const rsrc_t rua = rsrc(UA + b * rowU, rowU * 2);
    const rsrc_t rul = rsrc((has_ualo ? UAlo : UA) + b * rowU, rowU * 2);
    const rsrc_t rc = rsrc(Cq + b * rowC, rowC * 2);
    const rsrc_t rcl = rsrc((has_clo ? Clo : Cq) + b * rowC, rowC * 2);
    const rsrc_t rp = rsrc(P + b * rowP, rowP * 2);
    const uint32_t lane16 = static_cast<uint32_t>(lane * 16);
    // this wave's raw c tile: 32-column tile wave / 4, position quarter wave % 4
    const uint32_t c_lane = (wave < 4 || nt1) ? lane16 + wave * TB : OOB;
    // the intra matrix tiles of both row halves: this wave's own (imt) half, the
    // other out of range (zeros), so the product needs no branch; every tile
    // out of range outside key group 0
    uint32_t p_lane[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) p_lane[mt] = (intra && mt == imt) ? lane16 + (mt * 4 + iq) * TB : OOB;
    // uniform key-block offsets (bytes) into a rows and into the update operand; OOB past the group
    uint32_t a_blk[MH], u_blk[MH];
#pragma unroll
    for (int mh = 0; mh < MH; ++mh) {
        const int blk = blk0 + wave + WAVES * mh;
        a_blk[mh] = uniform(blk < blk1 ? static_cast<uint32_t>(2 * blk) * TB : OOB);
        u_blk[mh] = uniform(blk < blk1 ? static_cast<uint32_t>(4 * blk) * TB : OOB);
    }
    float *out_k = out + static_cast<size_t>(kgi) * Btot * T * V;

    auto chunk_of = [&](int st) { return REV ? NT - 1 - st : st; };
    auto c_off = [&](int n) { return uniform(static_cast<uint32_t>(n * VT32 + v0 / 32) * 4 * TB); };
    auto p_off = [&](int n) { return uniform(static_cast<uint32_t>(n * 8) * TB); };
    auto a_off = [&](int n, int mh, int hb, int mt) {
        return lane16 + uniform(static_cast<uint32_t>((2 * n + mt) * KT16) * TB) + a_blk[mh] + hb * TB;
    };
    auto load_a = [&](bf16x8 (&a)[MH][2][2], int n) {
#pragma unroll
        for (int mh = 0; mh < MH; ++mh)
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) a[mh][hb][mt] = bld(ra, a_off(n, mh, hb, mt));
    };
    // Stage this wave's c tile for walk step st: decayed by lam^(63-j) / s'
    // (lam^j / s' reversed) as bf16 hi (+ lo), and raw for the intra product.
    // Lane element e is chunk position j = 16 (wave % 4) + 8 lh + e; its decay
    // is a lane part times a uniform part, both powers of lam at most 1:
    //   forward  lam^(56 - 16 (wave%4) - 8 lh) * lam^(7-e)
    //   reversed lam^(16 (wave%4) + 8 lh)      * lam^e
    const float dlane = __expf(gl * static_cast<float>(REV ? 16 * (wave % 4) + 8 * lh : 56 - 16 * (wave % 4) - 8 * lh));
    float duni[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) duni[e] = uniform(__expf(gl * static_cast<float>(REV ? e : 7 - e)));
    // fin: the final update of the state output, position j decayed by
    // lam^(Tl-1-j) / s' (zero past the Tl positions of the chunk)
    auto stage_c = [&](bf16x8 raw, bf16x8 rlo, float s_new, bool fin) {
        const float inv_s = 1.f / s_new;
        const float dl = dlane * inv_s;
        bf16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float x = static_cast<float>(raw[e]);
            if (has_clo) x += static_cast<float>(rlo[e]);
            float f = dl * duni[e];
            if (fin) {
                const int j = 16 * (wave % 4) + 8 * lh + e;
                f = j < Tl ? __expf(gl * static_cast<float>(Tl - 1 - j)) * inv_s : 0.f;
            }
            const float y = x * f;
            hi[e] = static_cast<bf16>(y);
            lo[e] = static_cast<bf16>(y - static_cast<float>(hi[e]));
        }
        *reinterpret_cast<bf16x8 *>(lds + UB_HI + wave * TB + lane16) = hi;
        if (UBSPLIT) *reinterpret_cast<bf16x8 *>(lds + UB_LO + wave * TB + lane16) = lo;
        *reinterpret_cast<bf16x8 *>(lds + C_RAW + wave * TB + lane16) = raw;
    };

    f32x16 G[MH][2];
#pragma unroll
    for (int mh = 0; mh < MH; ++mh)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) G[mh][nt][r] = 0.f;
    float s_state = 1.f;

    // ---- prologue: step 0's c staged (visible after the first barrier),
    // step 1's read-out operand in registers
    bf16x8 a_cur[MH][2][2];
    {
        const int n0 = chunk_of(0);
        const bf16x8 raw = bld(rc, c_lane + c_off(n0));
        const bf16x8 rlo = has_clo ? bld(rcl, c_lane + c_off(n0)) : bf16x8{};
        if (NT > 1) load_a(a_cur, chunk_of(1));
        const bool fin = want_state && NT == 1;
        stage_c(raw, rlo, fin ? (tiny ? 1.f : lamTl) : scale_after(1.f, 0), fin);
    }

    // Exchange of chunk nx: wave w sums rows 8w .. 8w+7 of the eight partials
    // (lane = column), applies the read-out row factor when P carries none of
    // it, and stores. It runs in the shadow of the next chunk's read-out MFMAs.
    auto exchange = [&](int nx, float s_rd) {
        const float *rb = xbuf + lane * OPITCH + ROWS_PER_WAVE * wave;
        f32x4 acc[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) acc[k] = *reinterpret_cast<const f32x4 *>(rb + 4 * k);
#pragma unroll
        for (int w2 = 1; w2 < WAVES; ++w2)
#pragma unroll
            for (int k = 0; k < 2; ++k) acc[k] += *reinterpret_cast<const f32x4 *>(rb + w2 * XPART + 4 * k);
        if (!rows_here) {
            float f = s_rd * xrow0;
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    acc[k][m] *= f;
                    f *= xstep;
                }
        }
        // value tiles hold their 32 columns in the order perm32
        const int col = v0 + 32 * (lane / 32) + perm32(lane % 32);
        if (col < V) {
            float *dst = out_k + (static_cast<size_t>(b) * T + nx * C + ROWS_PER_WAVE * wave) * V + col;
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    if (nx * C + ROWS_PER_WAVE * wave + 4 * k + m < T) dst[static_cast<size_t>(4 * k + m) * V] = acc[k][m];
        }
    };
    float s_read_prev = 1.f;   // read-out scale of the previous step
    bf16x8 raw_c = {}, rlo_c = {};   // the next step's raw c tile, staged at the top of that step

    for (int step = 0; step < NT; ++step) {
        const int n = chunk_of(step);
        const bool readout = step > 0;
        const bool last = step + 1 == NT;
        const bool update = !last || want_state;   // the last chunk's update is read only as the final state

        // ---- rescaling of G around the read-out (rarely): renormalisation
        // (G *= s, s = 1) before, when s fell below 2^-40, or, when lam^64 itself
        // is below that, the decay G *= lam^64 after.
        if (readout && !tiny && s_state < kRenorm) {
#pragma unroll
            for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) G[mh][nt][r] *= s_state;
            s_state = 1.f;
        }

        // ---- stage this chunk's c (every wave is past the previous update)
        if (step > 0) {
            const bool fin = want_state && last;
            stage_c(raw_c, rlo_c, fin ? (tiny ? 1.f : lamTl * s_state) : scale_after(s_state, step), fin);
        }

        // ---- read-out of H = s G (both 32-row halves; G converted once per block)
        f32x16 O[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int r = 0; r < 16; ++r) O[mt][nt][r] = 0.f;
        if (readout) {
#pragma unroll
            for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    bf16x8 gop[2];
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                        for (int e = 0; e < 8; ++e) gop[nt][e] = static_cast<bf16>(G[mh][nt][8 * hb + e]);
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt) O[mt][nt] = mfma(a_cur[mh][hb][mt], gop[nt], O[mt][nt]);
                        if (has_alo) {
                            const bf16x8 aol = bld(ral, a_off(n, mh, hb, mt));
#pragma unroll
                            for (int nt = 0; nt < 2; ++nt) O[mt][nt] = mfma(aol, gop[nt], O[mt][nt]);
                        }
                    }
                    // no scheduling barrier here: the next block's bf16 conversion
                    // of G overlaps this block's MFMAs (0.5% faster, no spills)
                }
        }
        // (no scheduling barrier: the first update-operand loads may move up into
        // the read-out's tail; with the two below, 1% faster per launch, no spills)

        // ---- this chunk's update operand b_n and intra matrix tile: the first
        // half of b_n in flight during the exchange, the rest after it, as the
        // registers allow (b_n loaded on the last step too: conditional loads
        // would keep the registers they replace alive across the whole iteration)
        bf16x8 ua[MH][4];
        const uint32_t urow = uniform(static_cast<uint32_t>(n * KT32) * 4 * TB);
#pragma unroll
        for (int mh = 0; mh < MH; ++mh)
#pragma unroll
            for (int ks = 0; ks < UA_EARLY; ++ks) ua[mh][ks] = bld(rua, lane16 + urow + u_blk[mh] + ks * TB);
        phase();
        if (step > 0) exchange(chunk_of(step - 1), s_read_prev);
        phase();
        bf16x8 p_cur[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) p_cur[mt] = bld(rp, p_lane[mt] + p_off(n));
#pragma unroll
        for (int mh = 0; mh < MH; ++mh)
#pragma unroll
            for (int ks = UA_EARLY; ks < 4; ++ks) ua[mh][ks] = bld(rua, lane16 + urow + u_blk[mh] + ks * TB);
        phase();

        const float s_read = s_state;   // the state scale of this read-out
        if (readout && rows_here) {
            // the read-out rows take s lam^(i+1) (s lam^(64-i) reversed) here.
            // Row i of the lane is 32 mt + 8 q + 4 lh + m; the factors run by
            // repeated multiplication from the row with the largest one, so
            // none overflows, and the loop keeps a single factor register.
            float glv = gl;
            asm volatile("" : "+v"(glv));   // recomputed per chunk, not held across the loop
            const float lam = __expf(glv), lam4 = __expf(4.f * glv);
            float f = s_read * __expf(glv * static_cast<float>(REV ? 5 - 4 * lh : 1 + 4 * lh));
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int mt = REV ? 1 - u / 4 : u / 4, q = REV ? 3 - u % 4 : u % 4;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int m = REV ? 3 - v : v;
                    O[mt][0][4 * q + m] *= f;
                    O[mt][1][4 * q + m] *= f;
                    f *= lam;
                }
                f *= lam4;
            }
        }
        if (readout && tiny) {   // lam^64 < 2^-40 (s = 1): G decays by lam^64 after the read-out
#pragma unroll
            for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) G[mh][nt][r] *= (want_state && last) ? lamTl : lam64;
        }
        s_state = tiny ? 1.f : ((want_state && last) ? lamTl : lam64) * s_state;   // scale after this chunk's update

        // every wave has finished reducing the previous chunk's partials, and
        // this chunk's c tiles are staged
        sync_lds();
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const bf16x8 ci = lds_tile(lds, C_RAW + (nt * 4 + iq) * TB + lane16);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) O[mt][nt] = mfma(p_cur[mt], ci, O[mt][nt]);
        }
        {
            // partial of wave w: column c, row i at floats w XPART + OPITCH c + i
            float *ob = xbuf + wave * XPART + lr * OPITCH + 4 * lh;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        f32x4 x;
#pragma unroll
                        for (int m = 0; m < 4; ++m) x[m] = O[mt][nt][4 * q + m];
                        *reinterpret_cast<f32x4 *>(ob + 32 * nt * OPITCH + 32 * mt + 8 * q) = x;
                    }
        }
        // (no scheduling barrier after the partial writes, see below)

        // ---- next chunk's operands: c and P now, the read-out operand in two
        // halves inside the update, each once the update operand registers it
        // replaces are consumed
        // (on the last step they re-read this chunk, unused)
        bf16x8 a_nxt[MH][2][2];
        const int nn = !last ? chunk_of(step + 1) : n;
        raw_c = bld(rc, c_lane + c_off(nn));
        if (has_clo) rlo_c = bld(rcl, c_lane + c_off(nn));
        // (no scheduling barrier: the partial writes and these loads may
        // interleave with the update's first MFMAs)

        // ---- state update G += b_n^T c~_n (+ the lo passes); skipped on the
        // last step, whose update is never read
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (update) {
                bf16x8 ubh[2], ubl[2];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    ubh[nt] = lds_tile(lds, UB_HI + (nt * 4 + ks) * TB + lane16);
                    if (UBSPLIT) ubl[nt] = lds_tile(lds, UB_LO + (nt * 4 + ks) * TB + lane16);
                }
#pragma unroll
                for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        G[mh][nt] = mfma(ua[mh][ks], ubh[nt], G[mh][nt]);
                        if (UBSPLIT) G[mh][nt] = mfma(ua[mh][ks], ubl[nt], G[mh][nt]);
                    }
            }
            if (ks % 2 == 1) {
                phase();
                const int hb = ks / 2;
#pragma unroll
                for (int mh = 0; mh < MH; ++mh)
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) a_nxt[mh][hb][mt] = bld(ra, a_off(nn, mh, hb, mt));
                phase();
            }
        }
        if (update && has_ualo) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                bf16x8 ubh[2];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) ubh[nt] = lds_tile(lds, UB_HI + (nt * 4 + ks) * TB + lane16);
#pragma unroll
                for (int mh = 0; mh < MH; ++mh) {
                    const bf16x8 ul = bld(rul, lane16 + urow + u_blk[mh] + ks * TB);
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) G[mh][nt] = mfma(ul, ubh[nt], G[mh][nt]);
                }
            }
        }

        // every partial of this chunk is written (exchanged at the next step's
        // read-out); every wave is past this chunk's update
        sync_lds();
        s_read_prev = s_read;
#pragma unroll
        for (int mh = 0; mh < MH; ++mh)
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) a_cur[mh][hb][mt] = a_nxt[mh][hb][mt];
    }
    exchange(chunk_of(NT - 1), s_read_prev);

    // ---- final state H = s G as state[b][column][key] (fp32, (B, V, K)). In a
    // state tile, registers 8k .. 8k+7 of lane (lr, lh) hold keys 16k + 8 lh + 0..7
    // (rows in the order perm32) of column perm32(lr) of the 32-column tile.
    if (want_state) {
#pragma unroll
        for (int mh = 0; mh < MH; ++mh) {
            const int blk = blk0 + wave + WAVES * mh;
            if (blk >= blk1) continue;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int col = v0 + 32 * nt + perm32(lr);
                if (col >= V) continue;
                float *dst = state + (static_cast<size_t>(b) * V + col) * K + 32 * blk + 8 * lh;
#pragma unroll
                for (int k = 0; k < 2; ++k)
#pragma unroll
                    for (int h4 = 0; h4 < 2; ++h4) {
                        f32x4 x;
#pragma unroll
                        for (int m = 0; m < 4; ++m) x[m] = s_state * G[mh][nt][8 * k + 4 * h4 + m];
                        *reinterpret_cast<f32x4 *>(dst + 16 * k + 4 * h4) = x;
                    }
            }
        }
    }
}

template <int MH, bool REV, bool UBSPLIT, bool FULL>
int launch(const uint16_t *a, const uint16_t *alo, const uint16_t *ua, const uint16_t *ualo, const uint16_t *c,
           const uint16_t *clo, const uint16_t *P, bool pscaled, const float *g, float *out, float *state, int B, int T,
           int K, int V, int nKG, int bpg, hipStream_t s) {
    const int NT = (T + C - 1) / C;
    const int nVT = (V + VT - 1) / VT;
    const long long total = static_cast<long long>(B) * nKG * nVT;
    static bool attr_done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return check_launch("hipGetDevice");
    if (!attr_done[dev]) {
        const void *fn = reinterpret_cast<const void *>(&la_kgroup_kernel<MH, REV, UBSPLIT, FULL>);
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES) != hipSuccess)
            return check_launch("la_kgroup_kernel attribute");
        attr_done[dev] = true;
    }
    int st = la_timer_begin(s, 0);
    if (st) return st;
    la_kgroup_kernel<MH, REV, UBSPLIT, FULL><<<dim3(static_cast<unsigned>(total)), WAVES * kWave, LDS_BYTES, s>>>(
        a, alo, ua, ualo, c, clo, P, pscaled ? 1 : 0, g, out, state, B, T, K, V, NT, nKG, bpg, nVT, static_cast<int>(total));
    st = check_launch("la_kgroup_kernel");
    if (st) return st;
    return la_timer_end(s);
}

template <int MH>
int launch_mh(const uint16_t *a, const uint16_t *alo, const uint16_t *ua, const uint16_t *ualo, const uint16_t *c,
              const uint16_t *clo, const uint16_t *P, bool pscaled, const float *g, float *out, float *state, int B,
              int T, int K, int V, int nKG, int bpg, bool reverse, bool ubsplit, hipStream_t s) {
    const bool full = alo || ualo || clo;
    const int sel = (reverse ? 4 : 0) + (ubsplit ? 2 : 0) + (full ? 1 : 0);
    switch (sel) {
    case 0: return launch<MH, false, false, false>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
    case 1: return launch<MH, false, false, true>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
    case 2: return launch<MH, false, true, false>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
    case 3: return launch<MH, false, true, true>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
    case 4: return launch<MH, true, false, false>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
    case 5: return launch<MH, true, false, true>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
    case 6: return launch<MH, true, true, false>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
    default: return launch<MH, true, true, true>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, s);
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
// and c (+ clo) in the Q layout. The read-out contracts a with the state; the
// update adds ua^T c~, where c~ is c decayed and scaled in the kernel (+ the
// rounding remainder of c~ when ubsplit, + ualo^T c~). c is also the value
// operand of the intra-chunk product with P (P_lo forward or P_up reversed, of
// chunk_scores, pscaled as chunk_scores' `scaled`). alo, ualo, clo may each be null.
// out: la_kgroup_groups(K) x (B, T, V) fp32, fully written (no accumulation).
// state (forward walk only, may be null): the state after position T-1,
// sum_s lam^(T-1-s) b_s c_s^T, as fp32 (B, V, K), 16-byte aligned.
int launch_la_kgroup(const uint16_t *a, const uint16_t *alo, const uint16_t *ua, const uint16_t *ualo,
                     const uint16_t *c, const uint16_t *clo, const uint16_t *P, bool pscaled, const float *g,
                     float *out, float *state, int B, int T, int K, int V, bool reverse, bool ubsplit, hipStream_t s) {
    if (!la_kgroup_supported(B, T, K, V))
        return fail(ULM_ERR_UNSUPPORTED, "K-group kernel: B=%d T=%d K=%d V=%d unsupported", B, T, K, V);
    if (state && (reverse || reinterpret_cast<uintptr_t>(state) % 16))
        return fail(ULM_ERR_INVALID, "K-group kernel: the state output needs the forward walk and 16-byte alignment");
    const int nKG = la_kgroup_groups(K);
    const int nb = K / 32;
    const int bpg = (nb + nKG - 1) / nKG;   // <= 24 blocks, so at most 3 per wave
    const int mh = (bpg + kgrp::WAVES - 1) / kgrp::WAVES;
    switch (mh) {
    case 1:
        return kgrp::launch_mh<1>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, reverse, ubsplit, s);
    case 2:
        return kgrp::launch_mh<2>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, reverse, ubsplit, s);
    default:
        return kgrp::launch_mh<3>(a, alo, ua, ualo, c, clo, P, pscaled, g, out, state, B, T, K, V, nKG, bpg, reverse, ubsplit, s);
    }
}

}  // namespace ulm
