// Block-pair products of the fast memory: the same sums as the chunked
// products (la_kgroup.hip), evaluated over pairs of position blocks instead of
// through a carried state. For one batch row, with lam = exp(g):
//
//   scores   P[t][s]  = lam^(t-s) (q_t . k_s)             s <= t, else 0
//   apply    fast_t   = sum_s P[t][s] v_s                  (_la's output, kernel.py:75-101)
//   dscores  dS[t][s] = lam^(t-s) (dfast_t . v_s)         s <= t, else 0
//            dg      += sum_{s<=t} (t-s) P[t][s] (dfast_t . v_s)
//   dq_f     dq_f_t   = sum_s dS[t][s] k_s                 dk_f_s = sum_t dS[t][s] q_t
//   dv       dv_s     = sum_t P[t][s] dfast_t
//
// These are the four products of the role table (docs/kernel.md:22-27) with
// the intra-chunk matrix of _la_attn_kernel (kernel.py:51-72) extended to every
// earlier block. Per token and product the state form costs 4 K V flops
// (update + read-out), this form about T (K + V) / 2: it is the cheaper one
// for sequences up to a few thousand positions at the widths of the trained
// models, and it needs no state in registers. The decay gradient is summed
// directly over the (t, s) pairs with its lag weight, so it involves no
// difference of large positional sums.
//
// Every product is a tile GEMM C[m][n] = sum_k A[m][k] B[n][k] per batch row
// on bf16 operand tiles (ulm_common.h: 32 rows x 16 contraction elements,
// 1 KB, one v_mfma_f32_32x32x16_bf16 operand per lane-ordered tile):
//
//   product  m  n  k   A                      B      contraction range
//   scores   s  t  a   k (R layout)           q (R)  all slots; tiles with s-block <= t-block
//   apply    t  d  s   P                      v (Q)  s < end of t's block
//   dscores  s  t  d   v (R)                  dO (R) all features; s-block <= t-block
//   dq_f     t  a  s   dS                     k (Q)  s < end of t's block
//   dk_f     s  a  t   dS^T                   q (Q)  t >= start of s's block
//   dv       s  d  t   P^T                    dO (Q) t >= start of s's block
//
// P, dS and their transposes are stored per batch row as bf16 tiles with rows
// t (s for the transposes) and contraction s (t) (the "P layout", the R layout
// of a Tq x Tq matrix, Tq = T padded to 128). The scores / dscores epilogue
// holds, in the MFMA accumulator, one t per lane and four consecutive s per
// register group, so each lane writes 8 contiguous bytes of a P-layout tile
// and 2-byte elements of the transpose; every product then reads its operands
// plain.
//
// Workgroup: TM x TN output tile, 4 waves (2 x 2), one wave per SIMD holding a
// (TM/2) x (TN/2) fp32 accumulator (in AGPRs at 256 x 256). Each 32-element
// k-step of A and B is copied into LDS by buffer_load ... lds (no registers),
// NSTAGE stages (3 to 5, nstage below), so the copies of the next NSTAGE - 1
// k-steps run during the MFMAs of the current one. All global loads are
// range-checked buffer loads (rows or contraction past a matrix read as zero)
// and all global stores are range-checked buffer stores. Epilogues: the
// scores and dscores (P-layout outputs, the dg pair sum), rows of a (B, T, F)
// output, the dq_f product's backward statistics (EPI_DQSTATS) and the dk_f
// product's accumulation into dr (OUT_DRADD).
#include "ulm_common.h"

#include <mutex>
#include <type_traits>

namespace ulm {

int la_timer_begin(hipStream_t s, int tag);
int la_timer_end(hipStream_t s);

namespace pair {

constexpr uint32_t TB = 1024;           // bytes per operand tile
constexpr uint32_t OOB = 0x80000000u;   // buffer offset past every range: loads return zeros
constexpr int kNT = 2;                  // buffer cache policy: non-temporal (streamed, evicted first)

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t v2u32_t __attribute__((ext_vector_type(2)));
// The 16-byte buffer builtins take and return a vector_size(16) type. Their
// values go through float ext-vectors by bit cast: elements read one by one
// from a uint ext-vector made from the load were shrunk to one dword and
// splatted by this compiler.
typedef float v4f32_t __attribute__((ext_vector_type(4)));
typedef uint32_t gv4u32_t __attribute__((__vector_size__(16)));

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ rsrc_t rsrc(const void *base, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ uint32_t uniform(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// One operand matrix of one batch row in tile layout: element (row r,
// contraction k) lies in tile (r / 32, k / 16) at byte
//   (r / 32) rt + (k / 64) ks + ((k % 64) / 16) TB + 16 (r % 32 + 32 ((k % 16) / 8)) + 2 (k % 8).
// Tiles at or past nrt row tiles or nkt contraction tiles read as zero.
struct Mat {
    const uint16_t *p;   // batch row 0
    size_t bstride;      // bytes per batch row
    uint32_t rt, ks;     // bytes between 32-row tiles and between 64-element k-steps
    int nrt, nkt;
};

enum Epi { EPI_SCORES = 0, EPI_DSCORES = 1, EPI_ROWS = 2, EPI_DQSTATS = 3 };
// EPI_ROWS output kinds: OUT % 3 = the ulm_dtype of the output, 3..5 the same
// plus an fp32 residual, OUT_DRADD the backward's dr accumulation of dk_f
constexpr int OUT_DRADD = 6;
enum KRange { K_FULL = 0, K_CAUSAL = 1, K_ANTI = 2 };
// EPI_SCORES with fewer 128 x 128 tile jobs than CUs: one workgroup per CU
// holds them all, so its stages go to depth instead (96 KB: five k-steps of
// copies in flight instead of two, against the latency of each k-step's reads)
constexpr int kScoresDeep = 1;

// LDS stages of operand copies (NSTAGE - 1 k-steps in flight): all 160 KB of LDS
// at 256 x 256 tiles (32 KB per stage); at 128 x 128, 64 KB (two workgroups
// per CU) for the products whose jobs vary in length, and 48 KB (three per
// CU) for the scores and dscores, whose equal jobs (B T^2 / 2 G^2 of them)
// would otherwise leave a short second wave
template <int TM, int EPI, int OUT = 0> constexpr int nstage() {
    if (TM == 128 && EPI == EPI_SCORES && OUT == kScoresDeep) return 6;
    return TM == 256 ? 5 : (EPI == EPI_SCORES || EPI == EPI_DSCORES || OUT == OUT_DRADD ? 3 : 4);
}
template <int TM, int EPI, int OUT = 0> constexpr int min_blocks() {
    return TM == 256 ? 1 : (nstage<TM, EPI, OUT>() == 3 ? 3 : 2);
}
// Waves per workgroup, in a (waves / 2) x 2 layout: eight for the 256 x 256
// scores (two per SIMD, one workgroup per CU), else four
template <int TM, int EPI> constexpr int waves_of() { return TM == 256 && EPI == EPI_SCORES ? 8 : 4; }

struct Args {
    Mat a, b;
    int T;
    int mt, nt;              // output tiles per batch row along m and n
    int tri;                 // only tiles with m-tile <= n-tile (TM == TN)
    int krange, nks;         // contraction range kind, k-steps of the whole contraction
    int jobs_per_row, jobs;
    const float *g;
    // EPI_SCORES / EPI_DSCORES: bf16 output in the P layout
    uint16_t *pout;          // rows t, contraction s (the P layout)
    uint16_t *pout_t;        // the transpose: rows s, contraction t
    uint16_t *pout_lo;       // EPI_SCORES: the bf16 residual P - bf16(P), P layout
    size_t p_bstride;
    uint32_t p_rt;
    const uint16_t *pin;     // EPI_DSCORES: P and its residual, for the decay gradient
    const uint16_t *pin_lo;
    double *dg_part;         // EPI_DSCORES: one sum per job
    // EPI_ROWS: (B, T, F) row-major output, rows = positions, columns = features
    void *out;
    int out_dt, F, nperm;    // nperm: B's rows are features in the order perm32 within 32-blocks
    int mperm;               // EPI_ROWS: A's rows too (an output row index in perm32 order)
    const float *resid;      // fp32 (B, T, F) added, or null
    // EPI_DQSTATS (dq_f with the backward statistics) and OUT_DRADD (dk_f into dr)
    const float *r;          // r (B, T, A) fp32, or null: r = relu(pre + bias)^2 / denom
    const void *pre;
    int pre_dt;
    const float *bias, *denom;
    const void *xq;          // the extra gradient of q: xq_kind 0 none, 1 dq_out fp32, 2 + dtype d(w q)
    int xq_kind;
    const float *nck, *w;    // n at every 64-position chunk start (B, NT, A); the prior mass
    int NT;
    float *dr;               // (B, T, A)
    float *tS, *tK, *tW;     // per (batch row, 128-position tile, slot) statistics, (B, MT, A)
    int drtile;              // OUT_DRADD: the dr accumulation (the carry formed from tS)
    int MT;
    // EPI_SCORES: bf16 tile copies of a (B, T, cp_X) tensor done by workgroups
    // past the tile jobs (cp_jobs tile_copy_bf16 jobs, cp_gx per chunk), into
    // the Q layout (cp_q) and the R layout (cp_r, or null)
    const uint16_t *cp_src;
    uint16_t *cp_q, *cp_r;
    int cp_X, cp_gx, cp_jobs;
    int tag;                 // the launch timer's product tag (ULM_PRODUCT_*)
};

// tile job -> (m-tile, n-tile) of one batch row
__device__ __forceinline__ void job_tiles(const Args &p, int j, int &mb, int &nb) {
    if (p.tri) {
        // n-tile nb holds m-tiles 0 .. nb, in rows of the lower triangle
        int n = static_cast<int>((sqrtf(8.f * j + 1.f) - 1.f) * 0.5f);
        while ((n + 1) * (n + 2) / 2 <= j) ++n;
        while (n * (n + 1) / 2 > j) --n;
        nb = n;
        mb = j - n * (n + 1) / 2;
    } else if (p.krange == K_CAUSAL) {   // work grows with the m-tile: the longest first
        mb = p.mt - 1 - j / p.nt;
        nb = j % p.nt;
    } else {                             // K_ANTI: work shrinks with the m-tile
        mb = j / p.nt;
        nb = j % p.nt;
    }
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8). Issued through the builtin, not inline asm, so that the
// compiler's own wait insertion knows which counters are already drained.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitLgkm0 = 0xC07F;   // lgkmcnt(0), nothing else

// s_waitcnt vmcnt(n) for n = 0 .. 4 k-steps of LPW copies each
template <int LPW>
__device__ __forceinline__ void wait_copies(int ksteps) {
    switch (ksteps) {
    case 0: __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); break;
    case 1: __builtin_amdgcn_s_waitcnt(waitcnt_vm(LPW)); break;
    case 2: __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * LPW)); break;
    case 3: __builtin_amdgcn_s_waitcnt(waitcnt_vm(3 * LPW)); break;
    default: __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 * LPW)); break;
    }
}

// Output element types of the row epilogue: OUT % 3 = ulm_dtype of the
// output, OUT >= 3 adds an fp32 residual; the statistics epilogue uses OUT
// for its input kinds.
template <int TM, int TN, int KT, bool TA, bool TBt, int EPI, int OUT>
__global__ __launch_bounds__((waves_of<TM, EPI>() * 64), (min_blocks<TM, EPI, OUT>())) void pair_kernel(Args p) {
    constexpr int WV = waves_of<TM, EPI>(), WM = WV / 2;   // waves, and waves along m
    constexpr int MI = TM / (32 * WM), NI = TN / 64;       // 32-row / 32-column tiles per wave
    constexpr int KS = 16 * KT;                        // contraction elements per k-step
    constexpr int A_TILES = TM / 32 * KT, B_TILES = TN / 32 * KT;   // tiles per k-step
    constexpr uint32_t STAGE = (A_TILES + B_TILES) * TB;
    constexpr int AC = A_TILES / WV, BC = B_TILES / WV;             // copies per wave per k-step
    static_assert(A_TILES % WV == 0 && B_TILES % WV == 0 && MI % 2 == 0, "copies per wave and MFMA halves");
    constexpr int LPW = AC + BC;
    constexpr int NSTAGE = nstage<TM, EPI, OUT>();
    static_assert(KT % 2 == 0 && NSTAGE >= 2 && NSTAGE - 2 <= 4, "k-step and stage count");
    extern __shared__ __align__(16) char lds[];

    if constexpr (EPI == EPI_SCORES) {
        // the tile copies ride on the workgroups past the tile jobs: the
        // scores' tiles leave CUs idle, and copies need no MFMA. Each group of
        // 4 waves takes one job with its own part of the stage memory.
        if (static_cast<int>(blockIdx.x) >= p.jobs) {
            constexpr int WV = waves_of<TM, EPI>();
            const int grp = threadIdx.x / 256;
            const int job = (static_cast<int>(blockIdx.x) - p.jobs) * (WV / 4) + grp;
            const int per_b = p.cp_gx * p.NT;
            const bool live = job < p.cp_jobs;
            const int jj = live ? job : 0;
            tile_copy_bf16(p.cp_src, p.cp_q, p.cp_r, p.T, p.cp_X, p.NT, (jj % p.cp_gx) * kCopyBlocks * ULM_CHUNK,
                           (jj % per_b) / p.cp_gx, jj / per_b, threadIdx.x % 256, live,
                           reinterpret_cast<copy_tile_t *>(lds + grp * kCopyLds));
            return;
        }
    }

    const int wave = uniform(threadIdx.x / 64);
    const int lane = threadIdx.x % 64;
    const int wm = wave / 2, wn = wave % 2;

    int logical = blockIdx.x;
    if (p.jobs % 8 == 0) logical = (blockIdx.x % 8) * (p.jobs / 8) + blockIdx.x / 8;   // XCD-local rows
    const int b = logical / p.jobs_per_row;
    int mb, nb;
    job_tiles(p, logical % p.jobs_per_row, mb, nb);
    const int m0 = mb * TM, n0 = nb * TN;

    int kb = 0, ke = p.nks;
    if (p.krange == K_CAUSAL) ke = min(p.nks, (m0 + TM) / KS);
    else if (p.krange == K_ANTI) kb = m0 / KS;

    const rsrc_t ra = rsrc(reinterpret_cast<const char *>(p.a.p) + b * p.a.bstride, p.a.bstride);
    const rsrc_t rb = rsrc(reinterpret_cast<const char *>(p.b.p) + b * p.b.bstride, p.b.bstride);
    const uint32_t lane16 = 16u * lane;
    // A tile read transposed is stored in LDS with its 16-byte chunks permuted,
    // so that the transposed reads below fall on distinct banks while every 8
    // consecutive lanes of a copy still read one 128-byte line: LDS chunk P
    // (= the copying lane) holds tile chunk c with c's bits (x j4 j3 j2 j1 j0)
    // = (P5, P4, P3 ^ t, P2 ^ P5, P1, P0), t the parity of the tile's LDS slot
    // (the same for every tile a wave copies: slots w + 4 c).
    const int tpar = wave & 1;
    const uint32_t lane_tr = 16u * (32 * ((lane >> 5) & 1) + 16 * ((lane >> 4) & 1) + 8 * (((lane >> 3) & 1) ^ tpar) +
                                    4 * (((lane >> 2) & 1) ^ ((lane >> 5) & 1)) + (lane & 3));

    // The tile copies of k-step kk into stage st. Wave w copies the tiles
    // q = w + 4 c of each operand. Plain operand: tile q is row tile q / KT at
    // contraction tile KT kk + q % KT. Transposed operand (stored rows = this
    // product's contraction): tile q is stored row tile (KS / 32) kk +
    // q / (TM / 16) at stored contraction tile m0 / 16 + q % (TM / 16) (TN and
    // n0 for B). An invalid tile gets an offset past the buffer range and reads
    // as zero. The per-copy part of each offset (and its validity) is formed
    // once; a k-step adds a part common to all copies of an operand.
    static_assert(KT == 2, "the offset split below assumes 32-element k-steps");
    // k-step part: plain operands advance 2 contraction tiles (the 64-element
    // k-steps of the layouts hold 4), transposed ones one stored row tile
    auto kstep_off = [&](const Mat &m, bool trans, int kk) -> uint32_t {
        return trans ? kk * m.rt : (kk >> 1) * m.ks + (kk & 1) * 2 * TB;
    };
    // per-copy part of copy c's offset (OOB bit set when never valid) and the
    // k-steps kk < lim for which it is valid; independent of kk, so hoisted
    auto copy_off = [&](const Mat &m, bool trans, int tile0, int TX, uint32_t lane_off, int c, int &lim) -> uint32_t {
        const int q = wave + WV * c;
        if (!trans) {
            const int rt = tile0 / 32 + q / KT;
            lim = m.nkt / KT;                            // nkt is even: kt = 2 kk + q % 2 < nkt
            return (rt * m.rt + (q % KT) * TB + lane_off) | (rt < m.nrt ? 0u : OOB);
        }
        const int skt = tile0 / 16 + q % (TX / 16);
        lim = m.nrt - q / (TX / 16);                     // stored row tile kk + q / (TX / 16) < nrt
        return (q / (TX / 16) * m.rt + (skt / 4) * m.ks + (skt % 4) * TB + lane_off) | (skt < m.nkt ? 0u : OOB);
    };
    auto issue = [&](int kk, int st) {
        char *base = lds + st * STAGE;
        const uint32_t ka = kstep_off(p.a, TA, kk), kb2 = kstep_off(p.b, TBt, kk);
        const uint32_t past = kk < ke ? 0u : OOB;   // past this tile's contraction range: zeros, no traffic
#pragma unroll
        for (int c = 0; c < AC; ++c) {
            int lim;
            const uint32_t off = copy_off(p.a, TA, m0, TM, TA ? lane_tr : lane16, c, lim);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(base + (wave + WV * c) * TB), 16,
                                                     (off + ka) | (kk < lim ? past : OOB), 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < BC; ++c) {
            int lim;
            const uint32_t off = copy_off(p.b, TBt, n0, TN, TBt ? lane_tr : lane16, c, lim);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(base + (A_TILES + wave + WV * c) * TB), 16,
                                                     (off + kb2) | (kk < lim ? past : OOB), 0, 0, 0);
        }
    };

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // transposed operand: lane (g = lane / 16, q = lane % 16) reads stored row
    // 16 (u % 2) + 8 (g / 2) + q / 4 (+ 4) of stored k-tile 2 ir + g % 2 (A) or
    // 2 jn + g % 2 (B): 8 bytes of tile chunk (that row) + 32 x, x = (q >> 1) & 1,
    // at the chunk's permuted LDS place (the caller adds the 16 (u % 2) rows)
    const int tg = lane / 16, tq = lane % 16, tx = (tq >> 1) & 1;
    const uint32_t tr_base = 16u * (32 * tx + 8 * ((tg / 2) ^ (tg % 2)) + tq / 4) + 8u * (tq & 1) + (tg % 2) * TB;
    const uint32_t tr_lo = tr_base + 64u * tx, tr_hi = tr_base + 64u * (1 - tx);
    // the MFMA operands of substep u (16 contraction elements) of stage st
    auto tr_read = [&](const char *t0) {
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(t0 + tr_lo));
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(t0 + tr_hi));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    auto frags = [&](int st, int u, bf16x8 (&af)[MI], bf16x8 (&bf)[NI]) {
        const char *sa = lds + st * STAGE;
        const char *sb = sa + A_TILES * TB;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int ir = wm * MI + i;   // 32-row tile of the workgroup tile
            if constexpr (!TA) af[i] = *reinterpret_cast<const bf16x8 *>(sa + (ir * KT + u) * TB + lane16);
            else af[i] = tr_read(sa + ((u / 2) * (TM / 16) + 2 * ir) * TB + (u % 2) * 256);
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int jn = wn * NI + j;   // 32-column tile of the workgroup tile
            if constexpr (!TBt) bf[j] = *reinterpret_cast<const bf16x8 *>(sb + (jn * KT + u) * TB + lane16);
            else bf[j] = tr_read(sb + ((u / 2) * (TN / 16) + 2 * jn) * TB + (u % 2) * 256);
        }
    };

    // Pipeline: NSTAGE - 1 k-steps of copies in flight. Before the last
    // substep of step kk each wave finishes its reads of that stage, waits for
    // the copies of step kk + 1 and meets the others at the barrier (a bare
    // s_barrier: a fence would also wait for the later steps' copies). Past the
    // barrier the first half of the last substep's MFMAs is queued before the
    // copies of step kk + NSTAGE go into step kk's stage, so the MFMA pipe
    // does not drain while they issue. Copies are issued on every step (past
    // the contraction they read zeros into a stage no one reads again), so
    // that the number of copies in flight, and the wait, never change.
    // Operands alternate between two register sets. The next substep's
    // operands are read between the two halves of this substep's MFMAs: the set
    // they overwrite was last read by MFMAs issued at least half a substep
    // earlier (overwriting the set of MFMAs still queued waits for them to
    // read it), and the reads have the second half to land.
    bf16x8 af[2][MI], bf[2][NI];
    // OUT_DRADD: the carry of dkc into this 128-position tile is C_m = D_{m+1},
    // D_j = S_j + lam^128 D_{j+1} from the last tile down (D past it 0), with S
    // the tiles' local dkc at their start. Its inputs are read ahead of the
    // first copies (the loads complete in order, so the first wait below
    // covers them; a load issued after the copies would wait for all of them)
    // and the carry is formed while those copies land; thread f < TN keeps
    // slot n0 + f's carry and S of this tile for the epilogue. Only the waves
    // holding slots load, and only the tiles mt .. MT - 1 (branches on uniform
    // values: a skipped load costs no address cycles).
    constexpr int MAXMT = 32;   // T <= 4096 on this form
    float sv[OUT == OUT_DRADD ? MAXMT : 1], carry = 0.f, s_own = 0.f, kown = 0.f, lgr = 0.f;
    __shared__ double xr[WV];
    if constexpr (OUT == OUT_DRADD) {
        const int f = n0 + static_cast<int>(threadIdx.x), mt = m0 / TM;
        const bool fok = threadIdx.x < TN && f < p.F;
        const bool loads = wave < TN / 64;
        const rsrc_t rs = rsrc(p.tS + static_cast<size_t>(b) * p.MT * p.F, 4ull * p.MT * p.F);
        const rsrc_t rk = rsrc(p.tK + static_cast<size_t>(b) * p.MT * p.F, 4ull * p.MT * p.F);
        const rsrc_t rg = rsrc(p.g, 4);
        lgr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, 0u, 0, 0));
        if (loads)
            kown = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 rk, fok ? 4u * static_cast<uint32_t>(mt * p.F + f) : OOB, 0, 0));
#pragma unroll
        for (int j = 0; j < MAXMT; ++j) {
            sv[j] = 0.f;
            if (loads && j >= mt && j < p.MT)
                sv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                      rs, fok ? 4u * static_cast<uint32_t>(j * p.F + f) : OOB, 0, 0));
        }
    }
#pragma unroll
    for (int d = 0; d < NSTAGE - 1; ++d) issue(kb + d, d);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm((NSTAGE - 2) * LPW));
    __builtin_amdgcn_s_barrier();
    if constexpr (OUT == OUT_DRADD) {
        // this job's share of the decay gradient, -K_m C_m summed over its slots
        const int mt = m0 / TM;
        const float lam = __expf(lgr);
        float lam128 = lam;
#pragma unroll
        for (int e = 0; e < 7; ++e) lam128 *= lam128;
        lam128 = fminf(lam128, 3.0e38f);   // finite, so that 0 carried past the last tile stays 0
#pragma unroll
        for (int j = MAXMT - 1; j >= 0; --j) {
            const float d2 = sv[j] + lam128 * carry;
            carry = j > mt ? d2 : carry;   // S past the last tile reads 0
        }
        s_own = sv[mt < MAXMT ? mt : 0];
        double corr = -static_cast<double>(kown) * static_cast<double>(carry);   // 0 past the slots
        corr = wave_sum(corr);
        if (lane == 0) xr[wave] = corr;
    }
    issue(kb + NSTAGE - 1, NSTAGE - 1);
    frags(0, 0, af[0], bf[0]);
    // half h of a substep's MFMAs: A tiles [h MI / 2, (h + 1) MI / 2)
    auto mfmas = [&](const bf16x8 (&a)[MI], const bf16x8 (&bb)[NI], int h) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = h * (MI / 2); i < (h + 1) * (MI / 2); ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) acc[i][j] = mfma(a[i], bb[j], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int kk = kb; kk < ke; ++kk) {
        const int st = (kk - kb) % NSTAGE;
#pragma unroll
        for (int u = 0; u + 1 < KT; ++u) {
            mfmas(af[u % 2], bf[u % 2], 0);
            frags(st, u + 1, af[(u + 1) % 2], bf[(u + 1) % 2]);
            mfmas(af[u % 2], bf[u % 2], 1);
        }
        // the last substep (its drain and barrier on every step, so that no
        // path reaches its MFMAs without them); step kk + 1's first operands
        // are read mid-substep (on the last step: stale data, unused)
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm((NSTAGE - 2) * LPW));
        __builtin_amdgcn_s_barrier();
        mfmas(af[(KT - 1) % 2], bf[(KT - 1) % 2], 0);
        issue(kk + NSTAGE, st);
        frags((st + 1) % NSTAGE, 0, af[0], bf[0]);
        mfmas(af[(KT - 1) % 2], bf[(KT - 1) % 2], 1);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));   // the trailing zero copies have landed

    // ---- epilogue. Accumulator (lane l, register r) -> row 8 (r / 4) + 4 (l / 32) + r % 4,
    // column l % 32 of its 32 x 32 tile.
    const int h = lane / 32, lc = lane % 32;
    if constexpr (EPI == EPI_SCORES || EPI == EPI_DSCORES) {
        const float g = p.g[0];
        // the transpose and the residual are optional (a prefill has no backward
        // to read them): without them their buffers have no range, and the
        // stores to them are dropped
        const rsrc_t rp = rsrc(reinterpret_cast<char *>(p.pout) + b * p.p_bstride, p.p_bstride);
        const bool want_t = p.pout_t != nullptr;
        const rsrc_t rpt = rsrc(want_t ? reinterpret_cast<char *>(p.pout_t) + b * p.p_bstride : nullptr,
                                want_t ? p.p_bstride : 0);
        // DSCORES reads P and its residual; SCORES writes the residual
        const rsrc_t rpin = rsrc(EPI == EPI_DSCORES ? reinterpret_cast<const char *>(p.pin) + b * p.p_bstride
                                                    : reinterpret_cast<const char *>(p.pout), p.p_bstride);
        const char *lo = EPI == EPI_DSCORES ? reinterpret_cast<const char *>(p.pin_lo)
                                            : reinterpret_cast<const char *>(p.pout_lo);
        const rsrc_t rplo = rsrc(lo ? lo + b * p.p_bstride : nullptr, lo ? p.p_bstride : 0);
        float dg = 0.f;
        // the transpose goes through the stage memory as bf16 [s][t] (rows
        // padded to XS elements), then out in 16-byte runs of t
        constexpr int XS = TN + 8;
        static_assert(TM * XS * 2 <= nstage<TM, EPI>() * (TM / 32 * KT + TN / 32 * KT) * TB, "transpose staging");
        uint16_t *Xt = reinterpret_cast<uint16_t *>(lds);
        __syncthreads();   // every wave past its last operand read
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int t = n0 + wn * (TN / 2) + 32 * j + lc;
            auto off_of = [&](int i, int r4) -> uint32_t {
                const int s0 = m0 + wm * (TM / WM) + 32 * i + 8 * r4 + 4 * h;
                return (t / 32) * p.p_rt + (s0 / 16) * TB + 16u * (t % 32 + 32 * ((s0 % 16) / 8)) + 2u * (s0 % 8);
            };
            // DSCORES: this column's P and residual loads all issued before its
            // first store: as far as the compiler knows a store may alias them, so
            // interleaved, each load pair waited for the stores before it
            v2u32_t pvs[MI][4], pls[MI][4];
            if constexpr (EPI == EPI_DSCORES) {
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
                        pvs[i][r4] = __builtin_amdgcn_raw_buffer_load_b64(rpin, off_of(i, r4), 0, 0);
                        pls[i][r4] = __builtin_amdgcn_raw_buffer_load_b64(rplo, off_of(i, r4), 0, 0);
                    }
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int s0 = m0 + wm * (TM / WM) + 32 * i + 8 * r4 + 4 * h;
                    const uint32_t off = off_of(i, r4);
                    float x[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int s = s0 + e;
                        const bool ok = s <= t && t < p.T;
                        x[e] = ok ? acc[i][j][4 * r4 + e] * __expf(g * static_cast<float>(t - s)) : 0.f;
                    }
                    if constexpr (EPI == EPI_DSCORES) {
                        // P to about 16 significant bits (bf16 value + bf16 residual):
                        // the lag-weighted sum cancels heavily, and one bf16 rounding
                        // of P alone moves it by about 1e-2
                        const v2u32_t pv = pvs[i][r4], pl = pls[i][r4];
                        const float pe[4] = {bf16_to_f32(pv[0] & 0xffffu) + bf16_to_f32(pl[0] & 0xffffu),
                                             bf16_to_f32(pv[0] >> 16) + bf16_to_f32(pl[0] >> 16),
                                             bf16_to_f32(pv[1] & 0xffffu) + bf16_to_f32(pl[1] & 0xffffu),
                                             bf16_to_f32(pv[1] >> 16) + bf16_to_f32(pl[1] >> 16)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int s = s0 + e;
                            if (s <= t && t < p.T) dg += static_cast<float>(t - s) * pe[e] * acc[i][j][4 * r4 + e];
                        }
                    }
                    uint16_t xb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) xb[e] = f32_to_bf16_bits(x[e]);
                    v2u32_t v;
                    v[0] = static_cast<uint32_t>(xb[0]) | (static_cast<uint32_t>(xb[1]) << 16);
                    v[1] = static_cast<uint32_t>(xb[2]) | (static_cast<uint32_t>(xb[3]) << 16);
                    __builtin_amdgcn_raw_buffer_store_b64(v, rp, off, 0, 0);
                    if constexpr (EPI == EPI_SCORES) {
                        uint16_t lb[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) lb[e] = f32_to_bf16_bits(x[e] - bf16_to_f32(xb[e]));
                        v2u32_t vl;
                        vl[0] = static_cast<uint32_t>(lb[0]) | (static_cast<uint32_t>(lb[1]) << 16);
                        vl[1] = static_cast<uint32_t>(lb[2]) | (static_cast<uint32_t>(lb[3]) << 16);
                        __builtin_amdgcn_raw_buffer_store_b64(vl, rplo, off, 0, 0);
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) Xt[(s0 - m0 + e) * XS + (t - n0)] = xb[e];
                }
        }
        __syncthreads();
        // the transpose: rows s, contraction t, 16 bytes (8 t) of one s per lane;
        // 32 consecutive lanes take the 32 rows s of one P-layout tile
#pragma unroll 4
        for (int c = threadIdx.x; want_t && c < TM * TN / 8; c += WV * 64) {
            const int sl = 32 * (c / (32 * (TN / 8))) + c % 32, t8 = (c / 32) % (TN / 8);
            const int s = m0 + sl, t = n0 + 8 * t8;
            const gv4u32_t v = *reinterpret_cast<const gv4u32_t *>(Xt + sl * XS + 8 * t8);
            __builtin_amdgcn_raw_buffer_store_b128(v, rpt, (t / 16) * TB + 16u * 32 * ((t % 16) / 8) + (s / 32) * p.p_rt + 16u * (s % 32),
                                                   0, 0);
        }
        if constexpr (EPI == EPI_DSCORES) {
            // the wave sums meet in the stage memory, once every wave is past
            // its last (unused) operand read
            double *red = reinterpret_cast<double *>(lds);
            __syncthreads();
            const double w = wave_sum(static_cast<double>(dg));
            if (lane == 0) red[wave] = w;
            __syncthreads();
            if (threadIdx.x == 0) p.dg_part[logical] = (red[0] + red[1]) + (red[2] + red[3]);
        }
    } else if constexpr (EPI == EPI_DQSTATS) {
        // The per-slot statistics of the backward for this tile's 128 positions
        // (t) and 128 slots (a), from dq_f in the accumulators (the recurrences
        // of fm_stats.hip's backward, kernel.py:142-178):
        //   c_t  = w + n_t, n from the chunk checkpoint as the forward forms it
        //   dq   = dq_f + dq_out (or + w d(w q)),  dc = -dq q / c,  q = r / c
        //   L_t  = sum_{t <= t' in this tile} lam^(t'-t) dc_t'   (dkc without
        //          the carry from later tiles)
        //   dr_t = dq_t / c_t + L_{t+1}        (dk_f and the carry are added by
        //                                       the dk_f product, OUT_DRADD)
        // and per (row, tile, slot) S = L at the tile start, K = sum_t (t - tau)
        // k_t lam^(tile end - t) (the carry's share of the decay gradient), W =
        // the tile's part of dw; the tile's own part of the decay gradient,
        // sum_t (t - tau) (dc (c - w) - k L), goes to dg_part. The k L term is
        // summed as sum_t' dc_t' V_t' with V_t' = sum_{t <= t'} (t - tau) k_t
        // lam^(t' - t), a forward scan like n.
        // Layout: four rounds of 32 slots; thread (segment j = tid / 32, slot
        // column tid % 32) holds positions 16 j .. 16 j + 15 of the tile (chunk
        // j / 4, that chunk's 16-position segment j % 4, as the forward
        // statistics split it), so that c is formed with the forward's
        // operations; segments meet through LDS.
        static_assert(TM == 128 && TN == 128 && WV * 64 == 256, "statistics epilogue: 128 x 128 tiles");
        constexpr int SEG = 16, NSEG = TM / SEG;
        // segment totals: forward (xa, xb) and reverse (ya, yb), each in two
        // copies used by alternate rounds, so that two barriers per round order
        // every write after the reads it could overwrite
        __shared__ float xa[2][NSEG][32], xb[2][NSEG][32], ya[2][NSEG][32], yb[2][NSEG][32];
        __shared__ double xg[WV];
        __shared__ float sidn[TM + 1];               // 1 / denom at positions m0 - 1 .. m0 + 127
        float *F = reinterpret_cast<float *>(lds);   // [128 t][128 a] fp32: the 64 KB of stage memory
        __syncthreads();                             // every wave past its last operand read
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int n = wn * (TN / 2) + 32 * j + lc;
            const int fl = (n & ~31) + perm32(n & 31);   // the B operand's rows are slots in perm32 order
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) F[(wm * (TM / WM) + 32 * i + 8 * (r / 4) + 4 * h + r % 4) * 128 + fl] = acc[i][j][r];
        }
        if constexpr (OUT / 2 != 0) {
            if (threadIdx.x <= TM) {
                const int t = m0 - 1 + static_cast<int>(threadIdx.x);
                sidn[threadIdx.x] = (t >= 0 && t < p.T) ? 1.f / p.denom[static_cast<size_t>(b) * p.T + t] : 0.f;
            }
        }
        __syncthreads();
        const int sj = threadIdx.x / 32, col = threadIdx.x % 32;
        const int tl0 = SEG * sj, t0 = m0 + tl0;    // this thread's first position
        const int cs = (sj / 4) * 4;                // the first segment of its chunk
        const float g = p.g[0];
        const float lam = __expf(g);
        float lam16 = 1.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) lam16 *= lam;
        const double tau = 0.5 * (p.T - 1);
        const size_t brow = static_cast<size_t>(b) * p.T;
        const bool xw = p.xq_kind >= 2;   // d(w q): dq gets w d(w q), dw gets q d(w q)
        double dg_acc = 0.0;
        // this batch row of r (or pre and denom), of the extra gradient of q and
        // of dr, through buffer loads and stores that return zeros and drop
        // writes past the range: the loads of a round issue together, with no
        // branch per element between them
        // The input kinds are compile-time (OUT = 2 IN + X4): IN 0 reads r
        // (fp32), 1 pre (fp32), 2 pre (bf16 or fp16) with denom; X4 reads the
        // extra gradient of q in 4-byte elements (or there is none: a
        // zero-length range on a valid base, whose loads return zeros without
        // touching memory), else in 2-byte ones.
        constexpr int IN = OUT / 2;
        constexpr bool X4 = OUT % 2 == 1;
        constexpr uint32_t pes = IN == 2 ? 2u : 4u, xes = X4 ? 4u : 2u;
        const uint32_t rows = static_cast<uint32_t>(p.T) * p.F;
        const rsrc_t rs_in = IN == 0 ? rsrc(p.r + brow * p.F, 4ull * rows)
                                     : rsrc(static_cast<const char *>(p.pre) + brow * p.F * pes, static_cast<size_t>(pes) * rows);
        const rsrc_t rs_xq = rsrc(p.xq_kind ? static_cast<const char *>(p.xq) + brow * p.F * xes : static_cast<const char *>(p.xq ? p.xq : p.dr),
                                  p.xq_kind ? static_cast<size_t>(xes) * rows : 0);
        const rsrc_t rs_dr = rsrc(p.dr + brow * p.F, 4ull * rows);
        // The loads of round rd + 1 are issued while round rd computes: r (or
        // pre), the extra gradient of q, n at the chunk start, w and the bias
        // of this thread's slot, each through a range-checked buffer load (no
        // branch between them). r and the extra gradient are read once and dr
        // written once: their loads and stores carry the non-temporal hint
        // (kNT), so that they do not push the operand tiles out of the caches.
        const rsrc_t rs_nck = rsrc(p.nck + static_cast<size_t>(b) * p.NT * p.F, 4ull * p.NT * p.F);
        const rsrc_t rs_w = rsrc(p.w, 4ull * p.F);
        const rsrc_t rs_bias = rsrc(p.bias ? p.bias : p.w, p.bias ? 4ull * p.F : 0);
        uint32_t rraw[SEG + 1], xraw[SEG], nraw, wraw, braw;
        auto issue = [&](int rd) {
            // Each range covers one batch row, so positions t < 0 (a negative
            // offset wraps past 2^31) and t >= T read as zeros with no test;
            // slots past A carry the out-of-range bit.
            const int a = n0 + 32 * rd + col;
            const uint32_t bad_a = static_cast<uint32_t>(a >= p.F) << 31;
            const int ac = a < p.F ? a : 0;
#pragma unroll
            for (int i = 0; i <= SEG; ++i) {
                const uint32_t off = (pes * static_cast<uint32_t>((t0 - 1 + i) * p.F + ac)) | bad_a;
                rraw[i] = pes == 4u ? __builtin_amdgcn_raw_buffer_load_b32(rs_in, off, 0, kNT)
                                    : static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(rs_in, off, 0, kNT));
            }
#pragma unroll
            for (int i = 0; i < SEG; ++i) {
                const uint32_t off = (xes * static_cast<uint32_t>((t0 + i) * p.F + ac)) | bad_a;
                xraw[i] = X4 ? __builtin_amdgcn_raw_buffer_load_b32(rs_xq, off, 0, kNT)
                             : static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(rs_xq, off, 0, kNT));
            }
            nraw = __builtin_amdgcn_raw_buffer_load_b32(rs_nck, (4u * static_cast<uint32_t>((t0 / 64) * p.F + ac)) | bad_a, 0, 0);
            wraw = __builtin_amdgcn_raw_buffer_load_b32(rs_w, (4u * static_cast<uint32_t>(ac)) | bad_a, 0, 0);
            braw = __builtin_amdgcn_raw_buffer_load_b32(rs_bias, (4u * static_cast<uint32_t>(ac)) | bad_a, 0, 0);
        };
        issue(0);
        for (int round = 0; round < 4; ++round) {
            const int al = 32 * round + col;
            const int a = n0 + al;
            const bool va = a < p.F;
            const float wa = va ? __builtin_bit_cast(float, wraw) : 1.f;
            const float ba = __builtin_bit_cast(float, braw);   // 0 past the slots and without a bias
            const float nck0 = __builtin_bit_cast(float, nraw);
            // r at positions t0 - 1 .. t0 + 15 (0 outside 0 <= t < T and past the
            // slots), formed as the forward's statistics form it
            float rv[SEG + 1];
#pragma unroll
            for (int i = 0; i <= SEG; ++i) {
                const uint16_t h16 = static_cast<uint16_t>(rraw[i]);
                float x = pes == 4u ? __builtin_bit_cast(float, rraw[i])
                                    : (p.pre_dt == ULM_BF16 ? bf16_to_f32(h16) : static_cast<float>(__builtin_bit_cast(_Float16, h16)));
                if constexpr (IN != 0) {
                    // past the slots pre and the bias read as 0; sidn is 0 outside 0 <= t < T
                    x += ba;
                    x = x > 0.f ? x : 0.f;
                    x = (x * x) * sidn[tl0 + i];
                }
                rv[i] = x;
            }
            // the extra gradient of q at t0 .. t0 + 15 (0 past T and the slots)
            float xv[SEG];
#pragma unroll
            for (int i = 0; i < SEG; ++i) {
                const uint16_t h16 = static_cast<uint16_t>(xraw[i]);
                xv[i] = X4 ? __builtin_bit_cast(float, xraw[i])
                           : (p.xq_kind == 2 + ULM_BF16 ? bf16_to_f32(h16) : static_cast<float>(__builtin_bit_cast(_Float16, h16)));
            }
            if (round < 3) issue(round + 1);
            // local scans of n (k_t = r_{t-1}) and of V from the segment start
            // (t - tau is a multiple of 1/2 below 2^12 in magnitude: exact in fp32)
            const float ft0 = static_cast<float>(static_cast<double>(t0) - tau);
            float nl[SEG], vl[SEG];
            float an = 0.f, av = 0.f;
#pragma unroll
            for (int i = 0; i < SEG; ++i) {
                const float k = t0 + i < p.T ? rv[i] : 0.f;
                an = lam * an + rv[i];
                nl[i] = an;
                av = lam * av + (ft0 + static_cast<float>(i)) * k;
                vl[i] = av;
            }
            const int par = round & 1;
            xa[par][sj][col] = an;
            xb[par][sj][col] = av;
            __syncthreads();
            // n at the segment start: the chunk checkpoint and the chunk's earlier
            // segments; V at the segment start: the tile's earlier segments
            // (all eight segments' values read at once, then the same recurrences
            // over the ones that apply, so that no step waits on its own read)
            float ea[NSEG], eb[NSEG];
#pragma unroll
            for (int m = 0; m < NSEG; ++m) {
                ea[m] = xa[par][m][col];
                eb[m] = xb[par][m][col];
            }
            float cj = nck0, vin = 0.f;
#pragma unroll
            for (int m = 0; m < NSEG; ++m) {
                const float c2 = lam16 * cj + ea[m], v2 = lam16 * vin + eb[m];
                cj = (m >= cs && m < sj) ? c2 : cj;
                vin = m < sj ? v2 : vin;
            }
            // c, q, dq, dc; dc back into F; the local parts of dw and dg. The
            // segment's share of the decay gradient, sum_i (t0 + i - tau) dc_i
            // (c_i - w) - dc_i V_i, is summed in fp32 over the 16 positions as
            // (t0 - tau) s0 + s1 - s2 and added to the double total once.
            float dqc[SEG];
            float dw_acc = 0.f, pw = lam, ecar = 0.f, s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
            for (int i = 0; i < SEG; ++i) {
                const int tl = tl0 + i;
                const float c = wa + (pw * cj + nl[i]);
                const float ic = __builtin_amdgcn_rcpf(c);
                const float q = rv[i + 1] * ic;
                const float dq = F[tl * 128 + al] + (xw ? wa * xv[i] : xv[i]);
                const float dc = -(dq * q) * ic;
                dqc[i] = dq * ic;
                F[tl * 128 + al] = dc;
                dw_acc += dc;
                if (xw) dw_acc += q * xv[i];
                ecar += pw * dc;   // sum_i lam^(i+1) dc_i: the earlier segments' V reach t0 + i as lam^(i+1) vin
                const float e = dc * (c - wa);
                s0 += e;
                s1 += static_cast<float>(i) * e;
                s2 += dc * vl[i];
                pw *= lam;
            }
            dg_acc += static_cast<double>(ft0) * static_cast<double>(s0) + static_cast<double>(s1) -
                      static_cast<double>(s2) - static_cast<double>(vin) * static_cast<double>(ecar);
            // reverse: the local scan of dc, the segments' totals through LDS
            float rl[SEG];
            float racc = 0.f;
#pragma unroll
            for (int i = SEG - 1; i >= 0; --i) {
                racc = F[(tl0 + i) * 128 + al] + lam * racc;
                rl[i] = racc;
            }
            ya[par][sj][col] = racc;
            yb[par][sj][col] = dw_acc;
            __syncthreads();
            float ra[NSEG];
#pragma unroll
            for (int m = 0; m < NSEG; ++m) ra[m] = ya[par][m][col];
            float rj = 0.f;   // L at the first position after this segment
#pragma unroll
            for (int m = NSEG - 1; m > 0; --m) {
                const float r2 = ra[m] + lam16 * rj;
                rj = m > sj ? r2 : rj;
            }
            // dr_t = dq_t / c_t + L_{t+1}, L_{t+1} = rl[i+1] + lam^(15-i) rj
            float pr = 1.f;
#pragma unroll
            for (int i = SEG - 1; i >= 0; --i) {
                const float lnext = (i + 1 < SEG ? rl[i + 1] : 0.f) + pr * rj;
                const int t = t0 + i;
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, dqc[i] + lnext), rs_dr,
                                                      (4u * static_cast<uint32_t>(t * p.F + (va ? a : 0))) |
                                                          (static_cast<uint32_t>(!va) << 31), 0, kNT);
                pr *= lam;
            }
            if (sj == NSEG - 1 && va) {
                // K = sum_t (t - tau) k_t lam^(tile end - t) = lam V at the tile's last position
                const size_t o = (static_cast<size_t>(b) * p.MT + m0 / TM) * p.F + a;
                p.tK[o] = lam * (lam16 * vin + vl[SEG - 1]);
            }
            if (sj == 0 && va) {
                float wsum = 0.f;
#pragma unroll
                for (int m = 0; m < NSEG; ++m) wsum += yb[par][m][col];
                const size_t o = (static_cast<size_t>(b) * p.MT + m0 / TM) * p.F + a;
                p.tS[o] = rl[0] + lam16 * rj;
                p.tW[o] = wsum;
            }
        }
        const double wsum = wave_sum(dg_acc);
        if (lane == 0) xg[wave] = wsum;
        __syncthreads();
        if (threadIdx.x == 0) p.dg_part[logical] = (xg[0] + xg[1]) + (xg[2] + xg[3]);
    } else if constexpr (EPI == EPI_ROWS && OUT == OUT_DRADD) {
        // dk_f rows into dr at position - 1, with the carry of dkc into this
        // 128-position tile formed before the k-loop (and, on its first row, the
        // tile's own local dkc, which the dq_f epilogue of the tile before left
        // out). The tile goes through LDS in two halves of 64 rows (the halves
        // of the waves wm = 0 and 1), so that each half-wave reads, adds and
        // writes one dr row in 16-byte runs (lane = 4 slots); every dr read of the
        // tile is issued before the first store. Half a tile of LDS (34 KB)
        // stays within the three 16 KB stages: three workgroups per CU.
        static_assert(TM == 128 && TN == 128 && WV == 4, "dr accumulation: 128 x 128 tiles");
        constexpr int FS = TN + 4;                    // padded row stride in floats
        constexpr int HR = TM / 2;                    // rows per half
        float *Fk = reinterpret_cast<float *>(lds);   // [HR][FS] dk_f; then the carry C and S per slot
        float *sC = Fk + HR * FS, *sS = sC + TN;
        __syncthreads();                              // every wave past its last operand read
        const float g = lgr;
        const int cl = lane % 32, half = lane / 32, c0 = 4 * cl;   // this lane's 4 slots of the tile
        const int f0 = n0 + c0;
        const rsrc_t ro = rsrc(static_cast<float *>(p.out) + static_cast<size_t>(b) * p.T * p.F,
                               static_cast<size_t>(p.T) * p.F * 4);
        // rows 2 (wave + 4 k) + half, k = 0 .. 15: two rows per wave per step;
        // k < 8 in the first half, k >= 8 in the second
        auto row_of = [&](int k) { return 2 * (wave + WV * k) + half; };
        auto off_of = [&](int k, int e) -> uint32_t {
            const int pos = m0 + row_of(k);
            const bool ok = pos >= 1 && pos < p.T && f0 + e < p.F;
            return ok ? 4u * (static_cast<uint32_t>(pos - 1) * p.F + f0 + e) : OOB;
        };
        constexpr int KR = TM / (2 * WV);             // rows per half-wave
        const bool vec = p.F % 4 == 0;                // 16-byte aligned runs, wholly in or out of the slots
        v4f32_t old[KR];
        if (vec) {
#pragma unroll
            for (int k = 0; k < KR; ++k)
                old[k] = __builtin_bit_cast(v4f32_t, __builtin_amdgcn_raw_buffer_load_b128(ro, off_of(k, 0), 0, kNT));
        }
        if (threadIdx.x < TN) {
            sC[threadIdx.x] = carry;   // 0 past the slots: every S read there is 0
            sS[threadIdx.x] = s_own;
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            if (wm == hh) {
#pragma unroll
                for (int j = 0; j < NI; ++j) {
                    const int n = wn * (TN / 2) + 32 * j + lc;
                    const int fl = p.nperm ? (n & ~31) + perm32(n & 31) : n;
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int r = 0; r < 16; ++r) Fk[(32 * i + 8 * (r / 4) + 4 * h + r % 4) * FS + fl] = acc[i][j][r];
                }
            }
            __syncthreads();
            if (hh == 0 && threadIdx.x == 0) p.dg_part[logical] = (xr[0] + xr[1]) + (xr[2] + xr[3]);
            float cC[4], cS[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                cC[e] = sC[c0 + e];
                cS[e] = sS[c0 + e];
            }
            auto sum = [&](int k, int e, float o) {
                const int rw = row_of(k);
                float v = o + Fk[(rw - HR * hh) * FS + c0 + e] + __expf(g * static_cast<float>(TM - rw)) * cC[e];
                if (rw == 0) v += cS[e];
                return v;
            };
            if (vec) {
#pragma unroll
                for (int k = KR / 2 * hh; k < KR / 2 * (hh + 1); ++k) {
                    v4f32_t v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = sum(k, e, old[k][e]);
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(gv4u32_t, v), ro, off_of(k, 0), 0, kNT);
                }
            } else {
#pragma unroll 2
                for (int k = KR / 2 * hh; k < KR / 2 * (hh + 1); ++k) {
                    float o4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        o4[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ro, off_of(k, e), 0, 0));
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sum(k, e, o4[e])), ro, off_of(k, e), 0, 0);
                }
            }
            if (hh == 0) __syncthreads();   // the first half's rows read before the second's overwrite them
        }
    } else {
        // rows = positions, columns = features of a (B, T, F) tensor, written
        // through a range-checked buffer of this batch row; invalid elements
        // get an offset past the range
        constexpr int DT = OUT % 3;
        constexpr uint32_t ES = DT == ULM_F32 ? 4 : 2;
        const size_t row0 = static_cast<size_t>(b) * p.T * p.F;
        const uint32_t nbytes = static_cast<uint32_t>(p.T) * p.F * ES;
        const rsrc_t ro = rsrc(static_cast<char *>(p.out) + row0 * ES, nbytes);
        const rsrc_t rr = rsrc(OUT >= 3 ? reinterpret_cast<const char *>(p.resid + row0) : static_cast<const char *>(p.out),
                               static_cast<uint32_t>(p.T) * p.F * 4);
        // element (i, j, r) of this lane, and OOB in bad when it lies outside the tensor
        auto elem = [&](int i, int j, int r, uint32_t &bad) -> uint32_t {
            const int n = n0 + wn * (TN / 2) + 32 * j + lc;
            const int f = p.nperm ? (n & ~31) + perm32(n & 31) : n;
            const int mr = m0 + wm * (TM / WM) + 32 * i + 8 * (r / 4) + 4 * h + r % 4;
            const int pos = p.mperm ? (mr & ~31) + perm32(mr & 31) : mr;
            bad = (f < p.F && pos < p.T) ? 0u : OOB;
            return static_cast<uint32_t>(pos) * p.F + f;
        };
        // Every residual load is issued before the first store: as far as the
        // compiler knows a store may alias the residual, so interleaved, each
        // load would wait for the store before it to complete.
        float res[OUT >= 3 ? MI : 1][NI][16];
        if constexpr (OUT >= 3) {
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        uint32_t bad;
                        const uint32_t el = elem(i, j, r, bad);
                        res[i][j][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                     rr, (4u * el) | bad, 0, 0));
                    }
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    uint32_t bad;
                    const uint32_t el = elem(i, j, r, bad);
                    float v = acc[i][j][r];
                    if constexpr (OUT >= 3) v += res[i][j][r];
                    if constexpr (DT == ULM_F32) {
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ro, (4u * el) | bad, 0, 0);
                    } else {
                        const uint16_t hv = DT == ULM_BF16 ? f32_to_bf16_bits(v)
                                                           : __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
                        __builtin_amdgcn_raw_buffer_store_b16(hv, ro, (2u * el) | bad, 0, 0);
                    }
                }
        }
    }
}

// dw[a] = sum over batch rows of sum over tiles (last first) of the tiles'
// dw parts, in that fixed order: blocks of 16 slots x 16 batch rows, the rows
// summed through LDS. The last block sums the n1 + n2 decay-gradient partials
// into dg in a fixed order.
constexpr int kFinalSlots = 16;
__global__ __launch_bounds__(256) void final_kernel(const float *__restrict__ tW, int MT, const double *__restrict__ p1,
                                                    int n1, const double *__restrict__ p2, int n2,
                                                    float *__restrict__ dw, float *__restrict__ dg, int B, int A) {
    __shared__ double red[4];
    __shared__ float rows[16][kFinalSlots];
    if (blockIdx.x + 1 < gridDim.x) {
        const int al = threadIdx.x % kFinalSlots, bl = threadIdx.x / kFinalSlots;
        const int a = blockIdx.x * kFinalSlots + al;
        float s = 0.f;
        for (int b0 = 0; b0 < B; b0 += 16) {
            const int b = b0 + bl;
            float row = 0.f;
            if (a < A && b < B) {
                float v[8];
                int m = MT - 1;
                for (; m >= 7; m -= 8) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) v[u] = tW[(static_cast<size_t>(b) * MT + m - u) * A + a];
#pragma unroll
                    for (int u = 0; u < 8; ++u) row += v[u];
                }
                for (; m >= 0; --m) row += tW[(static_cast<size_t>(b) * MT + m) * A + a];
            }
            rows[bl][al] = row;
            __syncthreads();
            if (bl == 0)
                for (int k = 0; k < 16 && b0 + k < B; ++k) s += rows[k][al];
            __syncthreads();
        }
        if (bl == 0 && a < A) dw[a] = s;
        return;
    }
    {
        // each thread's partials in index order; eight loads in flight at a time
        auto sum = [](const double *__restrict__ p, int n, double s) {
            int k = threadIdx.x;
            for (; k + 7 * 256 < n; k += 8 * 256) {
                double v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = p[k + 256 * u];
#pragma unroll
                for (int u = 0; u < 8; ++u) s += v[u];
            }
            for (; k < n; k += 256) s += p[k];
            return s;
        };
        double s = sum(p2, n2, sum(p1, n1, 0.0));
        s = wave_sum(s);
        if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = s;
        __syncthreads();
        if (threadIdx.x == 0) dg[0] = static_cast<float>((red[0] + red[1]) + (red[2] + red[3]));
    }
}

}  // namespace pair
}  // namespace ulm

namespace ulm {
namespace pair {

// the tile matrices of the operands (layouts of ulm_common.h)
Mat r_mat(const uint16_t *p, int NT, int F) {   // R layout: rows = positions, contraction = features
    Mat m{p, static_cast<size_t>(2 * NT) * (F / 16) * TB, static_cast<uint32_t>(F / 16) * TB, 4 * TB, 2 * NT, F / 16};
    return m;
}
Mat q_mat(const uint16_t *p, int NT, int F) {   // Q layout: rows = features (perm32), contraction = positions
    Mat m{p, static_cast<size_t>(NT) * (F / 32) * 4 * TB, 4 * TB, static_cast<uint32_t>(F / 32) * 4 * TB, F / 32, 4 * NT};
    return m;
}
Mat p_mat(const uint16_t *p, int Tq) {          // P layout: rows = t, contraction = s
    Mat m{p, static_cast<size_t>(Tq / 32) * (Tq / 16) * TB, static_cast<uint32_t>(Tq / 16) * TB, 4 * TB, Tq / 32, Tq / 16};
    return m;
}

constexpr int KT = 2;   // contraction tiles per k-step (32 elements): four 32 KB stages at 256 x 256

template <int G, bool TA, bool TBt, int EPI, int OUT>
int launch_g(Args a, int B, hipStream_t s) {
    const void *fn = reinterpret_cast<const void *>(&pair_kernel<G, G, KT, TA, TBt, EPI, OUT>);
    // the dr accumulation stages half its tile (64 x 132 fp32) and two slot rows in LDS
    constexpr int stages = nstage<G, EPI, OUT>() * (G / 32 * KT) * 2 * TB;
    constexpr int lds = OUT == OUT_DRADD && stages < (G / 2 * (G + 4) + 2 * G) * 4 ? (G / 2 * (G + 4) + 2 * G) * 4 : stages;
    static bool attr_done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return check_launch("hipGetDevice");
    if (!attr_done[dev]) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
            return check_launch("pair_kernel attribute");
        attr_done[dev] = true;
    }
    a.mt = a.mt ? a.mt : 1;
    a.jobs_per_row = a.tri ? a.mt * (a.mt + 1) / 2 : a.mt * a.nt;
    a.jobs = B * a.jobs_per_row;
    int grid = a.jobs;
    if constexpr (EPI == EPI_SCORES) {
        // tile copies: WV / 4 jobs per extra workgroup, each in its own kCopyLds of the stages
        constexpr int per_wg = waves_of<G, EPI>() / 4;
        static_assert(per_wg * kCopyLds <= lds, "tile copies fit in the stage memory");
        if (a.cp_jobs > 0) grid += (a.cp_jobs + per_wg - 1) / per_wg;
    }
    int st = la_timer_begin(s, a.tag);
    if (st) return st;
    pair_kernel<G, G, KT, TA, TBt, EPI, OUT><<<dim3(static_cast<unsigned>(grid)), waves_of<G, EPI>() * 64, lds, s>>>(a);
    st = check_launch("pair_kernel");
    if (st) return st;
    return la_timer_end(s);
}

template <bool TA, bool TBt, int EPI, int OUT>
int launch_o(const Args &a, int G, int B, hipStream_t s) {
    if constexpr (EPI == EPI_SCORES) {
        if (G == 256) return launch_g<256, TA, TBt, EPI, OUT>(a, B, s);
    }
    if (G != 128) return fail(ULM_ERR_UNSUPPORTED, "block-pair products: tile size %d", G);
    return launch_g<128, TA, TBt, EPI, OUT>(a, B, s);
}

// every product reads its operands plain (each matrix is stored in the
// orientation its consumers contract over); TA is kept for the transposed read
template <bool TA, int EPI>
int launch(const Args &a, int G, int B, hipStream_t s) {
    if constexpr (EPI == EPI_DQSTATS) {
        // OUT = 2 IN + X4 (the statistics epilogue's input kinds)
        const int in = a.r ? 0 : (a.pre_dt == ULM_F32 ? 1 : 2);
        const bool x4 = a.xq_kind == 0 || a.xq_kind == 1 || a.xq_kind == 2 + ULM_F32;
        switch (2 * in + (x4 ? 1 : 0)) {
        case 0: return launch_o<TA, false, EPI, 0>(a, G, B, s);
        case 1: return launch_o<TA, false, EPI, 1>(a, G, B, s);
        case 2: return launch_o<TA, false, EPI, 2>(a, G, B, s);
        case 3: return launch_o<TA, false, EPI, 3>(a, G, B, s);
        case 4: return launch_o<TA, false, EPI, 4>(a, G, B, s);
        default: return launch_o<TA, false, EPI, 5>(a, G, B, s);
        }
    } else if constexpr (EPI == EPI_SCORES) {
        const int tiles = B * (a.tri ? a.mt * (a.mt + 1) / 2 : a.mt * a.nt);
        if (G == 128 && tiles < 256) return launch_g<128, TA, false, EPI, kScoresDeep>(a, B, s);
        return launch_o<TA, false, EPI, 0>(a, G, B, s);
    } else if constexpr (EPI != EPI_ROWS) {
        return launch_o<TA, false, EPI, 0>(a, G, B, s);
    } else {
        if (a.drtile) return launch_o<TA, false, EPI, OUT_DRADD>(a, G, B, s);
        const int out = a.out_dt + (a.resid ? 3 : 0);
        switch (out) {
        case 0: return launch_o<TA, false, EPI, 0>(a, G, B, s);
        case 1: return launch_o<TA, false, EPI, 1>(a, G, B, s);
        case 2: return launch_o<TA, false, EPI, 2>(a, G, B, s);
        case 3: return launch_o<TA, false, EPI, 3>(a, G, B, s);
        case 4: return launch_o<TA, false, EPI, 4>(a, G, B, s);
        default: return launch_o<TA, false, EPI, 5>(a, G, B, s);
        }
    }
}

}  // namespace pair

// ---- the operator's products in block-pair form. The operand tiles are
// padded to multiples of 32 slots (A) and features (D) with zeros; the outputs
// have the natural widths.

// Block (output tile) size of the block-pair products: 128 x 128 tiles, two
// workgroups per CU (measured faster in total than 256 x 256 at the 110M shape).
int pair_block(int, int) { return 128; }
int pair_tq(int B, int T) {
    const int G = pair_block(B, T);
    return (T + G - 1) / G * G;
}
size_t pair_p_bytes(int B, int T) {
    const size_t Tq = pair_tq(B, T);
    return static_cast<size_t>(B) * Tq * Tq * 2;
}
int pair_dscore_jobs(int B, int T) {
    const int nb = pair_tq(B, T) / pair_block(B, T);
    return B * nb * (nb + 1) / 2;
}

// Flops per token of the six block-pair products, fwd + bwd, with their
// tile-granular causal ranges.
double pair_flops_per_token(int B, int T, int A, int D) {
    const double G = pair_block(B, T), nb = pair_tq(B, T) / G;
    return nb * (nb + 1) * G * G * 3.0 * (A + D) / T;
}

namespace {
// A second stream per device (default priority) and its fork / join events:
// the backward's dv product runs on it beside the dscores product, which
// leaves a quarter of the CUs' workgroup slots free
// The fork and join order work between two streams of one device: no timing,
// and no system-scope fence (a cache write-back and invalidate that only the
// host or another device would need)
constexpr unsigned kSideEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;
struct SideStream {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
int side_stream(SideStream *&out) {
    static SideStream sides[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return check_launch("hipGetDevice");
    SideStream &sd = sides[dev];
    if (!sd.s) {
        if (hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&sd.fork, kSideEventFlags) != hipSuccess ||
            hipEventCreateWithFlags(&sd.join, kSideEventFlags) != hipSuccess)
            return check_launch("side stream");
    }
    out = &sd;
    return ULM_OK;
}
}  // namespace

// P = scores(q, k) in the P layout (Tq x Tq per batch row), its transpose
// Pt and its bf16 residual Plo (P layout), then out = P v (+ resid) in out_dt
// (B, T, D). qR, kR: R layout (A); vQ: Q layout (D). With v (bf16 (B, T, D),
// D % 32 == 0, 16-byte aligned) the scores launch also writes vQ and vR (the R
// layout, or null) from it; else vQ is an input.
int launch_pair_forward(const uint16_t *qR, const uint16_t *kR, uint16_t *vQ, const float *g, uint16_t *P,
                        uint16_t *Pt, uint16_t *Plo, void *out, int out_dt, const float *resid, int B, int T, int A,
                        int D, hipStream_t s, const uint16_t *v, uint16_t *vR) {
    using namespace pair;
    const int G = pair_block(B, T), Tq = pair_tq(B, T), NT = (T + 63) / 64;
    const int Ap = (A + 31) / 32 * 32, Dp = (D + 31) / 32 * 32;   // operand tile widths
    Args a{};
    a.T = T;
    a.g = g;
    a.a = r_mat(kR, NT, Ap);
    a.b = r_mat(qR, NT, Ap);
    // the scores in 256 x 256 tiles where they tile Tq and their jobs fill at
    // least half the CUs: twice the flops per operand byte of 128 x 128 tiles,
    // whose k-steps are bound by the copies (at B = 32, T = 256 one 256 tile per
    // batch row would leave 224 of the 256 CUs idle: 34.5 us, against about
    // 12 us in three 128 tiles per row)
    const int n256 = Tq / 256;
    const int Gs = Tq % 256 == 0 && B * n256 * (n256 + 1) / 2 >= 128 ? 256 : G;
    a.mt = a.nt = Tq / Gs;
    a.tri = 1;
    a.krange = K_FULL;
    a.nks = (Ap + 16 * KT - 1) / (16 * KT);
    const Mat pm = p_mat(P, Tq);
    a.pout = P;
    a.pout_t = Pt;
    a.pout_lo = Plo;
    a.p_bstride = pm.bstride;
    a.p_rt = pm.rt;
    if (v) {
        if (D % 32 || reinterpret_cast<uintptr_t>(v) % 16)
            return fail(ULM_ERR_INVALID, "pair forward: v tile copies need D %% 32 == 0 and 16-byte rows (D=%d)", D);
        a.NT = NT;
        a.cp_src = v;
        a.cp_q = vQ;
        a.cp_r = vR;
        a.cp_X = D;
        a.cp_gx = (D + kCopyBlocks * ULM_CHUNK - 1) / (kCopyBlocks * ULM_CHUNK);
        a.cp_jobs = a.cp_gx * NT * B;
    }
    a.tag = ULM_PRODUCT_SCORES;
    ULM_TRY((launch<false, EPI_SCORES>(a, Gs, B, s)));
    Args f{};
    f.T = T;
    f.g = g;
    f.a = pm;
    f.b = q_mat(vQ, NT, Dp);
    f.mt = Tq / G;
    f.nt = (D + G - 1) / G;
    f.krange = K_CAUSAL;
    f.nks = Tq / (16 * KT);
    f.out = out;
    f.out_dt = out_dt;
    f.F = D;
    f.nperm = 1;
    f.resid = resid;
    f.tag = ULM_PRODUCT_APPLY;
    return launch<false, EPI_ROWS>(f, G, B, s);
}

// The decode state after position T-1 of every batch row, as one product over
// positions: S[b][d][a] = sum_s v[b][s][d] kd[b][s][a], with kd the keys
// decayed to T-1 (k_s lam^(T-1-s), fwd_stats' decayed Q-layout copy) and v in the
// Q layout (Dp features). Rows of both operands are features in the perm32
// order, so the row epilogue un-permutes both. S (B, D, A) fp32, overwritten.
int launch_pair_state(const uint16_t *vQ, const uint16_t *kdQ, float *S, int B, int T, int A, int D, hipStream_t s) {
    using namespace pair;
    const int G = 128, NT = (T + 63) / 64;
    const int Ap = (A + 31) / 32 * 32, Dp = (D + 31) / 32 * 32;
    Args a{};
    a.T = D;             // output rows: features d
    a.a = q_mat(vQ, NT, Dp);
    a.b = q_mat(kdQ, NT, Ap);
    a.mt = (D + G - 1) / G;
    a.nt = (A + G - 1) / G;
    a.krange = K_FULL;
    a.nks = 2 * NT;      // every position (those past T are zero in both operands)
    a.out = S;
    a.out_dt = ULM_F32;
    a.F = A;
    a.nperm = 1;
    a.mperm = 1;
    a.tag = ULM_PRODUCT_STATE;
    return launch<false, EPI_ROWS>(a, G, B, s);
}

// Bytes of the statistics workspace of launch_pair_backward: the per (batch
// row, 128-position tile, slot) S, K, W and carry arrays, the per batch row dw
// sums and the decay-gradient partials of the dq_f tiles and of the carry.
namespace {
struct PairStats {
    float *tS, *tK, *tW;
    double *dgq, *dgk;
    size_t bytes;
};
PairStats pair_stats_layout(void *base, int B, int T, int A) {
    const int G = pair_block(B, T), MT = pair_tq(B, T) / G;
    const size_t nst = static_cast<size_t>(B) * MT * A;
    const size_t jobs = static_cast<size_t>(B) * MT * ((A + G - 1) / G);
    Carver c(base);
    PairStats w{};
    w.tS = c.take<float>(nst);
    w.tK = c.take<float>(nst);
    w.tW = c.take<float>(nst);
    w.dgq = c.take<double>(2 * jobs);   // the dq_f jobs' partials, then the dk_f jobs'
    w.dgk = w.dgq + jobs;
    w.bytes = c.off;
    return w;
}
}  // namespace

size_t pair_stats_bytes(int B, int T, int A) { return pair_stats_layout(nullptr, B, T, A).bytes; }



namespace {
// The launches of launch_pair_backward after the fork: dv on the second stream
// (sd, or s when null), then dscores, dq_f with the statistics, dk_f into dr and
// the final sums on s.
int pair_backward_products(const SideStream *sd, const uint16_t *vR, const uint16_t *doR, const uint16_t *doQ,
                           const uint16_t *kQ, const uint16_t *qQ, const uint16_t *P, const uint16_t *Pt,
                           const uint16_t *Plo, const float *g, uint16_t *dS, uint16_t *dSt, double *dg_part,
                           const RSrc &rsrc_in, const void *xq, int xq_kind, const float *nck, const float *w,
                           float *dr, float *dw, float *dg, const PairStats &st, void *dv, int dv_dt, int B, int T,
                           int A, int D, hipStream_t s) {
    using namespace pair;
    const int G = pair_block(B, T), Tq = pair_tq(B, T), NT = (T + 63) / 64, MT = Tq / G;
    const int Ap = (A + 31) / 32 * 32, Dp = (D + 31) / 32 * 32;   // operand tile widths
    const Mat sm = p_mat(dS, Tq);
    {
        Args d{};
        d.T = T;
        d.g = g;
        d.mt = MT;
        d.nks = Tq / (16 * KT);
        d.nperm = 1;
        d.krange = K_ANTI;
        d.a = p_mat(Pt, Tq);
        d.b = q_mat(doQ, NT, Dp);
        d.nt = (D + G - 1) / G;
        d.out = dv;
        d.out_dt = dv_dt;
        d.F = D;
        d.tag = ULM_PRODUCT_DV;
        ULM_TRY((launch<false, EPI_ROWS>(d, G, B, sd ? sd->s : s)));
    }
    Args a{};
    a.T = T;
    a.g = g;
    a.a = r_mat(vR, NT, Dp);
    a.b = r_mat(doR, NT, Dp);
    a.mt = a.nt = MT;
    a.tri = 1;
    a.krange = K_FULL;
    a.nks = (Dp + 16 * KT - 1) / (16 * KT);
    a.pout = dS;
    a.pout_t = dSt;
    a.p_bstride = sm.bstride;
    a.p_rt = sm.rt;
    a.pin = P;
    a.pin_lo = Plo;
    a.dg_part = dg_part;
    a.tag = ULM_PRODUCT_DSCORES;
    ULM_TRY((launch<false, EPI_DSCORES>(a, G, B, s)));
    Args r{};
    r.T = T;
    r.g = g;
    r.mt = MT;
    r.nks = Tq / (16 * KT);
    r.nperm = 1;
    r.F = A;
    r.r = rsrc_in.r;
    r.pre = rsrc_in.pre;
    r.pre_dt = rsrc_in.pre_dt;
    r.bias = rsrc_in.bias;
    r.denom = rsrc_in.denom;
    r.xq = xq;
    r.xq_kind = xq_kind;
    r.nck = nck;
    r.w = w;
    r.NT = NT;
    r.dr = dr;
    r.tS = st.tS;
    r.tK = st.tK;
    r.tW = st.tW;
    r.MT = MT;
    // dq_f = dS k, and the statistics
    r.a = sm;
    r.b = q_mat(kQ, NT, Ap);
    r.nt = (A + G - 1) / G;
    r.krange = K_CAUSAL;
    r.dg_part = st.dgq;
    r.tag = ULM_PRODUCT_DQSTATS;
    ULM_TRY((launch<false, EPI_DQSTATS>(r, G, B, s)));
    // dk_f = dS^T q (rows s of dSt, contraction t >= the start of s's block), into dr
    // with the carry between tiles, which its epilogue forms from the tiles' S
    r.a = p_mat(dSt, Tq);
    r.b = q_mat(qQ, NT, Ap);
    r.krange = K_ANTI;
    r.out = dr;
    r.out_dt = ULM_F32;
    r.drtile = 1;
    r.dg_part = st.dgk;
    r.tag = ULM_PRODUCT_DKDR;
    ULM_TRY((launch<false, EPI_ROWS>(r, G, B, s)));
    const int jobs = B * MT * ((A + G - 1) / G);
    pair::final_kernel<<<(A + pair::kFinalSlots - 1) / pair::kFinalSlots + 1, 256, 0, s>>>(
        st.tW, MT, st.dgq, 2 * jobs, dg_part, pair_dscore_jobs(B, T), dw, dg, B, A);
    return check_launch("final_kernel");
}
}  // namespace

// The backward: dv = P^T dfast in dv_dt (B, T, D), on the device's second
// stream (forked from s and joined back into s before the return, so that work
// later on s is ordered after it); dS = dscores(dfast, v) and its transpose dSt
// with the pair part of the decay gradient; dq_f = dS k with the per-slot
// statistics in its epilogue (dr without dk_f and the carry; the tile
// statistics); dk_f = dS^T q added into dr with the carry of dkc between
// tiles, formed in that product; dw (A,) and dg (1,) reduced in a fixed order.
// Calls from several host threads enqueue one at a time: the fork and join
// events are shared. vR, doR: R
// layout (D); kQ, qQ: Q layout (A); doQ: Q layout (D); P, Pt, Plo from the
// forward. r: the read addresses (or their address inputs); xq / xq_kind: the
// extra gradient of q (0 none, 1 dq_out fp32, 2 + dtype d(w q)); nck: the
// forward's chunk checkpoints; ws: pair_stats_bytes(B, T, A) bytes.
int launch_pair_backward(const uint16_t *vR, const uint16_t *doR, const uint16_t *doQ, const uint16_t *kQ,
                         const uint16_t *qQ, const uint16_t *P, const uint16_t *Pt, const uint16_t *Plo,
                         const float *g, uint16_t *dS, uint16_t *dSt, double *dg_part, const RSrc &rsrc_in,
                         const void *xq, int xq_kind, const float *nck, const float *w, float *dr, float *dw,
                         float *dg, void *ws, void *dv, int dv_dt, int B, int T, int A, int D, hipStream_t s) {
    const int Tq = pair_tq(B, T), MT = Tq / pair_block(B, T);
    const PairStats st = pair_stats_layout(ws, B, T, A);
    if (MT > 32) return fail(ULM_ERR_UNSUPPORTED, "block-pair backward: %d position tiles (at most 32)", MT);
    // dv = P^T dfast on the second stream, beside dscores (joined at the end),
    // where its work outweighs the fork and join: each event between two
    // dependent kernels costs several microseconds of gap
    static std::mutex side_mu;
    const std::lock_guard<std::mutex> lock(side_mu);
    SideStream *sd = nullptr;
    if (static_cast<double>(B) * Tq * Tq * D >= 2e9) {
        ULM_TRY(side_stream(sd));
        if (hipEventRecord(sd->fork, s) != hipSuccess || hipStreamWaitEvent(sd->s, sd->fork, 0) != hipSuccess)
            return check_launch("side stream fork");
    }
    // From the fork on, every return joins the second stream back into s, the
    // error returns included: the caller frees the workspace (and may reuse dv)
    // in stream order on s once this returns, so s must not run ahead of dv.
    const int rc = pair_backward_products(sd, vR, doR, doQ, kQ, qQ, P, Pt, Plo, g, dS, dSt, dg_part, rsrc_in, xq,
                                          xq_kind, nck, w, dr, dw, dg, st, dv, dv_dt, B, T, A, D, s);
    if (sd && (hipEventRecord(sd->join, sd->s) != hipSuccess || hipStreamWaitEvent(s, sd->join, 0) != hipSuccess)) {
        const int jrc = check_launch("side stream join");
        return rc != ULM_OK ? rc : jrc;
    }
    return rc;
}

}  // namespace ulm
