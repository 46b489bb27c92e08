// Chunked causal linear attention with one scalar decay, fp32 state on chip.
//
//   o_t = sum_{s<=t} lam^(t-s) (a_t . b_s) c_s          (s >= t, time reversed, if REV)
//
// This is the `_la` building block of kernel.py:183-196; its four uses (the
// role table of docs/kernel.md:22-27) are fast = LA(q, k, v), dq = LA(dfast,
// v, k), dk = LA_rev(v, dfast, q), dv = LA_rev(k, q, dfast). Unlike `_la` the
// chunk state never goes to HBM: each workgroup keeps an fp32 tile of it in
// registers while it walks the chunks of one batch row.
//
// Per chunk n (positions 64n .. 64n+63, chunk-local index i, j):
//   O    = diag(lam^(i+1)) a H                       read of the carried state
//   O   += P c,  P_ij = [j<=i] lam^(i-j) (a_i . b_j) intra-chunk part
//   H    = lam^64 H + btilde^T c,  btilde_j = lam^(63-j) b_j
// where H (K x V) is the state carried into the chunk.
//
// Work split: a 256-thread workgroup (4 waves) owns the state tile
// H[k0:k0+128, v0:v0+256] of one batch row; wave w owns columns v0+64w ..
// v0+64w+63, i.e. 4x2 MFMA accumulator tiles of 32x32 fp32 (128 registers
// per lane). The contraction over K is split across workgroups, so each
// workgroup's O is a partial sum over its 128 keys, stored to that key tile's
// own partial plane and summed over the planes in a fixed order afterwards
// (deterministic); P is likewise the partial score over the workgroup's keys
// (P c is linear in P, so the partial products sum to the full one).
//
// MFMA: v_mfma_f32_32x32x16_bf16 (gfx950). Operand layouts, lane l,
// lr = l % 32, lh = l / 32:  A: A[lr][8 lh + e];  B: B[8 lh + e][lr];
// D: reg r -> D[8 (r/4) + 4 lh + r%4][lr]. A D tile is reused as a B operand
// for the read-out by permuting the contraction index: registers 8h..8h+7 of
// tile rows 32m.. hold rows 32m + 16h + 8(e/4) + 4lh + e%4, so the matching A
// operand takes a[i][that row] with two 8-byte LDS reads.
//
// LDS per workgroup (bf16): a and b tiles in natural layout [time][key] for
// the score and read-out operands, btilde^T [key][time] and c^T [value][time]
// for the operands that contract over time, and P [i][j].
#include "ulm_common.h"

namespace ulm {

constexpr int C = ULM_CHUNK;
constexpr int KT = 128;          // state rows (keys) per workgroup
constexpr int VT = 256;          // state columns (values) per workgroup
constexpr int WN = 64;           // state columns per wave
constexpr int LDK = KT + 8;      // row stride of the [time][key] tiles
constexpr int LDT = C + 8;       // row stride of the [*][time] tiles
constexpr int kThreads = 256;

struct LaSmem {
    uint16_t a[C][LDK];
    uint16_t b[C][LDK];
    uint16_t bt[KT][LDT];
    uint16_t ct[VT][LDT];
    uint16_t p[C][LDT];
    float lam_pow[C + 4];        // lam^0 .. lam^64
};

__device__ __forceinline__ bf16x8 lds_x8(const uint16_t *p) { return *reinterpret_cast<const bf16x8 *>(p); }
__device__ __forceinline__ bf16x4 lds_x4(const uint16_t *p) { return *reinterpret_cast<const bf16x4 *>(p); }
__device__ __forceinline__ bf16x8 cat4(bf16x4 lo, bf16x4 hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}
__device__ __forceinline__ float lo_bf(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float hi_bf(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

// One tile row pair (rows 2p, 2p+1) x 8 columns, as 2 x 16 bytes.
struct Pair8 {
    uint4 r0, r1;
};

template <bool VEC>
__device__ __forceinline__ uint4 load8(const uint16_t *__restrict__ base, size_t row_off, int col, int ncols, bool row_ok) {
    if (VEC) {
        if (!row_ok || col >= ncols) return make_uint4(0, 0, 0, 0);
        return *reinterpret_cast<const uint4 *>(base + row_off + col);
    }
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (row_ok && col + e < ncols) ? base[row_off + col + e] : 0;
    uint4 r;
    r.x = v[0] | (static_cast<uint32_t>(v[1]) << 16);
    r.y = v[2] | (static_cast<uint32_t>(v[3]) << 16);
    r.z = v[4] | (static_cast<uint32_t>(v[5]) << 16);
    r.w = v[6] | (static_cast<uint32_t>(v[7]) << 16);
    return r;
}

template <bool REV>
__device__ __forceinline__ int time_pos(int t, int T) { return REV ? T - 1 - t : t; }

template <bool REV, bool VEC>
__global__ __launch_bounds__(kThreads, 1) void la_kernel(const uint16_t *__restrict__ A_, const uint16_t *__restrict__ B_,
                                                         const uint16_t *__restrict__ C_, const float *__restrict__ g,
                                                         float *__restrict__ out, size_t plane, int T, int K, int V, int NT, int nK,
                                                         int nV, int total) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LaSmem &sm = *reinterpret_cast<LaSmem *>(smem_raw);

    // XCD-aware tile order: workgroups are dispatched round-robin over the 8
    // XCDs, so consecutive logical tiles (same batch row, same keys) are put
    // on one XCD and share its L2.
    int tile = blockIdx.x;
    if (total % 8 == 0) tile = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
    const int vt = tile % nV;
    const int kt = (tile / nV) % nK;
    const int bb = tile / (nV * nK);
    const int k0 = kt * KT, v0 = vt * VT;
    out += kt * plane;   // this key tile's partial plane (B, T, V)

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int lr = lane % 32, lh = lane / 32;

    const float gl = g[0];
    for (int e = tid; e <= C; e += kThreads) sm.lam_pow[e] = __expf(gl * static_cast<float>(e));

    const size_t rowA = static_cast<size_t>(bb) * T;

    // ---- global -> register staging of one chunk
    // a, b: 32 row pairs x 16 column groups = 512 tasks, 2 per thread.
    // c   : 32 row pairs x 32 column groups = 1024 tasks, 4 per thread.
    Pair8 ra[2], rb[2], rc[4];
    auto load_chunk = [&](int n) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int task = tid + kThreads * u;
            const int rp = task / 16, cg = task % 16;
            const int t0 = n * C + 2 * rp;
            const bool ok0 = t0 < T, ok1 = t0 + 1 < T;
            const size_t o0 = (rowA + time_pos<REV>(ok0 ? t0 : 0, T)) * K;
            const size_t o1 = (rowA + time_pos<REV>(ok1 ? t0 + 1 : 0, T)) * K;
            ra[u].r0 = load8<VEC>(A_, o0, k0 + cg * 8, K, ok0);
            ra[u].r1 = load8<VEC>(A_, o1, k0 + cg * 8, K, ok1);
            rb[u].r0 = load8<VEC>(B_, o0, k0 + cg * 8, K, ok0);
            rb[u].r1 = load8<VEC>(B_, o1, k0 + cg * 8, K, ok1);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int task = tid + kThreads * u;
            const int rp = task / 32, cg = task % 32;
            const int t0 = n * C + 2 * rp;
            const bool ok0 = t0 < T, ok1 = t0 + 1 < T;
            const size_t o0 = (rowA + time_pos<REV>(ok0 ? t0 : 0, T)) * V;
            const size_t o1 = (rowA + time_pos<REV>(ok1 ? t0 + 1 : 0, T)) * V;
            rc[u].r0 = load8<VEC>(C_, o0, v0 + cg * 8, V, ok0);
            rc[u].r1 = load8<VEC>(C_, o1, v0 + cg * 8, V, ok1);
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int task = tid + kThreads * u;
            const int rp = task / 16, cg = task % 16;
            *reinterpret_cast<uint4 *>(&sm.a[2 * rp][cg * 8]) = ra[u].r0;
            *reinterpret_cast<uint4 *>(&sm.a[2 * rp + 1][cg * 8]) = ra[u].r1;
            *reinterpret_cast<uint4 *>(&sm.b[2 * rp][cg * 8]) = rb[u].r0;
            *reinterpret_cast<uint4 *>(&sm.b[2 * rp + 1][cg * 8]) = rb[u].r1;
            // btilde^T: row j decayed by lam^(63-j)
            const float d0 = sm.lam_pow[C - 1 - 2 * rp], d1 = sm.lam_pow[C - 2 - 2 * rp];
            const uint32_t x0[4] = {rb[u].r0.x, rb[u].r0.y, rb[u].r0.z, rb[u].r0.w};
            const uint32_t x1[4] = {rb[u].r1.x, rb[u].r1.y, rb[u].r1.z, rb[u].r1.w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                *reinterpret_cast<uint32_t *>(&sm.bt[cg * 8 + 2 * h][2 * rp]) =
                    pack2(d0 * lo_bf(x0[h]), d1 * lo_bf(x1[h]));
                *reinterpret_cast<uint32_t *>(&sm.bt[cg * 8 + 2 * h + 1][2 * rp]) =
                    pack2(d0 * hi_bf(x0[h]), d1 * hi_bf(x1[h]));
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int task = tid + kThreads * u;
            const int rp = task / 32, cg = task % 32;
            const uint32_t x0[4] = {rc[u].r0.x, rc[u].r0.y, rc[u].r0.z, rc[u].r0.w};
            const uint32_t x1[4] = {rc[u].r1.x, rc[u].r1.y, rc[u].r1.z, rc[u].r1.w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                *reinterpret_cast<uint32_t *>(&sm.ct[cg * 8 + 2 * h][2 * rp]) = (x0[h] & 0xffffu) | (x1[h] << 16);
                *reinterpret_cast<uint32_t *>(&sm.ct[cg * 8 + 2 * h + 1][2 * rp]) =
                    (x0[h] >> 16) | (x1[h] & 0xffff0000u);
            }
        }
    };

    f32x16 H[KT / 32][2];
#pragma unroll
    for (int m = 0; m < KT / 32; ++m)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) H[m][nt][r] = 0.f;

    const int wcol = WN * wave;   // first state column of this wave inside the tile
    const int jt = wave >> 1, it = wave & 1;   // score tile of this wave

    load_chunk(0);
    for (int n = 0; n < NT; ++n) {
        __syncthreads();   // previous chunk done with LDS (and lam_pow written)
        store_chunk();
        if (n + 1 < NT) load_chunk(n + 1);
        __syncthreads();

        // ---- partial scores S^T[j][i] = b_j . a_i over this tile's keys -> P[i][j]
        {
            f32x16 s = {};
#pragma unroll
            for (int ks = 0; ks < KT / 16; ++ks) {
                const bf16x8 x = lds_x8(&sm.b[32 * jt + lr][16 * ks + 8 * lh]);
                const bf16x8 y = lds_x8(&sm.a[32 * it + lr][16 * ks + 8 * lh]);
                s = mfma(x, y, s);
            }
            const int i = 32 * it + lr;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int j0 = 32 * jt + 8 * rr + 4 * lh;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int lag = i - (j0 + e);
                    v[e] = lag >= 0 ? s[4 * rr + e] * sm.lam_pow[lag] : 0.f;
                }
                uint2 pk;
                pk.x = pack2(v[0], v[1]);
                pk.y = pack2(v[2], v[3]);
                *reinterpret_cast<uint2 *>(&sm.p[i][j0]) = pk;
            }
        }

        // ---- read-out of the carried state: O = diag(lam^(i+1)) a H
        f32x16 O[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int r = 0; r < 16; ++r) O[mt][nt][r] = 0.f;
        if (n > 0) {
#pragma unroll
            for (int mh = 0; mh < KT / 32; ++mh) {
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    bf16x8 hop[2];
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                        for (int e = 0; e < 8; ++e) hop[nt][e] = static_cast<bf16>(H[mh][nt][8 * hb + e]);
                    const int kc = 32 * mh + 16 * hb + 4 * lh;
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt) {
                        const uint16_t *row = &sm.a[32 * mt + lr][0];
                        const bf16x8 x = cat4(lds_x4(row + kc), lds_x4(row + kc + 8));
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt) O[mt][nt] = mfma(x, hop[nt], O[mt][nt]);
                    }
                }
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float sc = sm.lam_pow[32 * mt + 8 * (r / 4) + 4 * lh + (r % 4) + 1];
                    O[mt][0][r] *= sc;
                    O[mt][1][r] *= sc;
                }
        }
        __syncthreads();   // P complete

        // ---- intra-chunk part: O += P c
        bf16x8 cop[2][4];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) cop[nt][ks] = lds_x8(&sm.ct[wcol + 32 * nt + lr][16 * ks + 8 * lh]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const bf16x8 pp = lds_x8(&sm.p[32 * mt + lr][16 * ks + 8 * lh]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) O[mt][nt] = mfma(pp, cop[nt][ks], O[mt][nt]);
            }

        // ---- store the partial output (every position and column of the
        // plane is written by exactly one workgroup, once)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int col = v0 + wcol + 32 * nt + lr;
            if (col < V) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int t = n * C + 32 * mt + 8 * (r / 4) + 4 * lh + (r % 4);
                        if (t < T) out[(rowA + time_pos<REV>(t, T)) * V + col] = O[mt][nt][r];
                    }
            }
        }

        // ---- state update: H = lam^64 H + btilde^T c
        if (n + 1 < NT) {
            const float dC = sm.lam_pow[C];
#pragma unroll
            for (int mh = 0; mh < KT / 32; ++mh) {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) H[mh][nt][r] *= dC;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const bf16x8 x = lds_x8(&sm.bt[32 * mh + lr][16 * ks + 8 * lh]);
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) H[mh][nt] = mfma(x, cop[nt][ks], H[mh][nt]);
                }
            }
        }
    }
}

// ---- launch timer (diagnostics): HIP events around every chunked-kernel
// launch while enabled, so a benchmark can read the kernel's own average
// duration on the stream it runs on. Process-wide and not thread-safe.
namespace {
constexpr int kTimerTags = 8;   // 0: untagged, else a ULM_PRODUCT_* value
struct LaTimer {
    bool on = false;
    int cap = 0, used = 0;
    hipEvent_t *ev = nullptr;
    int *tag = nullptr;
    double tag_ms[kTimerTags] = {};   // the last stop()'s sums per tag
    int tag_n[kTimerTags] = {};
};
LaTimer g_la_timer;
bool g_la_timer_open = false;   // a begin without its end
}  // namespace

int la_timer_begin(hipStream_t s, int tag) {
    g_la_timer_open = g_la_timer.on && g_la_timer.used < g_la_timer.cap;
    if (!g_la_timer_open) return ULM_OK;
    g_la_timer.tag[g_la_timer.used] = tag >= 0 && tag < kTimerTags ? tag : 0;
    if (hipEventRecord(g_la_timer.ev[2 * g_la_timer.used], s) != hipSuccess) return check_launch("timer");
    return ULM_OK;
}

int la_timer_end(hipStream_t s) {
    if (!g_la_timer_open) return ULM_OK;
    g_la_timer_open = false;
    if (hipEventRecord(g_la_timer.ev[2 * g_la_timer.used + 1], s) != hipSuccess) return check_launch("timer");
    ++g_la_timer.used;
    return ULM_OK;
}

int launch_partial_reduce(const float *part, int nK, size_t n, void *out, int odt, hipStream_t s,
                          const float *resid);

// Key tiles of the generic kernel: the partial planes launch_la_generic needs.
int la_generic_parts(int K) { return (K + KT - 1) / KT; }

// Generic chunked kernel, any K and V: out (B, T, V) fp32 = o, fully written.
// With more than one key tile (la_generic_parts(K) > 1) the tiles' partial
// outputs go to part (la_generic_parts(K) x B x T x V fp32) and are summed
// into out in tile order.
int launch_la_generic(const uint16_t *a, const uint16_t *b, const uint16_t *c, const float *g, float *out, float *part,
                      int B, int T, int K, int V, bool reverse, hipStream_t s) {
    const int NT = (T + C - 1) / C;
    const int nK = (K + KT - 1) / KT, nV = (V + VT - 1) / VT;
    if (nK > 1 && !part) return fail(ULM_ERR_INVALID, "chunked kernel: %d key tiles need a partial buffer", nK);
    const size_t plane = static_cast<size_t>(B) * T * V;
    float *dst = nK > 1 ? part : out;
    const long long total = static_cast<long long>(B) * nK * nV;
    if (total > 0x7fffffffLL) return fail(ULM_ERR_UNSUPPORTED, "chunked kernel: grid of %lld workgroups", total);
    const bool vec = (K % 8 == 0) && (V % 8 == 0);
    const size_t lds = sizeof(LaSmem);
    const void *fn = reverse ? (vec ? reinterpret_cast<const void *>(&la_kernel<true, true>)
                                    : reinterpret_cast<const void *>(&la_kernel<true, false>))
                             : (vec ? reinterpret_cast<const void *>(&la_kernel<false, true>)
                                    : reinterpret_cast<const void *>(&la_kernel<false, false>));
    // the LDS opt-in is a host call of its own; make it once per kernel and device
    static bool attr_done[4][64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return check_launch("hipGetDevice");
    bool &done = attr_done[(reverse ? 2 : 0) + (vec ? 1 : 0)][dev];
    if (!done) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
            return check_launch("la_kernel attribute");
        done = true;
    }
    const dim3 grid(static_cast<unsigned>(total));
    const int tot = static_cast<int>(total);
    int st = la_timer_begin(s, 0);
    if (st) return st;
    if (reverse) {
        if (vec) la_kernel<true, true><<<grid, kThreads, lds, s>>>(a, b, c, g, dst, plane, T, K, V, NT, nK, nV, tot);
        else la_kernel<true, false><<<grid, kThreads, lds, s>>>(a, b, c, g, dst, plane, T, K, V, NT, nK, nV, tot);
    } else {
        if (vec) la_kernel<false, true><<<grid, kThreads, lds, s>>>(a, b, c, g, dst, plane, T, K, V, NT, nK, nV, tot);
        else la_kernel<false, false><<<grid, kThreads, lds, s>>>(a, b, c, g, dst, plane, T, K, V, NT, nK, nV, tot);
    }
    st = check_launch("la_kernel");
    if (st) return st;
    st = la_timer_end(s);
    if (st || nK == 1) return st;
    return launch_partial_reduce(part, nK, plane, out, ULM_F32, s, nullptr);
}

}  // namespace ulm

using namespace ulm;

extern "C" int ulm_la_timer_start(int max_launches) {
    ULM_REQUIRE(max_launches > 0 && max_launches <= 1 << 16, "ulm_la_timer_start: bad capacity %d", max_launches);
    if (g_la_timer.cap < max_launches) {
        int *tag = new int[max_launches];
        delete[] g_la_timer.tag;
        g_la_timer.tag = tag;
        hipEvent_t *ev = new hipEvent_t[2 * max_launches];
        for (int i = 0; i < 2 * g_la_timer.cap; ++i) ev[i] = g_la_timer.ev[i];
        for (int i = 2 * g_la_timer.cap; i < 2 * max_launches; ++i)
            // timing only: no system-scope fence, which would write the caches back
            // and invalidate them between the timed kernels
            if (hipEventCreateWithFlags(&ev[i], hipEventDisableSystemFence) != hipSuccess) {
                delete[] ev;
                return check_launch("hipEventCreate");
            }
        delete[] g_la_timer.ev;
        g_la_timer.ev = ev;
        g_la_timer.cap = max_launches;
    }
    g_la_timer.used = 0;
    g_la_timer.on = true;
    return ULM_OK;
}

extern "C" int ulm_la_timer_stop(double *total_ms, int *launches) {
    ULM_REQUIRE(total_ms && launches, "ulm_la_timer_stop: null pointer");
    g_la_timer.on = false;
    double tot = 0.0;
    for (int t = 0; t < kTimerTags; ++t) {
        g_la_timer.tag_ms[t] = 0.0;
        g_la_timer.tag_n[t] = 0;
    }
    for (int i = 0; i < g_la_timer.used; ++i) {
        if (hipEventSynchronize(g_la_timer.ev[2 * i + 1]) != hipSuccess) return check_launch("hipEventSynchronize");
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, g_la_timer.ev[2 * i], g_la_timer.ev[2 * i + 1]) != hipSuccess)
            return check_launch("hipEventElapsedTime");
        tot += ms;
        g_la_timer.tag_ms[g_la_timer.tag[i]] += ms;
        ++g_la_timer.tag_n[g_la_timer.tag[i]];
    }
    *total_ms = tot;
    *launches = g_la_timer.used;
    g_la_timer.used = 0;
    return ULM_OK;
}

extern "C" int ulm_la_timer_product(int tag, double *total_ms, int *launches) {
    ULM_REQUIRE(total_ms && launches, "ulm_la_timer_product: null pointer");
    ULM_REQUIRE(tag > 0 && tag < kTimerTags, "ulm_la_timer_product: bad product tag %d", tag);
    *total_ms = g_la_timer.tag_ms[tag];
    *launches = g_la_timer.tag_n[tag];
    return ULM_OK;
}
