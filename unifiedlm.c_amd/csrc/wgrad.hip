// Weight-gradient GEMM of the block's linear layers: C = A^T B over the token
// dimension, A (K, N1) and B (K, N2) bf16 row-major, C (N1, N2) fp32, with K
// (= batch x positions) far larger than N1, N2. These are the weight
// gradients of the key, value and mu projections (model.py:64-68, the
// backward of F.linear under bf16 autocast), whose output has too few tiles
// to fill 256 CUs without splitting the contraction.
//
// Design: a workgroup owns a 256 x 256 tile of C and one of S contiguous
// ranges of K (split-K, S = 256 / tiles: one round of one workgroup per
// CU, which bounds the fp32 partial traffic); its 8 waves each hold a 64 x 128 fp32 accumulator
// (2 x 4 v_mfma_f32_32x32x16_bf16 tiles). Both operands are stored with K as
// the row index, so each 64-row k-step of A and B is staged in LDS as
// [k][column] (16-byte global loads along a row, double buffered) and read
// back with ds_read_b64_tr_b16, which hands each lane 4 consecutive k of one
// column: two reads form one MFMA operand (lane l: column l % 32, k 8(l/32) ..
// 8(l/32)+7). The S partial tiles are summed in a fixed order afterwards, so
// the result does not depend on scheduling.
#include "ulm_common.h"

namespace ulm {
namespace wg {

constexpr int TI = 256, TJ = 256;            // workgroup tile (N1 x N2)
constexpr int TK = 64;                       // k-step: rows of A and B staged per step
constexpr int DEPTH = 1;                     // k-steps whose loads are in flight ahead of the MFMAs
constexpr int kWaves = 8;                    // 4 (i) x 2 (j), each 64 x 128
constexpr int kThreads = kWaves * 64;
constexpr int PITCH = 256 + 16;              // LDS row pitch in bf16: rows 8 banks apart
constexpr int kStage = 2 * TK * PITCH;       // bf16 per LDS stage: A rows then B rows
constexpr size_t kLds = 2 * kStage * sizeof(uint16_t);
constexpr int kChunks = TK * 256 / 8 / kThreads;   // 16-byte chunks of A (and of B) per thread per step
constexpr int kCUs = 256, kXCDs = 8;         // one workgroup per CU, one round

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// One MFMA operand from a [k][column] LDS tile: column c0 + l % 32, k k0 + 8(l/32) .. +7.
__device__ __forceinline__ bf16x8 operand(const uint16_t *tile, int k0, int c0, int lane) {
    const int g = lane / 16, q = lane % 16;
    const int k = k0 + 8 * (g / 2) + q / 4, c = c0 + 16 * (g % 2) + 4 * (q % 4);
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(tile + k * PITCH + c));
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(tile + (k + 4) * PITCH + c));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

struct Staged {
    uint4 a[kChunks], b[kChunks];
};

// One workgroup per (split, tile) pair, n = S x tiles of them; part (S, N1, N2)
// fp32 (or C itself when S = 1). Workgroups go round-robin over the XCDs
// (blockIdx % 8), each with its own L2, so XCD x takes a contiguous range of
// the pairs in split-major order: the workgroups of one split, which read the
// same rows of A and B, share an L2 and walk k together. Loads run DEPTH
// k-steps ahead in register sets; the LDS holds two stages.
__global__ __launch_bounds__(kThreads, 1) void wgrad_kernel(const uint16_t *__restrict__ A,
                                                            const uint16_t *__restrict__ B,
                                                            float *__restrict__ part, int K, int N1, int N2,
                                                            int kchunk, int tiles_i, int tiles_j) {
    extern __shared__ __align__(16) uint16_t lds[];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int n = gridDim.x, x = blockIdx.x % kXCDs;
    const int pair = x * (n / kXCDs) + min(x, n % kXCDs) + blockIdx.x / kXCDs;
    const int tiles = tiles_i * tiles_j, split = pair / tiles, tile = pair % tiles;
    const int i0 = (tile / tiles_j) * TI, j0 = (tile % tiles_j) * TJ;
    const int kb = split * kchunk, ke = min(K, kb + kchunk);
    const int wi = wave / 2, wj = wave % 2;   // wave tile: rows 64 wi, columns 128 wj
    const int nsteps = (ke - kb + TK - 1) / TK;

    auto load = [&](Staged &r, int step) {
        const int k0 = kb + step * TK;
#pragma unroll
        for (int q = 0; q < kChunks; ++q) {
            const int c = tid + kThreads * q, row = c / 32, col = 8 * (c % 32);
            const int k = k0 + row;
            const bool oka = step < nsteps && k < ke && i0 + col < N1;
            const bool okb = step < nsteps && k < ke && j0 + col < N2;
            // clamped addresses, masked values: no load waits inside a branch
            const uint4 va = *reinterpret_cast<const uint4 *>(A + static_cast<size_t>(oka ? k : 0) * N1 +
                                                              (oka ? i0 + col : 0));
            const uint4 vb = *reinterpret_cast<const uint4 *>(B + static_cast<size_t>(okb ? k : 0) * N2 +
                                                              (okb ? j0 + col : 0));
            r.a[q] = oka ? va : make_uint4(0, 0, 0, 0);
            r.b[q] = okb ? vb : make_uint4(0, 0, 0, 0);
        }
    };
    auto store = [&](const Staged &r, int stage) {
        uint16_t *sa = lds + stage * kStage, *sb = sa + TK * PITCH;
#pragma unroll
        for (int q = 0; q < kChunks; ++q) {
            const int c = tid + kThreads * q, row = c / 32, col = 8 * (c % 32);
            *reinterpret_cast<uint4 *>(sa + row * PITCH + col) = r.a[q];
            *reinterpret_cast<uint4 *>(sb + row * PITCH + col) = r.b[q];
        }
    };

    f32x16 acc[2][4];
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[it][jt][r] = 0.f;

    // register set d holds the step congruent to d mod DEPTH
    Staged st[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(st[d], d);
    store(st[0], 0);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int s = s0 + d;
            if (s >= nsteps) break;
            // set d held step s, already in LDS stage s % 2: refill it with step s + DEPTH
            load(st[d], s + DEPTH);
            const uint16_t *sa = lds + (s % 2) * kStage, *sb = sa + TK * PITCH;
#pragma unroll
            for (int ks = 0; ks < TK; ks += 16) {
                bf16x8 a[2], b[4];
#pragma unroll
                for (int it = 0; it < 2; ++it) a[it] = operand(sa, ks, 64 * wi + 32 * it, lane);
#pragma unroll
                for (int jt = 0; jt < 4; ++jt) b[jt] = operand(sb, ks, 128 * wj + 32 * jt, lane);
#pragma unroll
                for (int it = 0; it < 2; ++it)
#pragma unroll
                    for (int jt = 0; jt < 4; ++jt) acc[it][jt] = mfma(a[it], b[jt], acc[it][jt]);
            }
            if (s + 1 < nsteps) store(st[(d + 1) % DEPTH], (s + 1) % 2);
            __syncthreads();
        }
    }

    // accumulator (lane l, register r) -> row 8(r/4) + 4(l/32) + r%4, column l%32
    float *out = part + static_cast<size_t>(split) * N1 * N2;
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const int j = j0 + 128 * wj + 32 * jt + lane % 32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = i0 + 64 * wi + 32 * it + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
                if (i < N1 && j < N2) out[static_cast<size_t>(i) * N2 + j] = acc[it][jt][r];
            }
        }
}

struct Plan {
    int tiles_i, tiles_j, splits, kchunk;
};

Plan plan(int K, int N1, int N2) {
    Plan p{};
    p.tiles_i = (N1 + TI - 1) / TI;
    p.tiles_j = (N2 + TJ - 1) / TJ;
    const int tiles = p.tiles_i * p.tiles_j;
    int S = std::max(1, kCUs / tiles);
    S = std::max(1, std::min(S, (K + 8 * TK - 1) / (8 * TK)));   // at least 8 k-steps per split
    p.kchunk = ((K + S - 1) / S + TK - 1) / TK * TK;
    p.splits = (K + p.kchunk - 1) / p.kchunk;
    return p;
}

}  // namespace wg

int launch_partial_reduce(const float *part, int nK, size_t n, void *out, int odt, hipStream_t s,
                          const float *resid);

}  // namespace ulm

using namespace ulm;

extern "C" size_t ulm_wgrad_workspace_bytes(int K, int N1, int N2) {
    if (K <= 0 || N1 <= 0 || N2 <= 0) return 0;
    const wg::Plan p = wg::plan(K, N1, N2);
    return p.splits > 1 ? align_up(static_cast<size_t>(p.splits) * N1 * N2 * sizeof(float), 256) : 0;
}

extern "C" int ulm_wgrad(const void *a, const void *b, float *c, int K, int N1, int N2, void *workspace,
                         size_t workspace_bytes, void *stream) {
    ULM_REQUIRE(K > 0 && N1 > 0 && N2 > 0, "ulm_wgrad: bad sizes K=%d N1=%d N2=%d", K, N1, N2);
    ULM_REQUIRE(N1 % 8 == 0 && N2 % 8 == 0, "ulm_wgrad: N1=%d and N2=%d must be multiples of 8", N1, N2);
    ULM_REQUIRE(a && b && c, "ulm_wgrad: null pointer");
    ULM_REQUIRE(reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0,
                "ulm_wgrad: A and B must be 16-byte aligned");
    const size_t need = ulm_wgrad_workspace_bytes(K, N1, N2);
    ULM_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), "ulm_wgrad: workspace of %zu bytes, need %zu",
                workspace_bytes, need);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const wg::Plan p = wg::plan(K, N1, N2);
    static bool attr_done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return check_launch("hipGetDevice");
    if (!attr_done[dev]) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(&wg::wgrad_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(wg::kLds)) != hipSuccess)
            return check_launch("wgrad_kernel attribute");
        attr_done[dev] = true;
    }
    float *part = p.splits > 1 ? static_cast<float *>(workspace) : c;
    const unsigned n = static_cast<unsigned>(p.tiles_i * p.tiles_j * p.splits);
    wg::wgrad_kernel<<<n, wg::kThreads, wg::kLds, s>>>(static_cast<const uint16_t *>(a),
                                                       static_cast<const uint16_t *>(b), part, K, N1, N2, p.kchunk,
                                                       p.tiles_i, p.tiles_j);
    ULM_TRY(check_launch("wgrad_kernel"));
    if (p.splits > 1) return launch_partial_reduce(part, p.splits, static_cast<size_t>(N1) * N2, c, ULM_F32, s, nullptr);
    return ULM_OK;
}
