// The fused fast-memory operator: forward and backward composites behind the
// C ABI (UnifiedMemory.forward / backward, kernel.py:202-233) and the bare
// chunked product ulm_la (`_la`, kernel.py:183-196).
//
// The four products follow the role table of docs/kernel.md:22-27:
//   fast = LA(q, k, v)          dq_f = LA(dfast, v, k)
//   dk_f = LA_rev(v, dfast, q)  dv   = LA_rev(k, q, dfast)
// and are evaluated in one of three forms (train_path below):
//  * block-pair form (pair.hip), sequences up to 4096 positions: the scores
//    P = (q k^T) o decay and dS = (dfast v^T) o decay as tile GEMMs, the
//    products as GEMMs over them, the decay gradient's pair part summed over
//    the (t, s) pairs. Saved: qQ, kQ (Q layout), vR (R layout), P, its
//    transpose and its bf16 residual, n_ckpt.
//  * chunked state form (la_kgroup.hip), A and D multiples of 32: operands are
//    the tiled copies of ulm_common.h, the read-out operand a in the R layout,
//    the update operands and the raw c of the intra-chunk product in the Q
//    layout, the intra-chunk matrices from chunk_scores. The reversed products
//    walk the forward chunks backwards, so one tiled copy per tensor serves
//    both directions and the score tiles pair up: P_dv = P_fwd^T, P_dk =
//    P_dq^T. The decay of the state update is applied in the kernel to c, the
//    value operand. The products behind the d/dg identity (dq and dk) add the
//    bf16 rounding remainder of the decayed c as a second update pass. When v
//    or dfast arrive in fp32 (or fp16), every operand made from them is also
//    carried as bf16 hi + lo, so both sides of the identity see the same
//    full-precision v and dfast. Saved: qR, kR, qQ, kQ (B, NT, 64 A) bf16
//    tiles; vR, vQ (+ their remainders) (B, NT, 64 D); P_dv (B, NT, 64, 64)
//    bf16 tiles; n_ckpt (B, NT, A) fp32.
//  * generic kernel (fm_chunk.hip), any widths, on natural bf16 copies of q,
//    k and v: the widths off the 32 grid past 4096 positions.
// The tiled copies are pad32(A) slots and pad32(D) features wide, the padding
// zero, so widths off the 32 grid run the pair form (and the chunked prefill)
// exactly. Every reduction runs in a fixed order: results are bitwise
// reproducible.
#include "ulm_common.h"

#include <stdlib.h>

#include <algorithm>

namespace ulm {

// fm_chunk.hip
int la_generic_parts(int K);
int launch_la_generic(const uint16_t *a, const uint16_t *b, const uint16_t *c, const float *g, float *out, float *part,
                      int B, int T, int K, int V, bool reverse, hipStream_t s);
// la_kgroup.hip
int la_kgroup_groups(int K);
bool la_kgroup_supported(int B, int T, int K, int V);
int launch_la_kgroup(const uint16_t *a, const uint16_t *alo, const uint16_t *ua, const uint16_t *ualo,
                     const uint16_t *c, const uint16_t *clo, const uint16_t *P, bool pscaled, const float *g,
                     float *out, float *state, int B, int T, int K, int V, bool reverse, bool ubsplit, hipStream_t s);
// fm_chunks.hip
int launch_chunk_transpose(const void *src, int src_dt, uint16_t *raw, uint16_t *raw_lo, uint16_t *xr,
                           uint16_t *xr_lo, int B, int T, int X, hipStream_t s, int XL = 0);
int launch_chunk_scores(const uint16_t *aR, const uint16_t *aL, const uint16_t *bR, const uint16_t *bL, const float *g,
                        uint16_t *Plo, uint16_t *Pup, int B, int T, int K, bool scaled, hipStream_t s);
int launch_partial_reduce(const float *part, int nK, size_t n, void *out, int odt, hipStream_t s,
                          const float *resid = nullptr);
int launch_unpad_sum(const float *part, int nK, int B, int R, int Rp, int F, int Fp, void *out, int odt, hipStream_t s,
                     const float *resid);
// fm_stats.hip
int launch_fwd_stats(const RSrc &src, const float *w, const float *g, float *q, uint16_t *q16n, uint16_t *k16n,
                     uint16_t *qR, uint16_t *kR, uint16_t *qQ, uint16_t *kQ, float *nck, float *c_last, int B, int T,
                     int A, hipStream_t s, void *qw = nullptr, int qw_dt = ULM_BF16, int AL = 0,
                     float *segtot = nullptr, int kq_decay = 0);
size_t fwd_stats_segtot_bytes(int B, int T, int A);
size_t bwd_stats_partial_bytes(int B, int T, int A);
int launch_bwd_stats(const float *dqf, const float *dqo, const RSrc &src, const float *nck,
                     const float *w, const float *g, const float *dkf, float *dr, float *dw, float *dg, void *part,
                     int B, int T, int A, hipStream_t s, const void *dqw = nullptr, int dqw_dt = ULM_BF16,
                     const double *dg_extra = nullptr, int nextra = 0);
// pair.hip
int pair_tq(int B, int T);
size_t pair_p_bytes(int B, int T);
int pair_dscore_jobs(int B, int T);
double pair_flops_per_token(int B, int T, int A, int D);
int launch_pair_forward(const uint16_t *qR, const uint16_t *kR, uint16_t *vQ, const float *g, uint16_t *P,
                        uint16_t *Pt, uint16_t *Plo, void *out, int out_dt, const float *resid, int B, int T, int A,
                        int D, hipStream_t s, const uint16_t *v, uint16_t *vR);
size_t pair_stats_bytes(int B, int T, int A);
int launch_pair_state(const uint16_t *vQ, const uint16_t *kdQ, float *S, int B, int T, int A, int D, hipStream_t s);
int launch_pair_backward(const uint16_t *vR, const uint16_t *doR, const uint16_t *doQ, const uint16_t *kQ,
                         const uint16_t *qQ, const uint16_t *P, const uint16_t *Pt, const uint16_t *Plo,
                         const float *g, uint16_t *dS, uint16_t *dSt, double *dg_part, const RSrc &r,
                         const void *xq, int xq_kind, const float *nck, const float *w, float *dr, float *dw,
                         float *dg, void *ws, void *dv, int dv_dt, int B, int T, int A, int D, hipStream_t s);

namespace {

size_t nt_of(int T) { return static_cast<size_t>((T + ULM_CHUNK - 1) / ULM_CHUNK); }

// both products of the operator (K = A, V = D and K = D, V = A) on the K-group kernel
bool fm_aligned(int B, int T, int A, int D) {
    return la_kgroup_supported(B, T, A, D) && la_kgroup_supported(B, T, D, A);
}

int pad32(int x) { return (x + 31) / 32 * 32; }

// How the training entries evaluate the products: the chunked state form
// (K-group kernel, A and D multiples of 32), the block-pair form (pair.hip,
// any A and D: its operand tiles are padded to multiples of 32 with zero slots
// and features, which add nothing to any product) or the generic kernel
// (fm_chunk.hip; widths off the 32 grid past 4096 positions). For aligned
// widths the cheaper of the first two serves: the pair form costs about
// T (A + D) flops per token and product, the state form 4 A D, so the pair form
// serves sequences up to a few thousand positions. ULM_FM_PATH=chunked, =pair
// or =generic in the environment forces one where it applies (it must not
// change between a forward and its backward).
enum Path { PATH_GENERIC = 0, PATH_CHUNKED = 1, PATH_PAIR = 2 };

bool pair_supported(int B, int T, int A, int D) { return T <= 4096 && fm_aligned(B, T, pad32(A), pad32(D)); }

// Whether a form can evaluate this shape at all.
bool path_supported(Path p, int B, int T, int A, int D) {
    return p == PATH_GENERIC || (p == PATH_PAIR && pair_supported(B, T, A, D)) ||
           (p == PATH_CHUNKED && fm_aligned(B, T, A, D));
}

Path train_path(int B, int T, int A, int D) {
    const char *env = getenv("ULM_FM_PATH");
    if (env && env[0] == 'g') return PATH_GENERIC;
    const bool pair_ok = pair_supported(B, T, A, D);
    // the pair form's flops and its saved scores (6 B Tq^2 bytes) grow with T.
    // Off the 32 grid the alternative is the generic kernel (natural bf16
    // copies, no scores saved), which runs its flops at a fraction of the pair
    // products' rate and whose decay gradient goes through the positional
    // identity (bf16 operands move it further): it serves sequences past 2048
    // positions where the pair form needs twice the state form's flops (at
    // the reference's 15M widths, A = 712 and D = 288, from about 2400
    // positions on)
    const double chunked = 16.0 * A * D + 8.0 * ULM_CHUNK * (A + D);
    const double pair = pair_flops_per_token(B, T, A, D);
    if (!fm_aligned(B, T, A, D)) {
        if (env && env[0] == 'p' && pair_ok) return PATH_PAIR;
        return pair_ok && (T <= 2048 || pair < 2.0 * chunked) ? PATH_PAIR : PATH_GENERIC;
    }
    if (env && env[0] == 'c') return PATH_CHUNKED;
    if (!pair_ok) return PATH_CHUNKED;
    if (env && env[0] == 'p') return PATH_PAIR;
    return pair < 0.8 * chunked ? PATH_PAIR : PATH_CHUNKED;
}

// The form of a prefill, a forward that also emits the decode state after
// position T-1: the chunked state form (the state is its walk's end), or the
// block-pair products for the output plus the state as one product over
// positions (the keys decayed to T-1), where those need fewer flops per token:
// the scores and the apply (a third of the pair form's six products) plus
// 2 A D for the state, against 4 A D + 2 C (A + D) for the state form's
// forward. At the 110M widths that is up to about 768 positions.
Path prefill_path(int B, int T, int A, int D) {
    const char *env = getenv("ULM_FM_PATH");
    const bool pair_ok = pair_supported(B, T, A, D);
    if (env && env[0] == 'c') return PATH_CHUNKED;
    if (!pair_ok) return PATH_CHUNKED;
    if (env && env[0] == 'p') return PATH_PAIR;
    const double pair = pair_flops_per_token(B, T, A, D) / 3.0 + 2.0 * A * D;
    const double chunked = 4.0 * A * D + 2.0 * ULM_CHUNK * (A + D);
    return pair < 0.8 * chunked ? PATH_PAIR : PATH_CHUNKED;
}

struct Saved {
    uint16_t *q16n, *k16n, *v16n;                                     // generic path
    uint16_t *qR, *kR, *qQ, *kQ, *vR, *vRl, *vQ, *vQl, *Pdv;   // K-group path (pair: qQ, kQ, vR)
    uint16_t *P, *Pt, *Plo;   // pair path: the scores, their transpose and their bf16 residual
    float *nck;
    size_t bytes;
};

// The tiled operand copies (R and Q layouts) of the pair and chunked paths
// are pad32(A) slots and pad32(D) features wide.
Saved saved_layout(void *base, int B, int T, int A, int D, int v_dtype, Path path) {
    const size_t NT = nt_of(T);
    const size_t na = static_cast<size_t>(B) * T * A, ta = B * NT * 64 * pad32(A), td = B * NT * 64 * pad32(D);
    Carver c(base);
    Saved s{};
    if (path == PATH_PAIR) {
        s.qQ = c.take<uint16_t>(ta);
        s.kQ = c.take<uint16_t>(ta);
        s.vR = c.take<uint16_t>(td);
        s.P = c.take<uint16_t>(pair_p_bytes(B, T) / 2);
        s.Pt = c.take<uint16_t>(pair_p_bytes(B, T) / 2);
        s.Plo = c.take<uint16_t>(pair_p_bytes(B, T) / 2);
    } else if (path == PATH_CHUNKED) {
        s.qR = c.take<uint16_t>(ta);
        s.kR = c.take<uint16_t>(ta);
        s.qQ = c.take<uint16_t>(ta);
        s.kQ = c.take<uint16_t>(ta);
        s.vR = c.take<uint16_t>(td);
        if (v_dtype != ULM_BF16) s.vRl = c.take<uint16_t>(td);
        s.vQ = c.take<uint16_t>(td);
        if (v_dtype != ULM_BF16) s.vQl = c.take<uint16_t>(td);
        s.Pdv = c.take<uint16_t>(B * NT * ULM_CHUNK * ULM_CHUNK);
    } else {
        s.q16n = c.take<uint16_t>(na);
        s.k16n = c.take<uint16_t>(na);
        s.v16n = c.take<uint16_t>(static_cast<size_t>(B) * T * D);
    }
    s.nck = c.take<float>(B * NT * A);
    s.bytes = c.off;
    return s;
}

struct FwdWs {
    float *gpart;  // generic path: the key tiles' partial planes
    uint16_t *Pf;
    uint16_t *qR, *kR, *vQ;   // pair path: the forward's operand tiles
    float *part;   // fp32 output or partials
    float *state;  // chunked prefill at widths off the 32 grid: the padded state
    float *segtot; // the statistics scan's segment totals (sequences past one segment)
    size_t bytes;
};

// resid: the output is x + fast, so the chunked products always go through fp32 partials.
// state: a chunked prefill (widths off the 32 grid keep a padded state here).
FwdWs fwd_layout(void *base, int B, int T, int A, int D, int fast_dtype, Path path, bool resid = false,
                 bool state = false) {
    const size_t NT = nt_of(T), nd = static_cast<size_t>(B) * T * D;
    const bool padded = A % 32 || D % 32;
    Carver c(base);
    FwdWs w{};
    if (path == PATH_PAIR) {
        // the block-pair products write the output directly
        w.qR = c.take<uint16_t>(B * NT * 64 * pad32(A));
        w.kR = c.take<uint16_t>(B * NT * 64 * pad32(A));
        w.vQ = c.take<uint16_t>(B * NT * 64 * pad32(D));
    } else if (path == PATH_CHUNKED) {
        w.Pf = c.take<uint16_t>(B * NT * ULM_CHUNK * ULM_CHUNK);
        const int nkg = la_kgroup_groups(pad32(A));
        if (nkg > 1 || fast_dtype != ULM_F32 || resid || padded)
            w.part = c.take<float>(nkg * static_cast<size_t>(B) * T * pad32(D));
        if (state && padded) w.state = c.take<float>(static_cast<size_t>(B) * pad32(D) * pad32(A));
    } else {
        if (fast_dtype != ULM_F32 || resid) w.part = c.take<float>(nd);
        if (la_generic_parts(A) > 1) w.gpart = c.take<float>(la_generic_parts(A) * nd);
    }
    const size_t stb = fwd_stats_segtot_bytes(B, T, A);
    if (stb) w.segtot = reinterpret_cast<float *>(c.take<char>(stb));
    w.bytes = c.off;
    return w;
}

struct BwdWs {
    float *gpart;                                            // generic path: partial planes
    uint16_t *do16;                                          // generic path
    uint16_t *doR, *doRl, *doQ, *doQl, *Pdq, *Pdk;   // K-group path (pair: doR, doQ)
    uint16_t *dS, *dSt;                                      // pair path: the score gradients, transposed
    double *dgx;                                             // pair path: dg partials of the pair products
    void *pstats;                                            // pair path: the fused statistics' arrays
    float *dqf, *dkf, *part;
    void *stats;
    size_t bytes;
};

BwdWs bwd_layout(void *base, int B, int T, int A, int D, int dfast_dtype, Path path) {
    const size_t NT = nt_of(T), nd = static_cast<size_t>(B) * T * D, na = static_cast<size_t>(B) * T * A;
    const size_t td = B * NT * 64 * D;
    Carver c(base);
    BwdWs w{};
    if (path != PATH_PAIR) {   // the pair path never materialises dq_f, dk_f
        w.dqf = c.take<float>(na);
        w.dkf = c.take<float>(na);
    }
    if (path == PATH_PAIR) {
        const size_t tdp = B * NT * 64 * pad32(D);
        w.doR = c.take<uint16_t>(tdp);
        w.doQ = c.take<uint16_t>(tdp);
        w.dS = c.take<uint16_t>(pair_p_bytes(B, T) / 2);
        w.dSt = c.take<uint16_t>(pair_p_bytes(B, T) / 2);
        w.dgx = c.take<double>(pair_dscore_jobs(B, T));
        w.pstats = c.take<char>(pair_stats_bytes(B, T, A));
    } else if (path == PATH_CHUNKED) {
        w.doR = c.take<uint16_t>(td);
        if (dfast_dtype != ULM_BF16) w.doRl = c.take<uint16_t>(td);
        w.doQ = c.take<uint16_t>(td);
        if (dfast_dtype != ULM_BF16) w.doQl = c.take<uint16_t>(td);
        w.Pdq = c.take<uint16_t>(B * NT * ULM_CHUNK * ULM_CHUNK);
        w.Pdk = c.take<uint16_t>(B * NT * ULM_CHUNK * ULM_CHUNK);
        const int nkd = la_kgroup_groups(D), nka = la_kgroup_groups(A);
        size_t part = static_cast<size_t>(nka) * nd;   // dv partials (or its fp32 copy)
        if (nkd > 1) part = part > nkd * na ? part : nkd * na;
        w.part = c.take<float>(part);
    } else {
        w.do16 = c.take<uint16_t>(nd);
        w.part = c.take<float>(nd);   // fp32 dv accumulator
        // dq_f and dk_f contract over D, dv over A
        const size_t gp = std::max(la_generic_parts(D) > 1 ? la_generic_parts(D) * na : 0,
                                   la_generic_parts(A) > 1 ? la_generic_parts(A) * nd : 0);
        if (gp) w.gpart = c.take<float>(gp);
    }
    if (path != PATH_PAIR) w.stats = c.take<char>(bwd_stats_partial_bytes(B, T, A));
    w.bytes = c.off;
    return w;
}

// The saved buffer's size names the form that filled it: the layout rounded
// up to 4 KB plus 256 (form + 1) bytes. ulm_fm_saved_bytes returns that size,
// ulm_fm_fwd evaluates the form it names and ulm_fm_bwd reads the buffer in
// the same form, so the forward and the backward of one call agree whatever
// ULM_FM_PATH says in between. Returns -1 for a size no form produces at this
// shape.
constexpr size_t kTagQuantum = 4096, kTagStep = 256;

size_t saved_tagged_bytes(int B, int T, int A, int D, int v_dtype, Path p) {
    return align_up(saved_layout(nullptr, B, T, A, D, v_dtype, p).bytes, kTagQuantum) +
           kTagStep * (static_cast<size_t>(p) + 1);
}

int saved_path(size_t bytes, int B, int T, int A, int D, int v_dtype) {
    const size_t tag = bytes % kTagQuantum / kTagStep;
    if (tag < 1 || tag > 3) return -1;
    const Path p = static_cast<Path>(tag - 1);
    if (!path_supported(p, B, T, A, D) || saved_tagged_bytes(B, T, A, D, v_dtype, p) != bytes) return -1;
    return static_cast<int>(p);
}

}  // namespace

}  // namespace ulm

using namespace ulm;

// ---------------------------------------------------------------------------
// bare chunked product

extern "C" size_t ulm_la_workspace_bytes(int B, int T, int K, int V) {
    if (B <= 0 || T <= 0 || K <= 0 || V <= 0) return 0;
    if (!la_kgroup_supported(B, T, K, V)) {
        // the generic kernel's partial planes, one per key tile past the first
        const int parts = la_generic_parts(K);
        return parts > 1 ? static_cast<size_t>(parts) * B * T * V * sizeof(float) : 0;
    }
    const size_t NT = nt_of(T), tk = B * NT * 64 * K, tv = B * NT * 64 * V;
    Carver c(nullptr);
    c.take<uint16_t>(2 * tk);                                 // a and b, R layout
    c.take<uint16_t>(tk);                                     // b, Q layout
    c.take<uint16_t>(tv);                                     // c, Q layout
    c.take<uint16_t>(2 * B * NT * ULM_CHUNK * ULM_CHUNK);     // P_lo, P_up
    const int nkg = la_kgroup_groups(K);
    if (nkg > 1) c.take<float>(static_cast<size_t>(nkg) * B * T * V);
    return c.off;
}

extern "C" int ulm_la(const uint16_t *a, const uint16_t *b, const uint16_t *c, const float *g, float *out, int B,
                      int T, int K, int V, int reverse, int split, void *workspace, size_t workspace_bytes,
                      void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && K > 0 && V > 0, "ulm_la: bad sizes B=%d T=%d K=%d V=%d", B, T, K, V);
    ULM_REQUIRE(a && b && c && g && out, "ulm_la: null pointer");
    const size_t need = ulm_la_workspace_bytes(B, T, K, V);
    ULM_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), "ulm_la: workspace of %zu bytes, need %zu",
                workspace_bytes, need);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!la_kgroup_supported(B, T, K, V))
        return launch_la_generic(a, b, c, g, out, static_cast<float *>(workspace), B, T, K, V, reverse != 0, s);
    const size_t NT = nt_of(T), tk = B * NT * 64 * K, tv = B * NT * 64 * V;
    Carver cv(workspace);
    uint16_t *aR = cv.take<uint16_t>(2 * tk);
    uint16_t *bR = aR + tk;
    uint16_t *bQ = cv.take<uint16_t>(tk);
    uint16_t *cQ = cv.take<uint16_t>(tv);
    uint16_t *Plo = cv.take<uint16_t>(2 * B * NT * ULM_CHUNK * ULM_CHUNK);
    uint16_t *Pup = Plo + B * NT * ULM_CHUNK * ULM_CHUNK;
    const int nkg = la_kgroup_groups(K);
    float *part = nkg > 1 ? cv.take<float>(static_cast<size_t>(nkg) * B * T * V) : out;
    ULM_TRY(launch_chunk_transpose(a, ULM_BF16, nullptr, nullptr, aR, nullptr, B, T, K, s));
    ULM_TRY(launch_chunk_transpose(b, ULM_BF16, bQ, nullptr, bR, nullptr, B, T, K, s));
    ULM_TRY(launch_chunk_transpose(c, ULM_BF16, cQ, nullptr, nullptr, nullptr, B, T, V, s));
    // split products keep P_up = P_lo^T exactly, as dq and dk do
    ULM_TRY(launch_chunk_scores(reverse ? bR : aR, nullptr, reverse ? aR : bR, nullptr, g, Plo, Pup, B, T, K, !split,
                                s));
    ULM_TRY(launch_la_kgroup(aR, nullptr, bQ, nullptr, cQ, nullptr, reverse ? Pup : Plo, !split, g, part, nullptr, B, T,
                             K, V, reverse != 0, split != 0, s));
    if (nkg > 1) ULM_TRY(launch_partial_reduce(part, nkg, static_cast<size_t>(B) * T * V, out, ULM_F32, s));
    return ULM_OK;
}

// ---------------------------------------------------------------------------
// fused operator

extern "C" int ulm_fm_path(int B, int T, int A, int D) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0) return -1;
    return static_cast<int>(train_path(B, T, A, D));
}

extern "C" size_t ulm_fm_saved_bytes(int B, int T, int A, int D, int v_dtype) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0 || !valid_dtype(v_dtype)) return 0;
    return saved_tagged_bytes(B, T, A, D, v_dtype, train_path(B, T, A, D));
}

extern "C" int ulm_fm_saved_path(size_t saved_bytes, int B, int T, int A, int D, int v_dtype) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0 || !valid_dtype(v_dtype)) return -1;
    return saved_path(saved_bytes, B, T, A, D, v_dtype);
}

extern "C" size_t ulm_fm_fwd_workspace_bytes(int B, int T, int A, int D, int fast_dtype) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0 || !valid_dtype(fast_dtype)) return 0;
    return fwd_layout(nullptr, B, T, A, D, fast_dtype, train_path(B, T, A, D)).bytes;
}

namespace {

// The forward composite of ulm_fm_fwd; with state (B, D, A) and c_last (B, A)
// (a prefill: the chunked or the block-pair form) it also emits the decode
// state after position T-1. q (fp32) and qw (w q in qw_dt) are each optional; with resid
// (fp32 (B,T,D)) the output is resid + fast.
int fm_forward(const RSrc &r, const void *v, int v_dtype, const float *g, const float *w, float *q, void *qw,
               int qw_dt, const float *resid, void *fast, int fast_dtype, void *saved, void *workspace, float *state,
               float *c_last, int B, int T, int A, int D, Path path, hipStream_t s) {
    const Saved sv = saved_layout(saved, B, T, A, D, v_dtype, path);
    const FwdWs ws = fwd_layout(workspace, B, T, A, D, fast_dtype, path, resid != nullptr, state != nullptr);
    const size_t nf = static_cast<size_t>(B) * T * D;
    if (path == PATH_PAIR) {
        // q, k: R layout for the scores (this pass only), Q layout for the
        // backward's dk_f, dq_f; v: Q layout for the apply, R layout for the
        // backward's dscores. bf16 v with D % 32 == 0 is tiled by the scores
        // launch, on the CUs its tiles leave idle; other v by a launch of its own.
        // A prefill (state wanted) has no backward: no qQ, vR, P^T or P residual;
        // kQ holds the keys decayed to T-1, and the state is one product of them
        // with v over the positions.
        const bool prefill = state != nullptr;
        if (prefill != (c_last != nullptr)) return fail(ULM_ERR_INVALID, "prefill: state and c_last go together");
        ULM_TRY(launch_fwd_stats(r, w, g, q, nullptr, nullptr, ws.qR, ws.kR, prefill ? nullptr : sv.qQ, sv.kQ, sv.nck,
                                 c_last, B, T, A, s, qw, qw_dt, pad32(A), ws.segtot, prefill ? 1 : 0));
        const bool ride = v_dtype == ULM_BF16 && D % 32 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0;
        uint16_t *vR = prefill ? nullptr : sv.vR;
        if (!ride) ULM_TRY(launch_chunk_transpose(v, v_dtype, ws.vQ, nullptr, vR, nullptr, B, T, D, s, pad32(D)));
        ULM_TRY(launch_pair_forward(ws.qR, ws.kR, ws.vQ, g, sv.P, prefill ? nullptr : sv.Pt, prefill ? nullptr : sv.Plo,
                                    fast, fast_dtype, resid, B, T, A, D, s,
                                    ride ? static_cast<const uint16_t *>(v) : nullptr, ride ? vR : nullptr));
        if (prefill) ULM_TRY(launch_pair_state(ws.vQ, sv.kQ, state, B, T, A, D, s));
        return ULM_OK;
    }
    if (path == PATH_CHUNKED) {
        // widths off the 32 grid (a prefill only) run on zero-padded tiles; the
        // output and the state drop the padding on the way out
        const int Ap = pad32(A), Dp = pad32(D);
        const bool padded = Ap != A || Dp != D;
        const int nkg = la_kgroup_groups(Ap);
        float *acc = ws.part ? ws.part : static_cast<float *>(fast);
        // a prefill (state wanted) has no backward, the only reader of q in the Q
        // layout and of v in the R layout: those tiles are not written then
        ULM_TRY(launch_fwd_stats(r, w, g, q, nullptr, nullptr, sv.qR, sv.kR, state ? nullptr : sv.qQ, sv.kQ, sv.nck,
                                 c_last, B, T, A, s, qw, qw_dt, Ap, ws.segtot));
        ULM_TRY(launch_chunk_transpose(v, v_dtype, sv.vQ, sv.vQl, state ? nullptr : sv.vR, state ? nullptr : sv.vRl, B,
                                       T, D, s, Dp));
        ULM_TRY(launch_chunk_scores(sv.qR, nullptr, sv.kR, nullptr, g, ws.Pf, sv.Pdv, B, T, Ap, true, s));
        // fast = LA(q, k, v): update k^T v~ (v~ from the full-precision v), intra on
        // bf16(v), as the reference's bf16 v (kernel.py:205). Its state, transposed,
        // is the decode state S (model.py:96-111).
        float *st = state && padded ? ws.state : state;
        ULM_TRY(launch_la_kgroup(sv.qR, nullptr, sv.kQ, nullptr, sv.vQ, sv.vQl, ws.Pf, true, g, acc, st, B, T, Ap, Dp,
                                 false, false, s));
        if (padded) {
            ULM_TRY(launch_unpad_sum(ws.part, nkg, B, T, T, D, Dp, fast, fast_dtype, s, resid));
            if (state) ULM_TRY(launch_unpad_sum(ws.state, 1, B, D, Dp, A, Ap, state, ULM_F32, s, nullptr));
        } else if (ws.part) {
            ULM_TRY(launch_partial_reduce(ws.part, nkg, nf, fast, fast_dtype, s, resid));
        }
        return ULM_OK;
    }
    if (state || c_last) return fail(ULM_ERR_UNSUPPORTED, "prefill state: not on the generic path");
    ULM_TRY(launch_fwd_stats(r, w, g, q, sv.q16n, sv.k16n, nullptr, nullptr, nullptr, nullptr, sv.nck, nullptr, B, T, A,
                             s, qw, qw_dt, 0, ws.segtot));
    ULM_TRY(launch_convert(v, v_dtype, sv.v16n, ULM_BF16, nf, s));
    float *acc = ws.part ? ws.part : static_cast<float *>(fast);
    ULM_TRY(launch_la_generic(sv.q16n, sv.k16n, sv.v16n, g, acc, ws.gpart, B, T, A, D, false, s));
    if (ws.part) ULM_TRY(launch_partial_reduce(acc, 1, nf, fast, fast_dtype, s, resid));
    return ULM_OK;
}

}  // namespace

extern "C" int ulm_fm_fwd(const float *r, const void *v, int v_dtype, const float *g, const float *w, float *q,
                          void *fast, int fast_dtype, void *saved, size_t saved_bytes, void *workspace,
                          size_t workspace_bytes, int B, int T, int A, int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && A > 0 && D > 0, "ulm_fm_fwd: bad sizes B=%d T=%d A=%d D=%d", B, T, A, D);
    ULM_REQUIRE(valid_dtype(v_dtype) && valid_dtype(fast_dtype), "ulm_fm_fwd: bad dtype %d/%d", v_dtype, fast_dtype);
    ULM_REQUIRE(r && v && g && w && q && fast && saved, "ulm_fm_fwd: null pointer");
    const int path = saved_path(saved_bytes, B, T, A, D, v_dtype);
    ULM_REQUIRE(path >= 0, "ulm_fm_fwd: a saved buffer of %zu bytes names no form at B=%d T=%d A=%d D=%d (pass "
                "the size ulm_fm_saved_bytes returned)", saved_bytes, B, T, A, D);
    const size_t need = fwd_layout(nullptr, B, T, A, D, fast_dtype, static_cast<Path>(path)).bytes;
    ULM_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), "ulm_fm_fwd: workspace of %zu bytes, need %zu",
                workspace_bytes, need);
    RSrc rs;
    rs.r = r;
    return fm_forward(rs, v, v_dtype, g, w, q, nullptr, ULM_F32, nullptr, fast, fast_dtype, saved, workspace, nullptr,
                      nullptr, B, T, A, D, static_cast<Path>(path), static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// prefill: the forward plus the decode state after position T-1, in the form
// prefill_path picks

extern "C" int ulm_fm_prefill_path(int B, int T, int A, int D) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0 || !fm_aligned(B, T, pad32(A), pad32(D))) return -1;
    return static_cast<int>(prefill_path(B, T, A, D));
}

extern "C" size_t ulm_fm_prefill_workspace_bytes(int B, int T, int A, int D, int v_dtype, int fast_dtype) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0 || !valid_dtype(v_dtype) || !valid_dtype(fast_dtype)) return 0;
    if (!fm_aligned(B, T, pad32(A), pad32(D))) return 0;
    const Path path = prefill_path(B, T, A, D);
    return align_up(saved_layout(nullptr, B, T, A, D, v_dtype, path).bytes, 256) +
           fwd_layout(nullptr, B, T, A, D, fast_dtype, path, false, true).bytes;
}

extern "C" int ulm_fm_prefill(const float *r, const void *v, int v_dtype, const float *g, const float *w, float *q,
                              void *fast, int fast_dtype, float *S, float *c_last, void *workspace,
                              size_t workspace_bytes, int B, int T, int A, int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && A > 0 && D > 0, "ulm_fm_prefill: bad sizes B=%d T=%d A=%d D=%d", B, T, A, D);
    ULM_REQUIRE(valid_dtype(v_dtype) && valid_dtype(fast_dtype), "ulm_fm_prefill: bad dtype %d/%d", v_dtype,
                fast_dtype);
    ULM_REQUIRE(r && v && g && w && q && fast && S && c_last && workspace, "ulm_fm_prefill: null pointer");
    ULM_REQUIRE(fm_aligned(B, T, pad32(A), pad32(D)), "ulm_fm_prefill: unsupported sizes B=%d T=%d A=%d D=%d", B, T,
                A, D);
    ULM_REQUIRE(reinterpret_cast<uintptr_t>(S) % 16 == 0, "ulm_fm_prefill: S must be 16-byte aligned");
    const size_t need = ulm_fm_prefill_workspace_bytes(B, T, A, D, v_dtype, fast_dtype);
    ULM_REQUIRE(workspace_bytes >= need, "ulm_fm_prefill: workspace of %zu bytes, need %zu", workspace_bytes, need);
    const Path path = prefill_path(B, T, A, D);
    char *saved = static_cast<char *>(workspace);
    char *ws = saved + align_up(saved_layout(nullptr, B, T, A, D, v_dtype, path).bytes, 256);
    RSrc rs;
    rs.r = r;
    return fm_forward(rs, v, v_dtype, g, w, q, nullptr, ULM_F32, nullptr, fast, fast_dtype, saved, ws, S, c_last, B, T,
                      A, D, path, static_cast<hipStream_t>(stream));
}

extern "C" size_t ulm_fm_bwd_workspace_bytes(int B, int T, int A, int D, int dfast_dtype, size_t saved_bytes,
                                             int v_dtype) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0 || !valid_dtype(dfast_dtype)) return 0;
    if (saved_bytes == 0) return bwd_layout(nullptr, B, T, A, D, dfast_dtype, train_path(B, T, A, D)).bytes;
    if (!valid_dtype(v_dtype)) return 0;
    const int path = saved_path(saved_bytes, B, T, A, D, v_dtype);
    return path < 0 ? 0 : bwd_layout(nullptr, B, T, A, D, dfast_dtype, static_cast<Path>(path)).bytes;
}

namespace {

// The backward composite of ulm_fm_bwd (arguments checked by the caller); dqw
// (d(w q) in dqw_dt, may be null) adds w dqw to dq_out and sum_t q dqw to dw.
int fm_backward(const RSrc &r, const float *g, const float *w, const void *saved, int v_dtype, const void *dfast,
                int dfast_dtype, const float *dq_out, const void *dqw, int dqw_dt, float *dr, void *dv, int dv_dtype,
                float *dg, float *dw, void *workspace, int B, int T, int A, int D, Path path, hipStream_t s) {
    const Saved sv = saved_layout(const_cast<void *>(saved), B, T, A, D, v_dtype, path);
    const BwdWs ws = bwd_layout(workspace, B, T, A, D, dfast_dtype, path);
    const size_t nd = static_cast<size_t>(B) * T * D, na = static_cast<size_t>(B) * T * A;
    if (path == PATH_PAIR) {
        ULM_TRY(launch_chunk_transpose(dfast, dfast_dtype, ws.doQ, nullptr, ws.doR, nullptr, B, T, D, s, pad32(D)));
        // the statistics run in the dq_f and dk_f products' epilogues
        const void *xq = dqw ? dqw : static_cast<const void *>(dq_out);
        const int xq_kind = dqw ? 2 + dqw_dt : (dq_out ? 1 : 0);
        if (dqw && dq_out) return fail(ULM_ERR_INVALID, "fm backward: dq_out and d(w q) are exclusive");
        return launch_pair_backward(sv.vR, ws.doR, ws.doQ, sv.kQ, sv.qQ, sv.P, sv.Pt, sv.Plo, g, ws.dS, ws.dSt,
                                    ws.dgx, r, xq, xq_kind, sv.nck, w, dr, dw, dg, ws.pstats, dv, dv_dtype, B, T, A,
                                    D, s);
    }
    if (path == PATH_CHUNKED) {
        const int nkd = la_kgroup_groups(D), nka = la_kgroup_groups(A);
        ULM_TRY(launch_chunk_transpose(dfast, dfast_dtype, ws.doQ, ws.doQl, ws.doR, ws.doRl, B, T, D, s));
        // unscaled: P_dk = P_dq^T exactly, so the intra-chunk terms of dq and dk
        // cancel in the d/dg identity
        ULM_TRY(launch_chunk_scores(ws.doR, ws.doRl, sv.vR, sv.vRl, g, ws.Pdq, ws.Pdk, B, T, D, false, s));
        // dq_f = LA(dfast, v, k): keys = D, values = A; update v^T k~.
        // dk_f = LA_rev(v, dfast, q): update dfast^T q~.
        // Both feed the positional d/dg identity, whose cancellation amplifies
        // rounding, so the decayed k~ / q~ take their bf16 remainder as a second
        // pass (and v, dfast their hi + lo pairs when they arrived in more than bf16).
        ULM_TRY(launch_la_kgroup(ws.doR, ws.doRl, sv.vQ, sv.vQl, sv.kQ, nullptr, ws.Pdq, false, g,
                                 nkd > 1 ? ws.part : ws.dqf, nullptr, B, T, D, A, false, true, s));
        if (nkd > 1) ULM_TRY(launch_partial_reduce(ws.part, nkd, na, ws.dqf, ULM_F32, s));
        ULM_TRY(launch_la_kgroup(sv.vR, sv.vRl, ws.doQ, ws.doQl, sv.qQ, nullptr, ws.Pdk, false, g,
                                 nkd > 1 ? ws.part : ws.dkf, nullptr, B, T, D, A, true, true, s));
        if (nkd > 1) ULM_TRY(launch_partial_reduce(ws.part, nkd, na, ws.dkf, ULM_F32, s));
        // dv = LA_rev(k, q, dfast): keys = A, values = D; update q^T dfast~ (from the
        // full-precision dfast), intra on bf16(dfast)
        const bool direct = nka == 1 && dv_dtype == ULM_F32;
        ULM_TRY(launch_la_kgroup(sv.kR, nullptr, sv.qQ, nullptr, ws.doQ, ws.doQl, sv.Pdv, true, g,
                                 direct ? static_cast<float *>(dv) : ws.part, nullptr, B, T, A, D, true, false, s));
        if (!direct) ULM_TRY(launch_partial_reduce(ws.part, nka, nd, dv, dv_dtype, s));
    } else {
        const uint16_t *do16 = static_cast<const uint16_t *>(dfast);
        if (dfast_dtype != ULM_BF16) {
            ULM_TRY(launch_convert(dfast, dfast_dtype, ws.do16, ULM_BF16, nd, s));
            do16 = ws.do16;
        }
        ULM_TRY(launch_la_generic(do16, sv.v16n, sv.k16n, g, ws.dqf, ws.gpart, B, T, D, A, false, s));
        ULM_TRY(launch_la_generic(sv.v16n, do16, sv.q16n, g, ws.dkf, ws.gpart, B, T, D, A, true, s));
        float *dv_acc = dv_dtype == ULM_F32 ? static_cast<float *>(dv) : ws.part;
        ULM_TRY(launch_la_generic(sv.k16n, sv.q16n, do16, g, dv_acc, ws.gpart, B, T, A, D, true, s));
        if (dv_dtype != ULM_F32) ULM_TRY(launch_convert(dv_acc, ULM_F32, dv, dv_dtype, nd, s));
    }
    return launch_bwd_stats(ws.dqf, dq_out, r, sv.nck, w, g, ws.dkf, dr, dw, dg, ws.stats, B, T, A, s, dqw, dqw_dt);
}

}  // namespace

extern "C" int ulm_fm_bwd(const float *r, const float *g, const float *w, const void *saved,
                          size_t saved_bytes, int v_dtype, const void *dfast, int dfast_dtype, const float *dq_out,
                          float *dr, void *dv, int dv_dtype, float *dg, float *dw, void *workspace,
                          size_t workspace_bytes, int B, int T, int A, int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && A > 0 && D > 0, "ulm_fm_bwd: bad sizes B=%d T=%d A=%d D=%d", B, T, A, D);
    ULM_REQUIRE(valid_dtype(v_dtype) && valid_dtype(dfast_dtype) && valid_dtype(dv_dtype),
                "ulm_fm_bwd: bad dtype %d/%d/%d", v_dtype, dfast_dtype, dv_dtype);
    ULM_REQUIRE(r && g && w && saved && dfast && dr && dv && dg && dw, "ulm_fm_bwd: null pointer");
    const int path = saved_path(saved_bytes, B, T, A, D, v_dtype);
    ULM_REQUIRE(path >= 0, "ulm_fm_bwd: a saved buffer of %zu bytes names no form at B=%d T=%d A=%d D=%d", saved_bytes,
                B, T, A, D);
    const size_t need = bwd_layout(nullptr, B, T, A, D, dfast_dtype, static_cast<Path>(path)).bytes;
    ULM_REQUIRE(workspace && workspace_bytes >= need, "ulm_fm_bwd: workspace of %zu bytes, need %zu",
                workspace_bytes, need);
    RSrc rs;
    rs.r = r;
    return fm_backward(rs, g, w, saved, v_dtype, dfast, dfast_dtype, dq_out, nullptr, ULM_BF16, dr, dv, dv_dtype, dg,
                       dw, workspace, B, T, A, D, static_cast<Path>(path), static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// the fast memory inside UnifiedBlock.forward (model.py:77-85): the read-out
// side emits w q for the mu GEMM and adds the residual to fast

extern "C" size_t ulm_block_fm_fwd_workspace_bytes(int B, int T, int A, int D) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0) return 0;
    return fwd_layout(nullptr, B, T, A, D, ULM_F32, train_path(B, T, A, D), true).bytes;
}

extern "C" int ulm_block_fm_fwd(const void *pre, int pre_dtype, const float *bias, const float *denom, const void *v,
                                int v_dtype, const float *g, const float *w, void *qw, int qw_dtype, const float *x,
                                float *y, void *saved, size_t saved_bytes, void *workspace, size_t workspace_bytes,
                                int B, int T, int A, int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && A > 0 && D > 0, "ulm_block_fm_fwd: bad sizes B=%d T=%d A=%d D=%d", B, T, A, D);
    ULM_REQUIRE(valid_dtype(pre_dtype) && valid_dtype(v_dtype) && valid_dtype(qw_dtype),
                "ulm_block_fm_fwd: bad dtype %d/%d/%d", pre_dtype, v_dtype, qw_dtype);
    ULM_REQUIRE(pre && denom && v && g && w && qw && x && y && saved && workspace, "ulm_block_fm_fwd: null pointer");
    ULM_REQUIRE(static_cast<const void *>(x) != static_cast<const void *>(y), "ulm_block_fm_fwd: y must not alias x");
    const int path = saved_path(saved_bytes, B, T, A, D, v_dtype);
    ULM_REQUIRE(path >= 0, "ulm_block_fm_fwd: a saved buffer of %zu bytes names no form at B=%d T=%d A=%d D=%d",
                saved_bytes, B, T, A, D);
    const size_t need = fwd_layout(nullptr, B, T, A, D, ULM_F32, static_cast<Path>(path), true).bytes;
    ULM_REQUIRE(workspace_bytes >= need, "ulm_block_fm_fwd: workspace of %zu bytes, need %zu", workspace_bytes, need);
    RSrc rs;
    rs.pre = pre;
    rs.pre_dt = pre_dtype;
    rs.bias = bias;
    rs.denom = denom;
    return fm_forward(rs, v, v_dtype, g, w, nullptr, qw, qw_dtype, x, y, ULM_F32, saved, workspace, nullptr, nullptr, B,
                      T, A, D, static_cast<Path>(path), static_cast<hipStream_t>(stream));
}

extern "C" int ulm_block_fm_bwd(const void *pre, int pre_dtype, const float *bias, const float *denom, const float *g,
                                const float *w, const void *saved, size_t saved_bytes, int v_dtype, const void *dfast,
                                int dfast_dtype, const void *dqw, int dqw_dtype, float *dr, void *dv, int dv_dtype,
                                float *dg, float *dw, void *workspace, size_t workspace_bytes, int B, int T, int A,
                                int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && A > 0 && D > 0, "ulm_block_fm_bwd: bad sizes B=%d T=%d A=%d D=%d", B, T, A, D);
    ULM_REQUIRE(valid_dtype(pre_dtype) && valid_dtype(v_dtype) && valid_dtype(dfast_dtype) &&
                    valid_dtype(dv_dtype) && valid_dtype(dqw_dtype),
                "ulm_block_fm_bwd: bad dtype %d/%d/%d/%d/%d", pre_dtype, v_dtype, dfast_dtype, dv_dtype, dqw_dtype);
    ULM_REQUIRE(pre && denom && g && w && saved && dfast && dqw && dr && dv && dg && dw,
                "ulm_block_fm_bwd: null pointer");
    const int path = saved_path(saved_bytes, B, T, A, D, v_dtype);
    ULM_REQUIRE(path >= 0, "ulm_block_fm_bwd: a saved buffer of %zu bytes names no form at B=%d T=%d A=%d D=%d",
                saved_bytes, B, T, A, D);
    const size_t need = bwd_layout(nullptr, B, T, A, D, dfast_dtype, static_cast<Path>(path)).bytes;
    ULM_REQUIRE(workspace && workspace_bytes >= need, "ulm_block_fm_bwd: workspace of %zu bytes, need %zu",
                workspace_bytes, need);
    RSrc rs;
    rs.pre = pre;
    rs.pre_dt = pre_dtype;
    rs.bias = bias;
    rs.denom = denom;
    return fm_backward(rs, g, w, saved, v_dtype, dfast, dfast_dtype, nullptr, dqw, dqw_dtype, dr, dv, dv_dtype, dg, dw,
                       workspace, B, T, A, D, static_cast<Path>(path), static_cast<hipStream_t>(stream));
}

// the block's prefill: ulm_block_fm_fwd plus the decode state after T-1

extern "C" size_t ulm_block_fm_prefill_workspace_bytes(int B, int T, int A, int D, int v_dtype) {
    if (B <= 0 || T <= 0 || A <= 0 || D <= 0 || !valid_dtype(v_dtype)) return 0;
    if (!fm_aligned(B, T, pad32(A), pad32(D))) return 0;
    const Path path = prefill_path(B, T, A, D);
    return align_up(saved_layout(nullptr, B, T, A, D, v_dtype, path).bytes, 256) +
           fwd_layout(nullptr, B, T, A, D, ULM_F32, path, true, true).bytes;
}

extern "C" int ulm_block_fm_prefill(const void *pre, int pre_dtype, const float *bias, const float *denom,
                                    const void *v, int v_dtype, const float *g, const float *w, void *qw, int qw_dtype,
                                    const float *x, float *y, float *S, float *c_last, void *workspace,
                                    size_t workspace_bytes, int B, int T, int A, int D, void *stream) {
    ULM_REQUIRE(B > 0 && T > 0 && A > 0 && D > 0, "ulm_block_fm_prefill: bad sizes B=%d T=%d A=%d D=%d", B, T, A, D);
    ULM_REQUIRE(valid_dtype(pre_dtype) && valid_dtype(v_dtype) && valid_dtype(qw_dtype),
                "ulm_block_fm_prefill: bad dtype %d/%d/%d", pre_dtype, v_dtype, qw_dtype);
    ULM_REQUIRE(pre && denom && v && g && w && qw && x && y && S && c_last && workspace,
                "ulm_block_fm_prefill: null pointer");
    ULM_REQUIRE(static_cast<const void *>(x) != static_cast<const void *>(y), "ulm_block_fm_prefill: y must not alias x");
    ULM_REQUIRE(fm_aligned(B, T, pad32(A), pad32(D)), "ulm_block_fm_prefill: unsupported sizes B=%d T=%d A=%d D=%d",
                B, T, A, D);
    ULM_REQUIRE(reinterpret_cast<uintptr_t>(S) % 16 == 0, "ulm_block_fm_prefill: S must be 16-byte aligned");
    const size_t need = ulm_block_fm_prefill_workspace_bytes(B, T, A, D, v_dtype);
    ULM_REQUIRE(workspace_bytes >= need, "ulm_block_fm_prefill: workspace of %zu bytes, need %zu", workspace_bytes,
                need);
    const Path path = prefill_path(B, T, A, D);
    char *saved = static_cast<char *>(workspace);
    char *ws = saved + align_up(saved_layout(nullptr, B, T, A, D, v_dtype, path).bytes, 256);
    RSrc rs;
    rs.pre = pre;
    rs.pre_dt = pre_dtype;
    rs.bias = bias;
    rs.denom = denom;
    return fm_forward(rs, v, v_dtype, g, w, nullptr, qw, qw_dtype, x, y, ULM_F32, saved, ws, S, c_last, B, T, A, D,
                      path, static_cast<hipStream_t>(stream));
}
