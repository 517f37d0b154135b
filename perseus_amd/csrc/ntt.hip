// Negacyclic NTT / INTT over 32-bit primes for gfx950, OpenFHE order (crates/pc-kernels/kernels/args.cuh:66-107):
// the forward transform is Cooley-Tukey with bit-reversed output, out[i] = a(psi^(2 brev(i) + 1)); the inverse is
// Gentleman-Sande with N^-1 (or a per-row scale) folded into its last pass. Twiddles: fw[m + i] = psi^brev(m + i) with
// Shoup companions (crates/pc-gpu/src/context.rs:190-230).
//
// A row of N = R x C words is viewed as R rows of C contiguous words (j = r C + c). The stages whose butterflies span
// more than C words only mix words of one column (same c): the "column pass" runs them as C independent R-point
// sub-transforms; the remaining stages stay inside one C-word block: the "row pass" runs R independent C-point
// sub-transforms. The forward runs columns then rows, the inverse rows then columns; every pass is one kernel that
// reads and writes its words once.
//
// Inside a pass each thread owns 16 words of one sub-transform of S points (T = S / 16 threads per sub-transform,
// 256 threads per workgroup): 4 butterfly stages on words spaced T apart in registers ("layout A": e = tau + T j),
// one transpose through LDS, then log2(T) stages on 16 consecutive words ("layout B": e = 16 tau + j). The inverse
// runs the same two phases in the opposite order. A row-pass sub-transform lives in one wave, so its transposes need
// only a wave barrier, and it moves its words with 16-byte accesses (layout B) around one more transpose.
//
// Butterflies are lazy. When every prime of the launch is below 2^30 (NttArgs.lazy != 0) they are Harvey's: forward
// words in [0, 4p), inverse words in [0, 2p). Otherwise (primes up to 2^31, where 4p overflows a word) forward words
// stay in [0, 2p) and inverse words canonical. Either way a transform returns canonical words.
#include "fused.h"
#include "ntt_core.h"

namespace pch {
namespace ntt {

// ------------------------------------------------------------------------------------------------ forward
// Column pass: workgroup (x, row i) takes columns [x CC, x CC + CC) of row i.
template <int LOGN, bool H>
__global__ void __launch_bounds__(WG) fwd_cols(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::COL_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p, p2 = 2 * p;
    const uint32_t* w = (const uint32_t*)A.fw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.fws + ((size_t)pid << LOGN);
    const int col = threadIdx.x % G::CC, tau = threadIdx.x / G::CC;
    const int c = B.x * G::CC + col;
    const RowSrc src = row_src(A, i, LOGN);
    uint32_t x[E];
    if (src.n == 1) {
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = src.p0[(size_t)(tau + G::TR * j) * G::C + c];
    } else {
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = ld_src(src, (size_t)(tau + G::TR * j) * G::C + c, p);
    }
    // stages h = R/2 .. TR (rows): index R/(2h) + r/(2h)
    auto base = [](int h) { return (uint32_t)(G::R / (2 * h)); };
    phase_a<true, H, G::TR, decltype(base), true>(x, w, ws, p, p2, base);
#pragma unroll
    for (int j = 0; j < E; ++j) lds[tau * G::WT + col + j * G::WS] = x[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = lds[tau * G::RT + col + j * G::RS];
    phase_b<true, H, G::TR>(x, tau, w, ws, p, p2, base);
    uint32_t* out = (uint32_t*)A.base + ((size_t)A.roff[i] << LOGN);
#pragma unroll
    for (int j = 0; j < E; ++j) out[(size_t)(E * tau + j) * G::C + c] = x[j];  // lazy words
}

// Row pass: workgroup (x, row i) takes blocks [x BB, x BB + BB) of row i (C contiguous words each). EPI: NttArgs.epi
// (0: in place; 1: eout = (x - v) s, 2: eout = d + (x - v) s, 3: eout = x s + v; x = the sum of xnum rows of ex,
// s = es[prime id]; args.cuh:66-80).
template <int LOGN, bool H, int EPI>
__global__ void __launch_bounds__(WG) fwd_rows(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::ROW_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p, p2 = 2 * p;
    const uint32_t* w = (const uint32_t*)A.fw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.fws + ((size_t)pid << LOGN);
    const int lb = threadIdx.x / G::TC, tau = threadIdx.x % G::TC;
    const int blk = B.x * G::BB + lb;
    const size_t r0 = ((size_t)A.roff[i] << LOGN) + (size_t)blk * G::C + E * tau;
    uint32_t* a = (uint32_t*)A.base + r0;
    uint32_t x[E];
    ld16(a, x);
    // the epilogue's operand is loaded with the row: every HBM read of the workgroup is in flight before the butterflies
    uint32_t ex[E];
    if (EPI != 0) ld16_src(RowSrc{(const uint32_t*)A.ex, A.xnum, A.xstride}, r0, p, ex);
    constexpr int LS = G::C + G::C / E;
    uint32_t* l = lds + lb * LS;
    // stage of half distance h (words): index N/(2h) + blk C/(2h) + c/(2h)
    auto base = [blk](int h) { return (uint32_t)((G::N / (2 * h)) + blk * (G::C / (2 * h))); };
    Tw ta, tb;
    load_tw_a<G::TC>(ta, w, ws, base);
    load_tw_b<G::TC>(tb, tau, w, ws, base);
    b_to_a<G::TC>(x, l, tau);
    phase_a_t<true, H>(x, ta, p, p2);
    a_to_b<G::TC>(x, l, tau);
    phase_b_t<true, H, G::TC>(x, tb, p, p2);
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = canon<H>(x[j], p, p2);
    if (EPI == 0) {
        st16(a, x);
        return;
    }
    const uint32_t s = ((const uint32_t*)A.es)[pid], ss = ((const uint32_t*)A.ess)[pid];
    uint32_t* o = (uint32_t*)A.eout + r0;
    uint32_t d[E];
    if (EPI == 2) ld16(A.ed ? (const uint32_t*)A.ed + r0 : o, d);
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (EPI == 3) {
            x[j] = addm(shoup(ex[j], s, ss, p), x[j], p);
        } else {
            const uint32_t y = shoup(ex[j] - x[j] + p, s, ss, p);
            x[j] = EPI == 2 ? addm(d[j], y, p) : y;
        }
    }
    st16(o, x);
}

// ------------------------------------------------------------------------------------------------ inverse
template <int LOGN, bool H>
__global__ void __launch_bounds__(WG) inv_rows(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::ROW_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p, p2 = 2 * p;
    const uint32_t* w = (const uint32_t*)A.iw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.iws + ((size_t)pid << LOGN);
    const int lb = threadIdx.x / G::TC, tau = threadIdx.x % G::TC;
    const int blk = B.x * G::BB + lb;
    const RowSrc src = row_src(A, i, LOGN);
    const size_t e0 = (size_t)blk * G::C + E * tau;
    uint32_t x[E];
    ld16_src(src, e0, p, x);
    auto base = [blk](int h) { return (uint32_t)((G::N / (2 * h)) + blk * (G::C / (2 * h))); };
    Tw ta, tb;
    load_tw_b<G::TC>(tb, tau, w, ws, base);
    load_tw_a<G::TC>(ta, w, ws, base);
    phase_b_t<false, H, G::TC>(x, tb, p, p2);
    constexpr int LS = G::C + G::C / E;
    uint32_t* l = lds + lb * LS;
    b_to_a<G::TC>(x, l, tau);
    phase_a_t<false, H>(x, ta, p, p2);
    a_to_b<G::TC>(x, l, tau);
    st16((uint32_t*)A.base + ((size_t)A.roff[i] << LOGN) + e0, x);  // [0, 2p) (Harvey) or canonical
}

template <int LOGN, bool H>
__global__ void __launch_bounds__(WG) inv_cols(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::COL_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p, p2 = 2 * p;
    const uint32_t* w = (const uint32_t*)A.iw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.iws + ((size_t)pid << LOGN);
    const int col = threadIdx.x % G::CC, tau = threadIdx.x / G::CC;
    const int c = B.x * G::CC + col;
    uint32_t* a = (uint32_t*)A.base + ((size_t)A.roff[i] << LOGN);
    uint32_t x[E];
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = a[(size_t)(E * tau + j) * G::C + c];
    auto base = [](int h) { return (uint32_t)(G::R / (2 * h)); };
    phase_b<false, H, G::TR>(x, tau, w, ws, p, p2, base);
#pragma unroll
    for (int j = 0; j < E; ++j) lds[tau * G::RT + col + j * G::RS] = x[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = lds[tau * G::WT + col + j * G::WS];
    phase_a<false, H, G::TR, decltype(base), true>(x, w, ws, p, p2, base);
    // the scale: es[i] per row (NttArgs ABI 17) or N^-1 of the prime; Shoup takes the lazy words whole
    uint32_t s, ss;
    if (A.es) {
        s = ((const uint32_t*)A.es)[i];
        ss = ((const uint32_t*)A.ess)[i];
    } else {
        s = ((const uint32_t*)A.ninv)[pid];
        ss = ((const uint32_t*)A.ninvs)[pid];
    }
#pragma unroll
    for (int j = 0; j < E; ++j) a[(size_t)(tau + G::TR * j) * G::C + c] = shoup(x[j], s, ss, p);
}

// ------------------------------------------------------------------------------------------------ launchers
inline int check(const NttArgs* a, bool fwd) {
    if (!a || a->nrows < 0 || !a->base || !a->roff || !a->rprime || !a->pr) return -1;
    if (fwd ? (!a->fw || !a->fws) : (!a->iw || !a->iws)) return -1;
    if (a->soff && (!a->src || a->snum < 1)) return -1;
    if (fwd && a->epi != 0) {
        if (a->epi < 1 || a->epi > 3 || !a->eout || !a->ex || !a->es || !a->ess || a->xnum < 1) return -2;
    } else if (a->epi != 0) {
        return -2;  // the epilogues exist on the forward transform only
    }
    if (!fwd && !a->es && (!a->ninv || !a->ninvs)) return -1;
    return 0;
}

template <int LOGN, bool H>
void fwd_pair(const NttArgs& A, int r0, int n, hipStream_t st) {
    using G = Geo<LOGN>;
    // a first pass out of place, then the row pass in place on base
    hipLaunchKernelGGL((fwd_cols<LOGN, H>), dim3(G::COL_WGS, n), dim3(WG), 0, st, A, r0);
    NttArgs B = A;
    B.soff = nullptr;
    const dim3 g(G::ROW_WGS, n);
    switch (A.epi) {
        case 0: hipLaunchKernelGGL((fwd_rows<LOGN, H, 0>), g, dim3(WG), 0, st, B, r0); break;
        case 1: hipLaunchKernelGGL((fwd_rows<LOGN, H, 1>), g, dim3(WG), 0, st, B, r0); break;
        case 2: hipLaunchKernelGGL((fwd_rows<LOGN, H, 2>), g, dim3(WG), 0, st, B, r0); break;
        default: hipLaunchKernelGGL((fwd_rows<LOGN, H, 3>), g, dim3(WG), 0, st, B, r0); break;
    }
}

template <int LOGN>
int fwd(const NttArgs* a, pc_stream_t s) {
    if (int rc = check(a, true)) return rc;
    const NttArgs A = *a;
    const int chunk = A.chunk > 0 ? A.chunk : (A.nrows > 0 ? A.nrows : 1);
    hipStream_t st = (hipStream_t)s;
    for (int r0 = 0; r0 < A.nrows; r0 += chunk) {
        const int n = A.nrows - r0 < chunk ? A.nrows - r0 : chunk;
        if (A.lazy) fwd_pair<LOGN, true>(A, r0, n, st);
        else fwd_pair<LOGN, false>(A, r0, n, st);
    }
    return launch_rc();
}

template <int LOGN, bool H>
void inv_pair(const NttArgs& A, int r0, int n, hipStream_t st) {
    using G = Geo<LOGN>;
    hipLaunchKernelGGL((inv_rows<LOGN, H>), dim3(G::ROW_WGS, n), dim3(WG), 0, st, A, r0);
    NttArgs B = A;
    B.soff = nullptr;
    hipLaunchKernelGGL((inv_cols<LOGN, H>), dim3(G::COL_WGS, n), dim3(WG), 0, st, B, r0);
}

template <int LOGN>
int inv(const NttArgs* a, pc_stream_t s) {
    if (int rc = check(a, false)) return rc;
    const NttArgs A = *a;
    const int chunk = A.chunk > 0 ? A.chunk : (A.nrows > 0 ? A.nrows : 1);
    hipStream_t st = (hipStream_t)s;
    for (int r0 = 0; r0 < A.nrows; r0 += chunk) {
        const int n = A.nrows - r0 < chunk ? A.nrows - r0 : chunk;
        if (A.lazy) inv_pair<LOGN, true>(A, r0, n, st);
        else inv_pair<LOGN, false>(A, r0, n, st);
    }
    return launch_rc();
}

// the row pass alone over every row of the args (after a column pass done elsewhere)
template <int LOGN>
int fwd_rows_only(const NttArgs* a, pc_stream_t s) {
    if (int rc = check(a, true)) return rc;
    using G = Geo<LOGN>;
    if (a->nrows == 0) return 0;
    NttArgs B = *a;
    B.soff = nullptr;
    const dim3 g(G::ROW_WGS, B.nrows);
    hipStream_t st = (hipStream_t)s;
#define PCH_ROWS(HH)                                                                               \
    switch (B.epi) {                                                                               \
        case 0: hipLaunchKernelGGL((fwd_rows<LOGN, HH, 0>), g, dim3(WG), 0, st, B, 0); break;     \
        case 1: hipLaunchKernelGGL((fwd_rows<LOGN, HH, 1>), g, dim3(WG), 0, st, B, 0); break;     \
        case 2: hipLaunchKernelGGL((fwd_rows<LOGN, HH, 2>), g, dim3(WG), 0, st, B, 0); break;     \
        default: hipLaunchKernelGGL((fwd_rows<LOGN, HH, 3>), g, dim3(WG), 0, st, B, 0); break;    \
    }
    if (B.lazy) {
        PCH_ROWS(true)
    } else {
        PCH_ROWS(false)
    }
#undef PCH_ROWS
    return launch_rc();
}

}  // namespace ntt

int ntt_fwd_rows_only(int logn, const NttArgs* a, pc_stream_t s) {
    switch (logn) {
        case 12: return ntt::fwd_rows_only<12>(a, s);
        case 13: return ntt::fwd_rows_only<13>(a, s);
        case 14: return ntt::fwd_rows_only<14>(a, s);
        case 15: return ntt::fwd_rows_only<15>(a, s);
        case 16: return ntt::fwd_rows_only<16>(a, s);
        default: return -2;
    }
}

#define PCH_NTT_INST(L)                                                             \
    int ntt_fwd_##L(const NttArgs* a, pc_stream_t s) { return ntt::fwd<L>(a, s); } \
    int ntt_inv_##L(const NttArgs* a, pc_stream_t s) { return ntt::inv<L>(a, s); }
PCH_NTT_INST(12)
PCH_NTT_INST(13)
PCH_NTT_INST(14)
PCH_NTT_INST(15)
PCH_NTT_INST(16)

}  // namespace pch
