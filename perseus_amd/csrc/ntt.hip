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
// runs the same two phases in the opposite order. Words stay canonical in [0, p) between stages.
#include "common.h"

namespace pch {
namespace ntt {

constexpr int E = 16;     // words per thread
constexpr int WG = 256;   // threads per workgroup

template <int LOGN>
struct Geo {
    static constexpr int LR = LOGN / 2, LC = LOGN - LR;
    static constexpr int N = 1 << LOGN, R = 1 << LR, C = 1 << LC;
    static constexpr int TR = R / E, TC = C / E;   // threads per column / row sub-transform
    static constexpr int CC = WG / TR;             // columns per column-pass workgroup
    static constexpr int BB = WG / TC;             // blocks per row-pass workgroup
    static constexpr int COL_WGS = C / CC;         // column-pass workgroups per row
    static constexpr int ROW_WGS = R / BB;         // row-pass workgroups per row
    static constexpr int CPAD = CC == 16 ? 1 : 0;  // LDS row padding of the column pass
    static constexpr int COL_LDS = R * (CC + CPAD);
    static constexpr int ROW_LDS = BB * (C + C / E);
    static constexpr int LDS = COL_LDS > ROW_LDS ? COL_LDS : ROW_LDS;
    static_assert(TR >= 2 && TC >= 2 && TR <= E && TC <= E, "sub-transforms of 32 to 256 points");
};

__device__ __forceinline__ void ct(uint32_t& a, uint32_t& b, uint32_t w, uint32_t ws, uint32_t p) {
    const uint32_t t = shoup(b, w, ws, p);
    b = subm(a, t, p);
    a = addm(a, t, p);
}
__device__ __forceinline__ void gs(uint32_t& a, uint32_t& b, uint32_t w, uint32_t ws, uint32_t p) {
    const uint32_t u = a, v = b;
    a = addm(u, v, p);
    b = shoup(subm(u, v, p), w, ws, p);
}

// NG consecutive twiddles (and companions) of one stage in one vector load each: a stage's groups are NG = 8 / (h / T)
// (layout A) or 8 / h (layout B) consecutive table entries, and their first index is a multiple of NG.
template <int NG>
__device__ __forceinline__ void ldtw(const uint32_t* p, uint32_t (&v)[8]) {
    if constexpr (NG == 8) {
        const uint4 a = ((const uint4*)p)[0], b = ((const uint4*)p)[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else if constexpr (NG == 4) {
        const uint4 a = *(const uint4*)p;
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
    } else if constexpr (NG == 2) {
        const uint2 a = *(const uint2*)p;
        v[0] = a.x, v[1] = a.y;
    } else {
        v[0] = *p;
    }
}

// Butterfly stages of one phase. `base(h)` is the twiddle index of group 0 of the stage of half distance h (in the
// sub-transform's word units); group g of that stage uses index base(h) + g.
// Layout A (e = tau + T j), stages h = 8T, 4T, 2T, T: pairs (j, j + h/T), group j / (2 h/T).
template <bool FWD, int T, int K, class Base>
__device__ __forceinline__ void stage_a(uint32_t (&x)[E], const uint32_t* w, const uint32_t* ws, uint32_t p, Base base) {
    constexpr int hh = 1 << K, NG = 8 >> K;
    const uint32_t b0 = base(T << K);
    uint32_t tw[8], tws[8];
    ldtw<NG>(w + b0, tw);
    ldtw<NG>(ws + b0, tws);
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (j & hh) continue;
        const int g = j >> (K + 1);
        if (FWD) ct(x[j], x[j + hh], tw[g], tws[g], p);
        else gs(x[j], x[j + hh], tw[g], tws[g], p);
    }
}
template <bool FWD, int T, class Base>
__device__ __forceinline__ void phase_a(uint32_t (&x)[E], const uint32_t* w, const uint32_t* ws, uint32_t p, Base base) {
    if (FWD) {
        stage_a<FWD, T, 3>(x, w, ws, p, base);
        stage_a<FWD, T, 2>(x, w, ws, p, base);
        stage_a<FWD, T, 1>(x, w, ws, p, base);
        stage_a<FWD, T, 0>(x, w, ws, p, base);
    } else {
        stage_a<FWD, T, 0>(x, w, ws, p, base);
        stage_a<FWD, T, 1>(x, w, ws, p, base);
        stage_a<FWD, T, 2>(x, w, ws, p, base);
        stage_a<FWD, T, 3>(x, w, ws, p, base);
    }
}
// Layout B (e = 16 tau + j), stages h = T/2 .. 1: pairs (j, j + h), group (16 tau + j) / (2h).
template <bool FWD, int K, class Base>
__device__ __forceinline__ void stage_b(uint32_t (&x)[E], int tau, const uint32_t* w, const uint32_t* ws, uint32_t p,
                                        Base base) {
    constexpr int h = 1 << K, NG = 8 >> K;
    const uint32_t b0 = base(h) + ((uint32_t)(E * tau) >> (K + 1));
    uint32_t tw[8], tws[8];
    ldtw<NG>(w + b0, tw);
    ldtw<NG>(ws + b0, tws);
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (j & h) continue;
        const int g = j >> (K + 1);
        if (FWD) ct(x[j], x[j + h], tw[g], tws[g], p);
        else gs(x[j], x[j + h], tw[g], tws[g], p);
    }
}
template <bool FWD, int T, class Base>
__device__ __forceinline__ void phase_b(uint32_t (&x)[E], int tau, const uint32_t* w, const uint32_t* ws, uint32_t p,
                                        Base base) {
    constexpr int LT = T == 16 ? 4 : T == 8 ? 3 : T == 4 ? 2 : 1;
    if (FWD) {
        if (LT > 3) stage_b<FWD, 3>(x, tau, w, ws, p, base);
        if (LT > 2) stage_b<FWD, 2>(x, tau, w, ws, p, base);
        if (LT > 1) stage_b<FWD, 1>(x, tau, w, ws, p, base);
        stage_b<FWD, 0>(x, tau, w, ws, p, base);
    } else {
        stage_b<FWD, 0>(x, tau, w, ws, p, base);
        if (LT > 1) stage_b<FWD, 1>(x, tau, w, ws, p, base);
        if (LT > 2) stage_b<FWD, 2>(x, tau, w, ws, p, base);
        if (LT > 3) stage_b<FWD, 3>(x, tau, w, ws, p, base);
    }
}

// The first pass's source words of row i: out of place (src + soff[i] N, the sum mod p of snum rows sstride apart)
// or in place (base + roff[i] N).
struct RowSrc {
    const uint32_t* p0;
    int n;
    uint64_t stride;
};
__device__ __forceinline__ RowSrc row_src(const NttArgs& A, int i, int logn) {
    if (A.soff) return RowSrc{(const uint32_t*)A.src + ((size_t)A.soff[i] << logn), A.snum, A.sstride};
    return RowSrc{(const uint32_t*)A.base + ((size_t)A.roff[i] << logn), 1, 0};
}
__device__ __forceinline__ uint32_t ld_src(const RowSrc& s, size_t off, uint32_t p) {
    uint32_t v = s.p0[off];
    for (int k = 1; k < s.n; ++k) v = addm(v, s.p0[off + k * s.stride], p);
    return v;
}

// the workgroup's logical (block in row, row) after the XCD renumbering of a (gx, rows) grid
struct Blk {
    int x, y;
};
__device__ __forceinline__ Blk blk_xy() {
    const uint32_t n = gridDim.x * gridDim.y;
    const uint32_t l = xcd_block(blockIdx.y * gridDim.x + blockIdx.x, n);
    return Blk{(int)(l % gridDim.x), (int)(l / gridDim.x)};
}

// ------------------------------------------------------------------------------------------------ forward
// Column pass: workgroup (bx, row i) takes columns [bx CC, bx CC + CC) of row i.
template <int LOGN>
__global__ void __launch_bounds__(WG) fwd_cols(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::COL_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p;
    const uint32_t* w = (const uint32_t*)A.fw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.fws + ((size_t)pid << LOGN);
    const int col = threadIdx.x % G::CC, tau = threadIdx.x / G::CC;
    const int c = B.x * G::CC + col;
    const RowSrc src = row_src(A, i, LOGN);
    uint32_t x[E];
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = ld_src(src, (size_t)(tau + G::TR * j) * G::C + c, p);
    // stages h = R/2 .. TR (rows): index R/(2h) + r/(2h)
    phase_a<true, G::TR>(x, w, ws, p, [](int h) { return (uint32_t)(G::R / (2 * h)); });
    constexpr int LS = G::CC + G::CPAD;
#pragma unroll
    for (int j = 0; j < E; ++j) lds[(tau + G::TR * j) * LS + col] = x[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = lds[(E * tau + j) * LS + col];
    phase_b<true, G::TR>(x, tau, w, ws, p, [](int h) { return (uint32_t)(G::R / (2 * h)); });
    uint32_t* out = (uint32_t*)A.base + ((size_t)A.roff[i] << LOGN);
#pragma unroll
    for (int j = 0; j < E; ++j) out[(size_t)(E * tau + j) * G::C + c] = x[j];
}

// NttArgs.epi on the final words v of row i at word offsets e0 + j (j < 16) (args.cuh:66-80, ntt.cuh:204-222):
// 1: eout = (x - v) s, 2: eout = d + (x - v) s, 3: eout = x s + v; x = the sum of xnum rows of ex, s = es[prime id].
__device__ __forceinline__ void epilogue(const NttArgs& A, size_t r0, int pid, uint32_t p, uint32_t (&v)[E]) {
    const uint32_t s = ((const uint32_t*)A.es)[pid], ss = ((const uint32_t*)A.ess)[pid];
    const uint32_t* ex = (const uint32_t*)A.ex + r0;
    uint32_t x[E];
    ld16(ex, x);
    for (int k = 1; k < A.xnum; ++k) {
        uint32_t y[E];
        ld16(ex + k * A.xstride, y);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = addm(x[j], y[j], p);
    }
    uint32_t* o = (uint32_t*)A.eout + r0;
    uint32_t d[E];
    if (A.epi == 2) ld16(A.ed ? (const uint32_t*)A.ed + r0 : o, d);
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (A.epi == 3) {
            v[j] = addm(shoup(x[j], s, ss, p), v[j], p);
        } else {
            uint32_t y = shoup(subm(x[j], v[j], p), s, ss, p);
            v[j] = A.epi == 2 ? addm(d[j], y, p) : y;
        }
    }
    st16(o, v);
}

// Row pass: workgroup (bx, row i) takes blocks [bx BB, bx BB + BB) of row i (C contiguous words each).
template <int LOGN>
__global__ void __launch_bounds__(WG) fwd_rows(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::ROW_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p;
    const uint32_t* w = (const uint32_t*)A.fw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.fws + ((size_t)pid << LOGN);
    const int lb = threadIdx.x / G::TC, tau = threadIdx.x % G::TC;
    const int blk = B.x * G::BB + lb;
    uint32_t* row = (uint32_t*)A.base + ((size_t)A.roff[i] << LOGN);
    uint32_t* a = row + (size_t)blk * G::C;
    uint32_t x[E];
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = a[tau + G::TC * j];
    // stage of half distance h (words): index N/(2h) + blk C/(2h) + c/(2h)
    auto base = [blk](int h) { return (uint32_t)((G::N / (2 * h)) + blk * (G::C / (2 * h))); };
    phase_a<true, G::TC>(x, w, ws, p, base);
    constexpr int LS = G::C + G::C / E;
    uint32_t* l = lds + lb * LS;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int e = tau + G::TC * j;
        l[e + e / E] = x[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int e = E * tau + j;
        x[j] = l[e + e / E];
    }
    phase_b<true, G::TC>(x, tau, w, ws, p, base);
    const size_t off = ((size_t)A.roff[i] << LOGN) + (size_t)blk * G::C + E * tau;
    if (A.epi) epilogue(A, off, pid, p, x);
    else st16(a + E * tau, x);
}

// ------------------------------------------------------------------------------------------------ inverse
template <int LOGN>
__global__ void __launch_bounds__(WG) inv_rows(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::ROW_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p;
    const uint32_t* w = (const uint32_t*)A.iw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.iws + ((size_t)pid << LOGN);
    const int lb = threadIdx.x / G::TC, tau = threadIdx.x % G::TC;
    const int blk = B.x * G::BB + lb;
    const RowSrc src = row_src(A, i, LOGN);
    uint32_t x[E];
    const size_t e0 = (size_t)blk * G::C + E * tau;
    if (src.n == 1) {
        ld16(src.p0 + e0, x);
    } else {
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = ld_src(src, e0 + j, p);
    }
    auto base = [blk](int h) { return (uint32_t)((G::N / (2 * h)) + blk * (G::C / (2 * h))); };
    phase_b<false, G::TC>(x, tau, w, ws, p, base);
    constexpr int LS = G::C + G::C / E;
    uint32_t* l = lds + lb * LS;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int e = E * tau + j;
        l[e + e / E] = x[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int e = tau + G::TC * j;
        x[j] = l[e + e / E];
    }
    phase_a<false, G::TC>(x, w, ws, p, base);
    uint32_t* a = (uint32_t*)A.base + ((size_t)A.roff[i] << LOGN) + (size_t)blk * G::C;
#pragma unroll
    for (int j = 0; j < E; ++j) a[tau + G::TC * j] = x[j];
}

template <int LOGN>
__global__ void __launch_bounds__(WG) inv_cols(NttArgs A, int row0) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[G::COL_LDS];
    const Blk B = blk_xy();
    const int i = row0 + B.y;
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p;
    const uint32_t* w = (const uint32_t*)A.iw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.iws + ((size_t)pid << LOGN);
    const int col = threadIdx.x % G::CC, tau = threadIdx.x / G::CC;
    const int c = B.x * G::CC + col;
    uint32_t* a = (uint32_t*)A.base + ((size_t)A.roff[i] << LOGN);
    uint32_t x[E];
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = a[(size_t)(E * tau + j) * G::C + c];
    auto base = [](int h) { return (uint32_t)(G::R / (2 * h)); };
    phase_b<false, G::TR>(x, tau, w, ws, p, base);
    constexpr int LS = G::CC + G::CPAD;
#pragma unroll
    for (int j = 0; j < E; ++j) lds[(E * tau + j) * LS + col] = x[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = lds[(tau + G::TR * j) * LS + col];
    phase_a<false, G::TR>(x, w, ws, p, base);
    // the scale: es[i] per row (NttArgs ABI 17) or N^-1 of the prime
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

template <int LOGN>
int fwd(const NttArgs* a, pc_stream_t s) {
    using G = Geo<LOGN>;
    if (int rc = check(a, true)) return rc;
    const NttArgs A = *a;
    const int chunk = A.chunk > 0 ? A.chunk : (A.nrows > 0 ? A.nrows : 1);
    hipStream_t st = (hipStream_t)s;
    for (int r0 = 0; r0 < A.nrows; r0 += chunk) {
        const int n = A.nrows - r0 < chunk ? A.nrows - r0 : chunk;
        // a first pass out of place, then the row pass in place on base
        hipLaunchKernelGGL(fwd_cols<LOGN>, dim3(G::COL_WGS, n), dim3(WG), 0, st, A, r0);
        NttArgs B = A;
        B.soff = nullptr;
        hipLaunchKernelGGL(fwd_rows<LOGN>, dim3(G::ROW_WGS, n), dim3(WG), 0, st, B, r0);
    }
    return launch_rc();
}

template <int LOGN>
int inv(const NttArgs* a, pc_stream_t s) {
    using G = Geo<LOGN>;
    if (int rc = check(a, false)) return rc;
    const NttArgs A = *a;
    const int chunk = A.chunk > 0 ? A.chunk : (A.nrows > 0 ? A.nrows : 1);
    hipStream_t st = (hipStream_t)s;
    for (int r0 = 0; r0 < A.nrows; r0 += chunk) {
        const int n = A.nrows - r0 < chunk ? A.nrows - r0 : chunk;
        hipLaunchKernelGGL(inv_rows<LOGN>, dim3(G::ROW_WGS, n), dim3(WG), 0, st, A, r0);
        NttArgs B = A;
        B.soff = nullptr;
        hipLaunchKernelGGL(inv_cols<LOGN>, dim3(G::COL_WGS, n), dim3(WG), 0, st, B, r0);
    }
    return launch_rc();
}

}  // namespace ntt

#define PCH_NTT_INST(L)                                              \
    int ntt_fwd_##L(const NttArgs* a, pc_stream_t s) { return ntt::fwd<L>(a, s); } \
    int ntt_inv_##L(const NttArgs* a, pc_stream_t s) { return ntt::inv<L>(a, s); }
PCH_NTT_INST(12)
PCH_NTT_INST(13)
PCH_NTT_INST(14)
PCH_NTT_INST(15)
PCH_NTT_INST(16)

}  // namespace pch
