// The composite one-pass rescale by the top one or two primes (semantics: crates/pc-kernels/kernels/args.cuh
// RescaleArgs / RescaleNttArgs :531-563; kernels rescale.cuh:12-263; host flow crates/pc-gpu/src/rescale.rs:318-516).
// With a = top, b = top - 1 and lift(y, q) = y - q when y > q/2 (else y), reduced mod q_i:
//   ndrop 1: tmp_i = A_i lift(y_a)                                (A_i = -q_a^-1 mod q_i)
//   ndrop 2: y' = qinv_ab y_b + C_ab lift(y_a) mod q_b             (q_a^-1 (y_b - lift(y_a)): the first rescale at b)
//            tmp_i = A_i lift(y_a) + B_i lift(y')                 (A_i = -(q_a q_b)^-1, B_i = -q_b^-1 mod q_i)
// in coefficient form, then x_i = alpha_i x_i + NTT(tmp_i): the same words as dropping a, then b, one at a time.
//
// rescale_coef: one pass over the tops writes every correction row; 4 consecutive coefficients per thread, the tops'
// words read once per row group (grid (N / 1024, RG, 2K)), the corrections streamed out row by row.
// rescale_fwd: the correction rows are never stored: a prep kernel writes the two sources of every coefficient (y_a,
// y') into tmp rows top and top - 1, and the forward NTT's column pass generates each correction row from them.
#include "fused.h"
#include "common.h"

namespace pch {
namespace rs {

constexpr int BX = 256;
constexpr int RG = 8;  // row groups of rescale_coef: each recomputes the tops' two sources, then writes rows y + RG k

__device__ __forceinline__ uint32_t* at(const PolyRef& r, int c, int part, int row, int logn) {
    return (uint32_t*)r.base + c * r.ct_stride + part * r.part_stride + ((size_t)row << logn);
}
__device__ __forceinline__ uint32_t mm(const PrimeConst& c) { return (uint32_t)(c.mu_lo >> 32); }

// y_a (scaled by ca) and, for ndrop 2, y' of 4 coefficients
struct Tops {
    uint32_t ya[4], yp[4];
};
__device__ __forceinline__ Tops tops(const RescaleArgs& A, int c, int part, uint32_t i, int logn) {
    Tops t;
    const int a = A.top, b = A.top - 1;
    const Red ra(A.pr[a]);
    const uint4 u = *(const uint4*)(at(A.x, c, part, a, logn) + i);
    t.ya[0] = u.x, t.ya[1] = u.y, t.ya[2] = u.z, t.ya[3] = u.w;
    if (A.ca != 1) {
#pragma unroll
        for (int w = 0; w < 4; ++w) t.ya[w] = ra.mul(t.ya[w], (uint32_t)A.ca);
    }
    if (A.ndrop == 2) {
        const Red rb(A.pr[b]);
        const uint32_t qa = ra.p, qb = rb.p, qar = red32(qa, qb, rb.m);
        const uint4 v = *(const uint4*)(at(A.x, c, part, b, logn) + i);
        uint32_t yb[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (A.ca != 1) yb[w] = rb.mul(yb[w], (uint32_t)A.cb);
            uint32_t la = red32(t.ya[w], qb, rb.m);
            if (t.ya[w] > (qa >> 1)) la = subm(la, qar, qb);
            t.yp[w] = addm(rb.mul((uint32_t)A.qinv_ab, yb[w]), rb.mul((uint32_t)A.C_ab, la), qb);
        }
    }
    return t;
}

__global__ void __launch_bounds__(BX) coef_k(RescaleArgs A, int logn) {
    const int c = blockIdx.z >> 1, part = blockIdx.z & 1;
    const uint32_t i = (blockIdx.x * BX + threadIdx.x) * 4;
    const Tops t = tops(A, c, part, i, logn);
    const uint32_t ha = (uint32_t)A.pr[A.top].p >> 1;
    const uint32_t hb = A.ndrop == 2 ? (uint32_t)A.pr[A.top - 1].p >> 1 : 0u;
    for (int row = blockIdx.y; row < A.nrows; row += gridDim.y) {
        const PrimeConst& pc = A.pr[row];
        const uint32_t q = (uint32_t)pc.p, m = mm(pc);
        const uint32_t av = ((const uint32_t*)A.A)[row], as = ((const uint32_t*)A.As)[row];
        const uint32_t qam = ((const uint32_t*)A.qam)[row];
        uint32_t r[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t la = red32(t.ya[w], q, m);
            if (t.ya[w] > ha) la = subm(la, qam, q);
            r[w] = shoup(la, av, as, q);
        }
        if (A.ndrop == 2) {
            const uint32_t bv = ((const uint32_t*)A.B)[row], bs = ((const uint32_t*)A.Bs)[row];
            const uint32_t qbm = ((const uint32_t*)A.qbm)[row];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t lb = red32(t.yp[w], q, m);
                if (t.yp[w] > hb) lb = subm(lb, qbm, q);
                r[w] = addm(r[w], shoup(lb, bv, bs, q), q);
            }
        }
        *(uint4*)(at(A.tmp, c, part, row, logn) + i) = make_uint4(r[0], r[1], r[2], r[3]);
    }
}

// rescale_fwd's sources: tmp rows top (y_a scaled by ca) and top - 1 (y'), ndrop 2
__global__ void __launch_bounds__(BX) prep_k(RescaleArgs A, int logn) {
    const int c = blockIdx.z >> 1, part = blockIdx.z & 1;
    const uint32_t i = (blockIdx.x * BX + threadIdx.x) * 4;
    const Tops t = tops(A, c, part, i, logn);
    *(uint4*)(at(A.tmp, c, part, A.top, logn) + i) = make_uint4(t.ya[0], t.ya[1], t.ya[2], t.ya[3]);
    *(uint4*)(at(A.tmp, c, part, A.top - 1, logn) + i) = make_uint4(t.yp[0], t.yp[1], t.yp[2], t.yp[3]);
}

inline int check(const RescaleArgs& a) {
    if (a.ndrop != 1 && a.ndrop != 2) return -1;
    if (!a.pr || !a.x.base || !a.tmp.base || !a.A || !a.As || !a.qam || a.K < 0 || a.nrows < 0) return -1;
    if (a.top < a.ndrop - 1 || (a.ndrop == 2 && (!a.B || !a.Bs || !a.qbm))) return -1;
    if (a.nrows > a.top + 1 - a.ndrop) return -1;  // a correction row of a dropped prime
    return 0;
}

template <int LOGN>
int coef(const RescaleArgs* a, pc_stream_t s) {
    if (!a || check(*a)) return -1;
    if (a->K == 0 || a->nrows == 0) return 0;
    hipLaunchKernelGGL(coef_k, dim3((1u << LOGN) / (BX * 4), RG, 2 * a->K), dim3(BX), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}

template <int LOGN>
int fwd(const RescaleNttArgs* a, pc_stream_t s) {
    if (!a) return -1;
    const RescaleArgs& R = a->rs;
    const NttArgs& T = a->ntt;
    if (R.ndrop != 2 || check(R) || T.soff || T.epi < 0 || T.epi > 3) return -1;
    if (T.epi && (!T.eout || !T.ex || !T.es || !T.ess)) return -1;
    if (R.K == 0) return 0;
    hipLaunchKernelGGL(prep_k, dim3((1u << LOGN) / (BX * 4), 1, 2 * R.K), dim3(BX), 0, (hipStream_t)s, R, LOGN);
    if (int rc = launch_rc()) return rc;
    NttArgs b = T;
    b.snum = 1;
    b.xnum = T.xnum > 1 ? T.xnum : 1;
    return ntt_fwd_rescale(LOGN, &b, &R, s);
}

}  // namespace rs

#define PCH_RS_INST(L)                                                                                     \
    int rescale_coef_##L(const RescaleArgs* a, pc_stream_t s) { return rs::coef<L>(a, s); }               \
    int rescale_fwd_##L(const RescaleNttArgs* a, pc_stream_t s) { return rs::fwd<L>(a, s); }
PCH_RS_INST(12)
PCH_RS_INST(13)
PCH_RS_INST(14)
PCH_RS_INST(15)
PCH_RS_INST(16)

}  // namespace pch
