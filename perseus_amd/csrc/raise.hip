// The bootstrap's raise kernels (semantics: crates/pc-kernels/kernels/args.cuh ModRaiseArgs / SmallIntArgs /
// SmallInt1Args :665-709, :890-907; kernels bts.cuh:14-221; host twins crates/pc-gpu/src/bts/raise.rs:159-292):
//   mod_raise:  x[t] = sum_{k < d} centred([x_k qhatinv_k]_{q_k}) qhat[k][t] mod q_t on rows t in [r0, r1)
//   small_int:  Garner from k <= 4 source rows to a multi-word integer, centred against Q_k / 2, optionally scaled by
//               R / 2^192 (rounded half up), reduced modulo every output prime with the sign restored
//   small_int1: the same from one source prime with a 64 x 64-bit scale mc / 2^sh
// All in coefficient form, u32 words, source primes below 2^31.
//
// mod_raise streams 4 consecutive coefficients per thread over one target row per workgroup row (the d source rows
// stay in L2 across the target rows). small_int and small_int1 give one coefficient per thread: its multi-word
// integer lives in registers (fixed trip counts over the table's maxima), and every source word of a coefficient is
// read before its first output word is written, so the outputs may overwrite the sources.
#include "common.h"

namespace pch {
namespace bts {

constexpr int BX = 256;
constexpr int XW = PC_SI_MAXW + PC_SI_MAXR;

__device__ __forceinline__ uint32_t m32(uint32_t q) { return 0xFFFFFFFFu / q; }  // floor(2^32 / q), q odd

// ------------------------------------------------------------------------------------------------ mod_raise
__global__ void __launch_bounds__(BX) mod_raise_k(ModRaiseArgs A, int logn) {
    const int t = A.r0 + blockIdx.y;
    const int c = blockIdx.z / A.nparts, part = blockIdx.z % A.nparts;
    const uint32_t i = (blockIdx.x * BX + threadIdx.x) * 4;
    uint32_t* x = (uint32_t*)A.x + c * A.ct_stride + part * A.part_stride;
    const Red rt(A.pr[t]);
    uint32_t acc[4] = {0, 0, 0, 0};
    for (int k = 0; k < A.d; ++k) {
        const Red rk(A.pr[k]);
        const uint32_t hk = (uint32_t)A.qhatinv[k], qh = (uint32_t)A.qhat[k][t];
        const uint32_t pkt = red32(rk.p, rt.p, rt.m);  // q_k mod q_t
        const uint4 s = *(const uint4*)(x + ((size_t)k << logn) + i);
        const uint32_t sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t y = rk.mul(sv[w], hk);
            uint32_t r = red32(y, rt.p, rt.m);
            if (y > (rk.p >> 1)) r = subm(r, pkt, rt.p);  // the centred y - q_k, reduced mod q_t
            acc[w] = addm(acc[w], rt.mul(r, qh), rt.p);
        }
    }
    *(uint4*)(x + ((size_t)t << logn) + i) = make_uint4(acc[0], acc[1], acc[2], acc[3]);
}

// ------------------------------------------------------------------------------------------------ small_int
__global__ void __launch_bounds__(BX) small_int_k(SmallIntArgs A, int logn) {
    const SmallIntTab& T = *A.tab;
    __shared__ uint32_t sq[PC_SI_MAXK], sm[PC_SI_MAXK], sw[PC_SI_MAXK][PC_SI_MAXK], sws[PC_SI_MAXK][PC_SI_MAXK];
    const int k = T.k < PC_SI_MAXK ? T.k : PC_SI_MAXK;
    const int nw = T.nw < PC_SI_MAXW ? T.nw : PC_SI_MAXW;
    const int nr = T.nr < PC_SI_MAXR ? T.nr : PC_SI_MAXR;
    const int nout = T.nout < PC_SI_MAXOUT ? T.nout : PC_SI_MAXOUT;
    if (threadIdx.x < PC_SI_MAXK * PC_SI_MAXK) {
        // the Garner constants q_j^-1 mod q_i with their Shoup companions, once per workgroup
        const int a = threadIdx.x / PC_SI_MAXK, b = threadIdx.x % PC_SI_MAXK;
        if (a < k) {
            const uint32_t q = T.q[a];
            if (b == 0) {
                sq[a] = q;
                sm[a] = m32(q);
            }
            if (b < a) {
                const uint32_t w = T.qinv[a][b];
                sw[a][b] = w;
                sws[a][b] = (uint32_t)(((uint64_t)w << 32) / q);
            }
        }
    }
    __syncthreads();
    const int part = blockIdx.y, c = blockIdx.z;
    const uint32_t idx = blockIdx.x * BX + threadIdx.x;
    const uint32_t* src = (const uint32_t*)A.src + c * A.src_ct_stride + part * A.src_part_stride;
    // Garner digits: X = v0 + v1 q0 + v2 q0 q1 + v3 q0 q1 q2
    uint32_t v[PC_SI_MAXK];
#pragma unroll
    for (int a = 0; a < PC_SI_MAXK; ++a) {
        v[a] = 0;
        if (a < k) {
            const uint32_t q = sq[a], m = sm[a];
            uint32_t d = red32(src[((size_t)a << logn) + idx], q, m);
#pragma unroll
            for (int b = 0; b < a; ++b) d = shoup(subm(d, red32(v[b], q, m), q), sw[a][b], sws[a][b], q);
            v[a] = d;
        }
    }
    // the digits to 32-bit words, Horner from the top digit
    uint32_t x[XW];
#pragma unroll
    for (int w = 0; w < XW; ++w) x[w] = 0;
#pragma unroll
    for (int a = PC_SI_MAXK - 1; a >= 0; --a) {
        if (a < k) {
            const uint32_t q = a == k - 1 ? 0u : sq[a];
            uint64_t carry = v[a];
#pragma unroll
            for (int w = 0; w < PC_SI_MAXK + 1; ++w) {
                const uint64_t s = (uint64_t)x[w] * q + carry;
                x[w] = (uint32_t)s;
                carry = s >> 32;
            }
        }
    }
    // centre: X > Q_k / 2 -> the magnitude Q_k - X, negative
    int cmp = 0;
#pragma unroll
    for (int w = PC_SI_MAXW - 1; w >= 0; --w)
        if (w < nw && cmp == 0 && x[w] != T.Qkh[w]) cmp = x[w] > T.Qkh[w] ? 1 : -1;
    const bool neg = cmp > 0;
    if (neg) {
        uint32_t borrow = 0;
#pragma unroll
        for (int w = 0; w < PC_SI_MAXW; ++w) {
            const uint64_t s = (uint64_t)(w < nw ? T.Qk[w] : 0u) - x[w] - borrow;
            x[w] = (uint32_t)s;
            borrow = (uint32_t)(s >> 63);
        }
    }
    int nq = nw;
    if (T.divide) {
        // floor((|X| R + 2^191) / 2^192): the product, the half, the top words
        uint32_t pr[XW];
#pragma unroll
        for (int w = 0; w < XW; ++w) pr[w] = 0;
#pragma unroll
        for (int a = 0; a < PC_SI_MAXW; ++a) {
            uint64_t carry = 0;
#pragma unroll
            for (int b = 0; b < PC_SI_MAXR; ++b) {
                const uint64_t s = (uint64_t)x[a] * (b < nr ? T.R[b] : 0u) + pr[a + b] + carry;
                pr[a + b] = (uint32_t)s;
                carry = s >> 32;
            }
#pragma unroll
            for (int b = a + PC_SI_MAXR; b < XW; ++b) {
                const uint64_t s = (uint64_t)pr[b] + carry;
                pr[b] = (uint32_t)s;
                carry = s >> 32;
            }
        }
        uint64_t carry = 1ull << 31;  // 2^191 = 2^31 in word 5
#pragma unroll
        for (int w = 5; w < XW; ++w) {
            const uint64_t s = (uint64_t)pr[w] + carry;
            pr[w] = (uint32_t)s;
            carry = s >> 32;
        }
        constexpr int DW = PC_SI_SHIFT / 32;
        nq = nw + nr - DW;
        nq = nq < 1 ? 1 : nq;
#pragma unroll
        for (int w = 0; w < XW; ++w) x[w] = (w < nq && w + DW < XW) ? pr[w + DW] : 0u;
    }
    uint32_t* out = (uint32_t*)A.out + c * A.ct_stride + part * A.part_stride;
    for (int o = 0; o < nout; ++o) {
        const int row = T.orow[o];
        const Red r(A.pr[row]);
        uint64_t lo = 0;
        uint32_t hi = 0;
#pragma unroll
        for (int w = 0; w < XW; ++w) {
            if (w < nq) {
                const uint64_t s = (uint64_t)x[w] * T.pow32[o][w];
                lo += s;
                hi += lo < s;
            }
        }
        uint32_t y = r.red96(lo, hi);
        if (neg && y) y = r.p - y;
        out[((size_t)row << logn) + idx] = y;
    }
}

// ------------------------------------------------------------------------------------------------ small_int1
__global__ void __launch_bounds__(BX) small_int1_k(SmallInt1Args A, int logn) {
    const int part = blockIdx.y, c = blockIdx.z;
    const uint32_t idx = blockIdx.x * BX + threadIdx.x;
    uint32_t* x = (uint32_t*)A.x + c * A.ct_stride + part * A.part_stride;
    const uint32_t q0 = (uint32_t)A.pr[0].p;
    const uint32_t v = x[idx];
    const bool neg = v > (q0 >> 1);
    const uint32_t mag = neg ? q0 - v : v;
    // |x| mc + 2^(sh - 1) as a 128-bit integer, shifted down by sh
    unsigned __int128 s = (unsigned __int128)mag * A.mc + ((unsigned __int128)1 << (A.sh - 1));
    const uint64_t q = (uint64_t)(s >> A.sh);
    for (int t = 0; t < A.nrows; ++t) {
        const Red r(A.pr[t]);
        uint32_t y = r(q);
        if (neg && y) y = r.p - y;
        x[((size_t)t << logn) + idx] = y;
    }
}

// ------------------------------------------------------------------------------------------------ launchers
// The reference's checks (bts.cuh:192-218), plus null pointers (-1) and an empty grid (0, no launch).
template <int LOGN>
int mod_raise(const ModRaiseArgs* a, pc_stream_t s) {
    if (!a || a->d < 1 || a->d > 4 || a->r0 < a->d || a->r1 > 64 || a->r1 <= a->r0 || a->nparts < 1 || a->nparts > 2)
        return -1;
    if (!a->x || !a->pr || a->K < 0) return -1;
    if (a->K == 0) return 0;
    hipLaunchKernelGGL(mod_raise_k, dim3((1u << LOGN) / (BX * 4), a->r1 - a->r0, a->K * a->nparts), dim3(BX), 0,
                       (hipStream_t)s, *a, LOGN);
    return launch_rc();
}
template <int LOGN>
int small_int(const SmallIntArgs* a, pc_stream_t s) {
    if (!a || a->nparts < 1 || a->nparts > 2 || a->K < 1) return -1;
    if (!a->src || !a->out || !a->tab || !a->pr) return -1;
    hipLaunchKernelGGL(small_int_k, dim3((1u << LOGN) / BX, a->nparts, a->K), dim3(BX), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}
template <int LOGN>
int small_int1(const SmallInt1Args* a, pc_stream_t s) {
    if (!a || a->sh < 1 || a->sh > 127 || a->nrows < 1 || a->nrows > 64 || a->K < 1 || a->nparts < 1 || a->nparts > 2)
        return -1;
    if (!a->x || !a->pr) return -1;
    hipLaunchKernelGGL(small_int1_k, dim3((1u << LOGN) / BX, a->nparts, a->K), dim3(BX), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}

}  // namespace bts

#define PCH_BTS_INST(L)                                                                                  \
    int mod_raise_##L(const ModRaiseArgs* a, pc_stream_t s) { return bts::mod_raise<L>(a, s); }         \
    int small_int_##L(const SmallIntArgs* a, pc_stream_t s) { return bts::small_int<L>(a, s); }         \
    int small_int1_##L(const SmallInt1Args* a, pc_stream_t s) { return bts::small_int1<L>(a, s); }
PCH_BTS_INST(12)
PCH_BTS_INST(13)
PCH_BTS_INST(14)
PCH_BTS_INST(15)
PCH_BTS_INST(16)

}  // namespace pch
