// The bootstrap's raise kernels (semantics: crates/pc-kernels/kernels/args.cuh ModRaiseArgs / SmallIntArgs /
// SmallInt1Args :665-709, :890-907; kernels bts.cuh:14-221; host twins crates/pc-gpu/src/bts/raise.rs:159-292):
//   mod_raise:  x[t] = sum_{k < d} centred([x_k qhatinv_k]_{q_k}) qhat[k][t] mod q_t on rows t in [r0, r1)
//   small_int:  Garner from k <= 4 source rows to a multi-word integer, centred against Q_k / 2, optionally scaled by
//               R / 2^192 (rounded half up), reduced modulo every output prime with the sign restored
//   small_int1: the same from one source prime with a 64 x 64-bit scale mc / 2^sh
// All in coefficient form, u32 words, source primes below 2^31.
//
// mod_raise streams 4 consecutive coefficients per thread over one target row per workgroup row (the d source rows
// stay in L2 across the target rows). small_int gives one coefficient per thread, its multi-word integer in registers
// (fixed trip counts over the table's maxima); small_int1 four. Every source word of a coefficient is read before its
// first output word is written, by the same thread, so the outputs may overwrite the sources.
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
// CRT by the sum form with a floating-point quotient, not mixed radix: X = S - u Q with S = sum_a y_a M_a,
// M_a = Q / q_a, y_a = [x_a (M_a^-1 mod q_a)]_{q_a} and u = floor(S / Q) = floor(sum_a y_a / q_a). The quotient is
// estimated in double (its error stays below 2^-48, so the estimate is u or u +- 1) and fixed with one exact multi-word
// comparison. The per-prime constants are derived in LDS at the start of each workgroup from the table's primes and
// Q_k alone (M_a by long division of Q_k, the inverse by Fermat), so the table's Garner constants (qinv) and its
// powers of 2^32 (pow32) are not read: the outputs are reduced by Horner's rule in 2^32 with the prime's own
// (2^32 mod p) Shoup pair from PrimeConst.
struct SiConst {
    uint32_t q[PC_SI_MAXK], qm[PC_SI_MAXK], c[PC_SI_MAXK], cs[PC_SI_MAXK];
    uint32_t M[PC_SI_MAXK][PC_SI_MAXW];
    double inv[PC_SI_MAXK];
};

__device__ uint32_t powmod32(uint32_t b, uint32_t e, uint32_t q) {
    uint64_t r = 1, x = b % q;
    for (; e; e >>= 1) {
        if (e & 1) r = r * x % q;
        x = x * x % q;
    }
    return (uint32_t)r;
}

// lane a < k: M_a = Q_k / q_a (exact long division from the top word), M_a^-1 mod q_a, 1 / q_a
__device__ void si_prologue(const SmallIntTab& T, int k, int nw, SiConst& L) {
    const int a = threadIdx.x;
    if (a >= k) return;
    const uint32_t q = T.q[a];
    uint64_t rem = 0;
    for (int w = PC_SI_MAXW - 1; w >= 0; --w) {
        const uint64_t cur = (rem << 32) | (w < nw ? T.Qk[w] : 0u);
        L.M[a][w] = (uint32_t)(cur / q);
        rem = cur % q;
    }
    uint64_t mr = 0;  // M_a mod q_a
    for (int w = PC_SI_MAXW - 1; w >= 0; --w) mr = ((mr << 32) | L.M[a][w]) % q;
    const uint32_t c = powmod32((uint32_t)mr, q - 2, q);
    L.q[a] = q;
    L.qm[a] = m32(q);
    L.c[a] = c;
    L.cs[a] = (uint32_t)(((uint64_t)c << 32) / q);
    L.inv[a] = 1.0 / (double)q;
}

// a 96-bit column accumulator of 64-bit products
struct Col {
    uint64_t lo = 0;
    uint32_t hi = 0;
    __device__ __forceinline__ void add(uint64_t v) {
        lo += v;
        hi += lo < v;
    }
    __device__ __forceinline__ uint32_t take() {  // the low word out, the rest shifted down
        const uint32_t w = (uint32_t)lo;
        lo = (lo >> 32) | ((uint64_t)hi << 32);
        hi = 0;
        return w;
    }
};

__global__ void __launch_bounds__(BX) small_int_k(SmallIntArgs A, int logn) {
    const SmallIntTab& T = *A.tab;
    const int k = min(T.k, PC_SI_MAXK), nw = min(T.nw, PC_SI_MAXW), nr = min(T.nr, PC_SI_MAXR);
    const int nout = min(T.nout, PC_SI_MAXOUT);
    __shared__ SiConst L;
    si_prologue(T, k, nw, L);
    __syncthreads();
    const int part = blockIdx.y, c = blockIdx.z;
    const size_t idx = (size_t)blockIdx.x * BX + threadIdx.x;
    const uint32_t* src = (const uint32_t*)A.src + c * A.src_ct_stride + part * A.src_part_stride + idx;
    // y_a and the quotient estimate; every source word is read here, before any output is written
    uint32_t y[PC_SI_MAXK];
    double f = 0.0;
#pragma unroll
    for (int a = 0; a < PC_SI_MAXK; ++a) {
        y[a] = 0;
        if (a < k) {
            y[a] = shoup(red32(src[(size_t)a << logn], L.q[a], L.qm[a]), L.c[a], L.cs[a], L.q[a]);
            f += (double)y[a] * L.inv[a];
        }
    }
    // S = sum_a y_a M_a, column by column
    uint32_t x[XW];
    {
        Col acc;
#pragma unroll
        for (int w = 0; w < PC_SI_MAXW; ++w) {
#pragma unroll
            for (int a = 0; a < PC_SI_MAXK; ++a) acc.add((uint64_t)y[a] * L.M[a][w]);
            x[w] = acc.take();
        }
#pragma unroll
        for (int w = PC_SI_MAXW; w < XW; ++w) x[w] = 0;
    }
    // X = S - u Q, then the one correction: + Q when negative, - Q when >= Q
    {
        const uint32_t u = (uint32_t)f;
        int64_t carry = 0;
#pragma unroll
        for (int w = 0; w < PC_SI_MAXW; ++w) {
            const int64_t d = (int64_t)x[w] - (int64_t)((uint64_t)u * T.Qk[w]) + carry;
            x[w] = (uint32_t)d;
            carry = d >> 32;
        }
        if (carry < 0) {
            uint64_t cy = 0;
#pragma unroll
            for (int w = 0; w < PC_SI_MAXW; ++w) {
                cy += (uint64_t)x[w] + T.Qk[w];
                x[w] = (uint32_t)cy;
                cy >>= 32;
            }
        } else {
            bool ge = true;  // X >= Q, decided from the top word down
            bool tie = true;
#pragma unroll
            for (int w = PC_SI_MAXW - 1; w >= 0; --w)
                if (tie && x[w] != T.Qk[w]) {
                    ge = x[w] > T.Qk[w];
                    tie = false;
                }
            if (ge) {
                int64_t b = 0;
#pragma unroll
                for (int w = 0; w < PC_SI_MAXW; ++w) {
                    const int64_t d = (int64_t)x[w] - T.Qk[w] + b;
                    x[w] = (uint32_t)d;
                    b = d >> 32;
                }
            }
        }
    }
    // the centred lift: X > floor(Q / 2) stands for X - Q, kept as its magnitude and a sign
    bool neg = false;
    {
        bool tie = true;
#pragma unroll
        for (int w = PC_SI_MAXW - 1; w >= 0; --w)
            if (tie && x[w] != T.Qkh[w]) {
                neg = x[w] > T.Qkh[w];
                tie = false;
            }
        if (neg) {
            int64_t b = 0;
#pragma unroll
            for (int w = 0; w < PC_SI_MAXW; ++w) {
                const int64_t d = (int64_t)T.Qk[w] - x[w] + b;
                x[w] = (uint32_t)d;
                b = d >> 32;
            }
        }
    }
    int nq = nw;
    if (T.divide) {
        // floor((|X| R + 2^191) / 2^192) by product scanning: column j sums x_a R_(j-a); 2^191 joins column 5 and
        // columns from 6 on are the quotient's words
        constexpr int DW = PC_SI_SHIFT / 32;
        uint32_t qw[XW];
        Col acc;
#pragma unroll
        for (int j = 0; j < XW; ++j) {
#pragma unroll
            for (int a = 0; a < PC_SI_MAXW; ++a)
                if (j - a >= 0 && j - a < PC_SI_MAXR) acc.add((uint64_t)x[a] * T.R[j - a]);
            if (j == DW - 1) acc.add(1ull << 31);
            const uint32_t w = acc.take();
            if (j >= DW) qw[j - DW] = w;
        }
#pragma unroll
        for (int j = XW - DW; j < XW; ++j) qw[j] = 0;
        nq = max(1, nw + nr - DW);
#pragma unroll
        for (int w = 0; w < XW; ++w) x[w] = w < nq ? qw[w] : 0u;
    }
    // sign(X) q mod p for every output row: Horner in 2^32 from the top word
    uint32_t* out = (uint32_t*)A.out + c * A.ct_stride + part * A.part_stride + idx;
    for (int o = 0; o < nout; ++o) {
        const int row = T.orow[o];
        const Red r(A.pr[row]);
        uint32_t h = 0;
#pragma unroll
        for (int w = XW - 1; w >= 0; --w)
            if (w < nq) h = r(((uint64_t)h << 32) | x[w]);
        out[(size_t)row << logn] = neg && h ? r.p - h : h;
    }
}

// ------------------------------------------------------------------------------------------------ small_int1
// Four coefficients per thread with 16-byte accesses: row 0 is read whole first (the outputs overwrite it), each
// magnitude scaled to q = floor((|x| mc + 2^(sh-1)) / 2^sh) in 128-bit arithmetic, then every output row is written
// four words at a time with the sign restored.
__global__ void __launch_bounds__(BX) small_int1_k(SmallInt1Args A, int logn) {
    const int part = blockIdx.y, c = blockIdx.z;
    const size_t idx = ((size_t)blockIdx.x * BX + threadIdx.x) * 4;
    uint32_t* x = (uint32_t*)A.x + c * A.ct_stride + part * A.part_stride + idx;
    const uint32_t q0 = (uint32_t)A.pr[0].p, half = q0 >> 1;
    const uint4 v4 = *(const uint4*)x;
    const uint32_t v[4] = {v4.x, v4.y, v4.z, v4.w};
    const unsigned __int128 rnd = (unsigned __int128)1 << (A.sh - 1);
    uint64_t q[4];
    uint32_t neg = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool n = v[j] > half;
        neg |= (uint32_t)n << j;
        const uint32_t mag = n ? q0 - v[j] : v[j];
        q[j] = (uint64_t)(((unsigned __int128)mag * A.mc + rnd) >> A.sh);
    }
    for (int t = 0; t < A.nrows; ++t) {
        const Red r(A.pr[t]);
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t h = r(q[j]);
            o[j] = (neg >> j & 1) && h ? r.p - h : h;
        }
        *(uint4*)(x + ((size_t)t << logn)) = make_uint4(o[0], o[1], o[2], o[3]);
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
    hipLaunchKernelGGL(small_int1_k, dim3((1u << LOGN) / (BX * 4), a->nparts, a->K), dim3(BX), 0, (hipStream_t)s, *a,
                       LOGN);
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
