// One-pass negacyclic NTT / INTT of N = 2^16 words for gfx950: the transform of ntt.hip (same order, same words:
// crates/pc-kernels/kernels/args.cuh:66-107), with one 1024-thread workgroup per row holding the whole row in its
// registers, 64 words per thread, so that every word is read from HBM once and written once (the two-pass transform
// moves each word through HBM twice). The 16 butterfly stages run as three phases over the word index e (16 bits):
//   P1: stages of half distance 2^15 .. 2^11; thread t = e bits 9..0, its words j = e bits 15..10;
//   P2: stages 2^10 .. 2^5;               thread (a, b) = e bits 15..11 and 4..0 (t = 32 a + b), words e bits 10..5;
//   P3: stages 2^4 .. 2^0;                thread t = e bits 15..6, its words m = e bits 5..0 (64 consecutive words).
// (The inverse runs P3, P2, P1 with Gentleman-Sande butterflies.) Between phases the words cross the workgroup through
// LDS in two rounds. Each round moves the half of the row whose split bit is r. The split bit is e bit 10 between P1
// and P2, and e bit 5 between P2 and P3: a bit that is a word bit on both sides, so each round every thread writes 32
// of its words and then reads 32 new words into the registers it has just freed (132 KiB of LDS, no thread ever holds
// more than 64 words). Where a phase's words land in the register array is a compile-time map (phys below). Both
// rounds' LDS addresses are padded so that the 64 lanes of every access hit 64 distinct banks.
//
// Twiddles: stage of half distance h = 2^lh pairs (e, e + h) with twiddle index (N + e) >> (lh + 1) (the table is
// fw[m + i] = psi^brev(m + i), ntt.hip). In P1 the index depends on the word only (uniform over the workgroup: scalar
// loads); in P2 and P3 each thread reads 2^(5 - lb) consecutive entries per stage, in 16-byte chunks.
#include "fused.h"
#include "ntt_core.h"

namespace pch {
namespace ntt1 {

constexpr int LOGN = 16, T = 1024, W = 64, E = ntt::E;
constexpr int LDSW = 33792;  // 2^15 words of one round + padding (max padded address 33790)

// Physical register of logical word u in each phase's layout. Forward: P1 identity (map 0); X1 puts P2 word j' (round
// j' >> 5) into the register P1 word 2 (j' & 31) + (j' >> 5) freed (map 1); X2 puts P3 word m (round m >> 5) into the
// register of P2 word 2 (m & 31) + (m >> 5) (map 2). Inverse: P3 identity (map 0); P2 word j' (round j' & 1) takes the
// register of P3 word 32 (j' & 1) + (j' >> 1) (map 3); P1 word j (round j & 1) that of P2 word 32 (j & 1) + (j >> 1)
// (map 4).
__host__ __device__ constexpr int phys(int map, int u) {
    return map == 0   ? u
           : map == 1 ? 2 * (u & 31) + (u >> 5)
           : map == 2 ? phys(1, 2 * (u & 31) + (u >> 5))
           : map == 3 ? 32 * (u & 1) + (u >> 1)
                      : phys(3, 32 * (u & 1) + (u >> 1));
}

template <int NG>
__device__ __forceinline__ void ldv(const uint32_t* q, uint32_t (&v)[4]) {
    if constexpr (NG == 4) {
        const uint4 a = *(const uint4*)q;
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
    } else if constexpr (NG == 2) {
        const uint2 a = *(const uint2*)q;
        v[0] = a.x, v[1] = a.y;
    } else {
        v[0] = *q;
    }
}

// One stage over the thread's 64 words: pairs of logical words (u, u + 2^LB) for u with bit LB clear, group
// g = u >> (LB + 1) taking twiddle base + g. UNI: base is uniform over the workgroup (scalar loads).
template <bool FWD, bool H, int LB, int MAP, bool UNI>
__device__ __forceinline__ void stage(uint32_t (&x)[W], const uint32_t* w, const uint32_t* ws, uint32_t base,
                                      uint32_t p, uint32_t p2) {
    constexpr int G = W >> (LB + 1), hh = 1 << LB, CH = G < 4 ? G : 4;
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += CH) {
        uint32_t tw[4], tws[4];
        if constexpr (UNI) {
            const ntt::cptr cw = (ntt::cptr)w, cs = (ntt::cptr)ws;
#pragma unroll
            for (int c = 0; c < CH; ++c) tw[c] = cw[base + g0 + c], tws[c] = cs[base + g0 + c];
        } else {
            ldv<CH>(w + base + g0, tw);
            ldv<CH>(ws + base + g0, tws);
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
#pragma unroll
            for (int r = 0; r < hh; ++r) {
                const int u = (g0 + c) * 2 * hh + r;
                if (FWD) ntt::ct<H>(x[phys(MAP, u)], x[phys(MAP, u + hh)], tw[c], tws[c], p, p2);
                else ntt::gs<H>(x[phys(MAP, u)], x[phys(MAP, u + hh)], tw[c], tws[c], p, p2);
            }
        }
    }
}

// LDS addresses of the two exchanges (within one round's half row). X1 (split e bit 10): P1 word j of thread t at
// (j >> 1) 1056 + t; P2 word j' of thread (a, b) at a 1056 + 32 (j' & 31) + b. X2 (split e bit 5): P2 word j' of
// (a, b) at (32 a + (j' >> 1)) 33 + b; P3 word m of thread t at 33 t + (m & 31).
__device__ __forceinline__ int x1_p1(int j, int t) { return (j >> 1) * 1056 + t; }
__device__ __forceinline__ int x1_p2(int a, int b, int jp) { return a * 1056 + 32 * (jp & 31) + b; }
__device__ __forceinline__ int x2_p2(int a, int b, int jp) { return (32 * a + (jp >> 1)) * 33 + b; }
__device__ __forceinline__ int x2_p3(int t, int m) { return 33 * t + (m & 31); }

// forward exchanges: P1 -> P2 (layout map 0 -> 1), P2 -> P3 (map 1 -> 2)
__device__ __forceinline__ void x1_fwd(uint32_t (&x)[W], uint32_t* l, int t) {
    const int a = t >> 5, b = t & 31;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) l[x1_p1(2 * k + r, t)] = x[2 * k + r];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) x[phys(1, 32 * r + k)] = l[x1_p2(a, b, 32 * r + k)];
    }
}
__device__ __forceinline__ void x2_fwd(uint32_t (&x)[W], uint32_t* l, int t) {
    const int a = t >> 5, b = t & 31;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) l[x2_p2(a, b, 2 * k + r)] = x[phys(1, 2 * k + r)];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) x[phys(2, 32 * r + k)] = l[x2_p3(t, 32 * r + k)];
    }
}
// inverse exchanges: P3 -> P2 (map 0 -> 3), P2 -> P1 (map 3 -> 4)
__device__ __forceinline__ void x2_inv(uint32_t (&x)[W], uint32_t* l, int t) {
    const int a = t >> 5, b = t & 31;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) l[x2_p3(t, 32 * r + k)] = x[32 * r + k];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) x[phys(3, 2 * k + r)] = l[x2_p2(a, b, 2 * k + r)];
    }
}
__device__ __forceinline__ void x1_inv(uint32_t (&x)[W], uint32_t* l, int t) {
    const int a = t >> 5, b = t & 31;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) l[x1_p2(a, b, 32 * r + k)] = x[phys(3, 32 * r + k)];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k) x[phys(4, 2 * k + r)] = l[x1_p1(2 * k + r, t)];
    }
}

// the workgroup's row after the XCD renumbering (each XCD takes a contiguous range of the launch's rows)
__device__ __forceinline__ int row_of(int row0) { return row0 + (int)xcd_block(blockIdx.x, gridDim.x); }

// Forward transform of one row per workgroup. EPI as ntt.hip's row pass (0: in place; 1: eout = (x - v) s;
// 2: eout = d + (x - v) s; 3: eout = x s + v; v = the sum of xnum rows of ex, s = es[prime id]). DENSE: row i at
// base + i N with prime id i mod xnum (no row tables; a compile-time choice, since a run-time one costs the kernel
// its register allocation).
template <bool H, int EPI, bool DENSE = false>
__global__ void __launch_bounds__(T) fwd1(NttArgs A, int row0) {
    __shared__ uint32_t lds[LDSW];
    const int i = row_of(row0);
    const int pid = DENSE ? i % A.xnum : A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p, p2 = 2 * p;
    const uint32_t* w = (const uint32_t*)A.fw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.fws + ((size_t)pid << LOGN);
    const int t = threadIdx.x;
    uint32_t x[W];
    {
        const ntt::RowSrc src = DENSE    ? ntt::RowSrc{(const uint32_t*)A.base + ((size_t)i << LOGN), 1, 0}
                                : A.soff ? ntt::RowSrc{(const uint32_t*)A.src + ((size_t)A.soff[i] << LOGN), A.snum,
                                                       A.sstride}
                                         : ntt::RowSrc{(const uint32_t*)A.base + ((size_t)A.roff[i] << LOGN), 1, 0};
        if (src.n == 1) {
#pragma unroll
            for (int j = 0; j < W; ++j) x[j] = src.p0[t + T * j];
        } else {
#pragma unroll
            for (int j = 0; j < W; ++j) x[j] = ntt::ld_src(src, t + T * j, p);
        }
    }
    // P1: lh = 15..11 (LB = lh - 10), index 2^(5 - LB) + g
    stage<true, H, 5, 0, true>(x, w, ws, 1, p, p2);
    stage<true, H, 4, 0, true>(x, w, ws, 2, p, p2);
    stage<true, H, 3, 0, true>(x, w, ws, 4, p, p2);
    stage<true, H, 2, 0, true>(x, w, ws, 8, p, p2);
    stage<true, H, 1, 0, true>(x, w, ws, 16, p, p2);
    x1_fwd(x, lds, t);
    // P2: lh = 10..5 (LB = lh - 5), index 2^(10 - LB) + a 2^(5 - LB) + g
    {
        const uint32_t a = (uint32_t)t >> 5;
        stage<true, H, 5, 1, false>(x, w, ws, 32 + a, p, p2);
        stage<true, H, 4, 1, false>(x, w, ws, 64 + 2 * a, p, p2);
        stage<true, H, 3, 1, false>(x, w, ws, 128 + 4 * a, p, p2);
        stage<true, H, 2, 1, false>(x, w, ws, 256 + 8 * a, p, p2);
        stage<true, H, 1, 1, false>(x, w, ws, 512 + 16 * a, p, p2);
        stage<true, H, 0, 1, false>(x, w, ws, 1024 + 32 * a, p, p2);
    }
    x2_fwd(x, lds, t);
    // P3: lh = 4..0 (LB = lh), index 2^(15 - LB) + t 2^(5 - LB) + g
    {
        const uint32_t u = (uint32_t)t;
        stage<true, H, 4, 2, false>(x, w, ws, 2048 + 2 * u, p, p2);
        stage<true, H, 3, 2, false>(x, w, ws, 4096 + 4 * u, p, p2);
        stage<true, H, 2, 2, false>(x, w, ws, 8192 + 8 * u, p, p2);
        stage<true, H, 1, 2, false>(x, w, ws, 16384 + 16 * u, p, p2);
        stage<true, H, 0, 2, false>(x, w, ws, 32768 + 32 * u, p, p2);
    }
    const size_t r0 = ((DENSE ? (size_t)i : (size_t)A.roff[i]) << LOGN) + (size_t)W * t;
    if (EPI == 0) {
        uint4* o = (uint4*)((uint32_t*)A.base + r0);
#pragma unroll
        for (int k = 0; k < W / 4; ++k)
            o[k] = make_uint4(ntt::canon<H>(x[phys(2, 4 * k)], p, p2), ntt::canon<H>(x[phys(2, 4 * k + 1)], p, p2),
                              ntt::canon<H>(x[phys(2, 4 * k + 2)], p, p2), ntt::canon<H>(x[phys(2, 4 * k + 3)], p, p2));
        return;
    }
    const uint32_t s = ((const uint32_t*)A.es)[pid], ss = ((const uint32_t*)A.ess)[pid];
    uint32_t* o = (uint32_t*)A.eout + r0;
    const uint32_t* xv = (const uint32_t*)A.ex + r0;  // one operand row (xnum == 1: the launcher's condition)
    // the epilogue's operands are read 16 words at a time after the butterflies (scheduling fences keep the loads from
    // being hoisted above them, where 64 more live words would spill)
#pragma unroll
    for (int q = 0; q < W / E; ++q) {
        __builtin_amdgcn_sched_barrier(0);
        uint32_t ex[E], d[E], y[E];
        ld16(xv + E * q, ex);
        if (EPI == 2) ld16(A.ed ? (const uint32_t*)A.ed + r0 + E * q : o + E * q, d);
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const uint32_t v = ntt::canon<H>(x[phys(2, E * q + j)], p, p2);
            if (EPI == 3) {
                y[j] = addm(shoup(ex[j], s, ss, p), v, p);
            } else {
                const uint32_t z = shoup(ex[j] - v + p, s, ss, p);
                y[j] = EPI == 2 ? addm(d[j], z, p) : z;
            }
        }
        st16(o + E * q, y);
    }
}

// Inverse transform of one row per workgroup, scaled by es[row] (NttArgs ABI 17) or the prime's N^-1.
template <bool H>
__global__ void __launch_bounds__(T) inv1(NttArgs A, int row0) {
    __shared__ uint32_t lds[LDSW];
    const int i = row_of(row0);
    const int pid = A.rprime[i];
    const uint32_t p = (uint32_t)A.pr[pid].p, p2 = 2 * p;
    const uint32_t* w = (const uint32_t*)A.iw + ((size_t)pid << LOGN);
    const uint32_t* ws = (const uint32_t*)A.iws + ((size_t)pid << LOGN);
    const int t = threadIdx.x;
    uint32_t x[W];
    {
        const ntt::RowSrc src = A.soff ? ntt::RowSrc{(const uint32_t*)A.src + ((size_t)A.soff[i] << LOGN), A.snum,
                                                      A.sstride}
                                       : ntt::RowSrc{(const uint32_t*)A.base + ((size_t)A.roff[i] << LOGN), 1, 0};
#pragma unroll
        for (int q = 0; q < W / E; ++q) {
            uint32_t y[E];
            ntt::ld16_src(src, (size_t)W * t + E * q, p, y);
#pragma unroll
            for (int j = 0; j < E; ++j) x[E * q + j] = y[j];
        }
    }
    {
        const uint32_t u = (uint32_t)t;
        stage<false, H, 0, 0, false>(x, w, ws, 32768 + 32 * u, p, p2);
        stage<false, H, 1, 0, false>(x, w, ws, 16384 + 16 * u, p, p2);
        stage<false, H, 2, 0, false>(x, w, ws, 8192 + 8 * u, p, p2);
        stage<false, H, 3, 0, false>(x, w, ws, 4096 + 4 * u, p, p2);
        stage<false, H, 4, 0, false>(x, w, ws, 2048 + 2 * u, p, p2);
    }
    x2_inv(x, lds, t);
    {
        const uint32_t a = (uint32_t)t >> 5;
        stage<false, H, 0, 3, false>(x, w, ws, 1024 + 32 * a, p, p2);
        stage<false, H, 1, 3, false>(x, w, ws, 512 + 16 * a, p, p2);
        stage<false, H, 2, 3, false>(x, w, ws, 256 + 8 * a, p, p2);
        stage<false, H, 3, 3, false>(x, w, ws, 128 + 4 * a, p, p2);
        stage<false, H, 4, 3, false>(x, w, ws, 64 + 2 * a, p, p2);
        stage<false, H, 5, 3, false>(x, w, ws, 32 + a, p, p2);
    }
    x1_inv(x, lds, t);
    stage<false, H, 1, 4, true>(x, w, ws, 16, p, p2);
    stage<false, H, 2, 4, true>(x, w, ws, 8, p, p2);
    stage<false, H, 3, 4, true>(x, w, ws, 4, p, p2);
    stage<false, H, 4, 4, true>(x, w, ws, 2, p, p2);
    stage<false, H, 5, 4, true>(x, w, ws, 1, p, p2);
    uint32_t s, ss;
    if (A.es) {
        s = ((const uint32_t*)A.es)[i];
        ss = ((const uint32_t*)A.ess)[i];
    } else {
        s = ((const uint32_t*)A.ninv)[pid];
        ss = ((const uint32_t*)A.ninvs)[pid];
    }
    uint32_t* o = (uint32_t*)A.base + ((size_t)A.roff[i] << LOGN);
#pragma unroll
    for (int j = 0; j < W; ++j) o[t + T * j] = shoup(x[phys(4, j)], s, ss, p);
}

}  // namespace ntt1

// Launchers over rows [r0, r0 + n) of the args (checked by the caller).
void ntt1_fwd(const NttArgs& A, int r0, int n, pc_stream_t s) {
    hipStream_t st = (hipStream_t)s;
    const dim3 g(n), b(ntt1::T);
#define PCH_F1(HH)                                                                                \
    switch (A.epi) {                                                                              \
        case 0: hipLaunchKernelGGL((ntt1::fwd1<HH, 0>), g, b, 0, st, A, r0); break;               \
        case 1: hipLaunchKernelGGL((ntt1::fwd1<HH, 1>), g, b, 0, st, A, r0); break;               \
        case 2: hipLaunchKernelGGL((ntt1::fwd1<HH, 2>), g, b, 0, st, A, r0); break;               \
        default: hipLaunchKernelGGL((ntt1::fwd1<HH, 3>), g, b, 0, st, A, r0); break;              \
    }
    if (!A.roff) {  // dense rows (internal launches, epilogue 0, non-lazy)
        hipLaunchKernelGGL((ntt1::fwd1<false, 0, true>), g, b, 0, st, A, r0);
    } else if (A.lazy) {
        PCH_F1(true)
    } else {
        PCH_F1(false)
    }
#undef PCH_F1
}

void ntt1_inv(const NttArgs& A, int r0, int n, pc_stream_t s) {
    hipStream_t st = (hipStream_t)s;
    if (A.lazy) hipLaunchKernelGGL((ntt1::inv1<true>), dim3(n), dim3(ntt1::T), 0, st, A, r0);
    else hipLaunchKernelGGL((ntt1::inv1<false>), dim3(n), dim3(ntt1::T), 0, st, A, r0);
}

}  // namespace pch
