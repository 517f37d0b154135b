// EvalMod and plaintext-product element-wise kernels: the tensor product of two ciphertexts, the ModDown / rescale
// epilogues, weighted sums, constants, plaintext-table products and their fused add / sub chains, and the
// pointer-list sums (semantics: crates/pc-kernels/kernels/args.cuh TensorArgs .. SubMulManyArgs :162-579; kernels
// em.cuh:12-575, rescale.cuh:63-77; host twin crates/pc-host/src/elem.rs:109-636).
//
// Q rows [0, n) of K ciphertexts, row index = prime id. Every kernel streams rows once: grid (N / 1024, rows, K or
// K x 2 parts), 256 threads, each owning 4 consecutive words of a row (16-byte accesses; rows are N-word aligned). The
// sums of products are accumulated exactly (a 64-bit sum and its carry count, reduced once), so every output is the
// canonical residue of the stated formula whatever the number of terms; the reference's lazy 64-bit sums give the same
// words inside the bounds its callers keep (2 npairs (p - 1)^2 < 2^64, nterm p^2 < 2^64).
#include "common.h"
#include "fused.h"

namespace pch {
namespace em {

constexpr int BX = 256;

struct W4 {
    uint32_t v[4];
};
__device__ __forceinline__ W4 ld4(const uint32_t* p) {
    const uint4 t = *(const uint4*)p;
    return W4{{t.x, t.y, t.z, t.w}};
}
__device__ __forceinline__ void st4(uint32_t* p, const W4& w) { *(uint4*)p = make_uint4(w.v[0], w.v[1], w.v[2], w.v[3]); }
__device__ __forceinline__ uint32_t* at(const PolyRef& r, int c, int part, int row, int logn) {
    return (uint32_t*)r.base + c * r.ct_stride + part * r.part_stride + ((size_t)row << logn);
}
__device__ __forceinline__ uint32_t lane_word() { return (blockIdx.x * BX + threadIdx.x) * 4; }
__device__ __forceinline__ uint32_t red_once(uint32_t k, uint32_t p) { return k >= p ? k - p : k; }

// An exact sum of 64-bit products: lo + hi 2^64
struct Acc {
    uint64_t lo = 0;
    uint32_t hi = 0;
    __device__ __forceinline__ void add(uint64_t v) {
        lo += v;
        hi += lo < v;
    }
    __device__ __forceinline__ uint32_t red(const Red& r) const { return r.red96(lo, hi); }
};
// The same sum in two instructions per product: the 64-bit product-sum a b + lo, then its carry-out added into hi
struct Acc2 {
    uint64_t lo = 0;
    uint32_t hi = 0;
    __device__ __forceinline__ void mad(uint32_t a, uint32_t b) {
        uint64_t s, c, c2;
        asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=v"(s), "=s"(c) : "v"(a), "v"(b), "v"(lo));
        asm("v_addc_co_u32 %0, %1, %2, 0, %3" : "=v"(hi), "=s"(c2) : "v"(hi), "s"(c));
        lo = s;
    }
    __device__ __forceinline__ uint32_t red(const Red& r) const { return r.red96(lo, hi); }
};

// Acc2, or (NARROW: the row's prime below 2^30, so that up to 8 products of (p - 1)^2 < 2^60 stay below 2^63) a plain
// 64-bit sum, one multiply-add per product and no carry
template <bool NARROW>
struct AccN {
    Acc2 a;
    __device__ __forceinline__ void mad(uint32_t x, uint32_t y) {
        if constexpr (NARROW) a.lo += (uint64_t)x * y;
        else a.mad(x, y);
    }
    __device__ __forceinline__ uint32_t red(const Red& r) const { return NARROW ? r(a.lo) : a.red(r); }
};

// ------------------------------------------------------------------------------------------------ tensor
// (c0, c1, d2) = sum_j (a_j0 b_j0, a_j0 b_j1 + a_j1 b_j0, a_j1 b_j1) over the pairs (the operands of pair j: A[j], B[j])
struct Tacc {
    Acc s0[4], s1[4], s2[4];
    __device__ __forceinline__ void mac(const W4& x0, const W4& x1, const W4& y0, const W4& y1) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            s0[w].add((uint64_t)x0.v[w] * y0.v[w]);
            s1[w].add((uint64_t)x0.v[w] * y1.v[w]);
            s1[w].add((uint64_t)x1.v[w] * y0.v[w]);
            s2[w].add((uint64_t)x1.v[w] * y1.v[w]);
        }
    }
};

// The tail shared by tensor, tensor_y and tensor_sum: reduce, += the old words (acc; d2 with acc2), double (dbl),
// +- y c (tensor_y), store; every input word is read before the first store, so outputs may alias inputs.
__device__ __forceinline__ void tensor_tail(const Tacc& s, const Red& red, uint32_t* o0, uint32_t* o1, uint32_t* o2,
                                            bool acc, bool acc2, bool dbl, const uint32_t* y0p, const uint32_t* y1p,
                                            uint32_t yc, uint32_t ycs, bool ysub, uint32_t* coef) {
    const uint32_t p = red.p;
    W4 r0, r1, r2;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        r0.v[w] = s.s0[w].red(red);
        r1.v[w] = s.s1[w].red(red);
        r2.v[w] = s.s2[w].red(red);
    }
    if (acc) {
        const W4 d0 = ld4(o0), d1 = ld4(o1);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            r0.v[w] = addm(r0.v[w], d0.v[w], p);
            r1.v[w] = addm(r1.v[w], d1.v[w], p);
        }
    }
    if (acc2) {
        const W4 d2 = ld4(o2);
#pragma unroll
        for (int w = 0; w < 4; ++w) r2.v[w] = addm(r2.v[w], d2.v[w], p);
    }
    if (dbl) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            r0.v[w] = addm(r0.v[w], r0.v[w], p);
            r1.v[w] = addm(r1.v[w], r1.v[w], p);
            r2.v[w] = addm(r2.v[w], r2.v[w], p);
        }
    }
    if (y0p) {
        const W4 y0 = ld4(y0p), y1 = ld4(y1p);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t m0 = shoup(y0.v[w], yc, ycs, p), m1 = shoup(y1.v[w], yc, ycs, p);
            r0.v[w] = ysub ? subm(r0.v[w], m0, p) : addm(r0.v[w], m0, p);
            r1.v[w] = ysub ? subm(r1.v[w], m1, p) : addm(r1.v[w], m1, p);
        }
    }
    st4(o0, r0);
    st4(o1, r1);
    st4(o2, r2);
    if (coef) st4(coef, r2);
}

template <bool Y>
__global__ void __launch_bounds__(BX) tensor_k(TensorArgs A, TensorYArgs B, int logn) {
    const int row = blockIdx.y, c = blockIdx.z;
    const uint32_t i = lane_word();
    const Red red(A.pr[row]);
    Tacc s;
    const int np = A.npairs < 2 ? A.npairs : 2;
    for (int j = 0; j < np; ++j) {
        const PolyRef& a = j ? A.a1 : A.a0;
        const PolyRef& b = j ? A.b1 : A.b0;
        s.mac(ld4(at(a, c, 0, row, logn) + i), ld4(at(a, c, 1, row, logn) + i), ld4(at(b, c, 0, row, logn) + i),
              ld4(at(b, c, 1, row, logn) + i));
    }
    uint32_t* coef = A.coef ? (uint32_t*)A.coef + c * A.coef_ct_stride + ((size_t)row << logn) + i : nullptr;
    tensor_tail(s, red, at(A.out, c, 0, row, logn) + i, at(A.out, c, 1, row, logn) + i, at(A.d2, c, 1, row, logn) + i,
                A.acc != 0, A.acc_d2 != 0, A.dbl != 0, Y ? at(B.y, c, 0, row, logn) + i : nullptr,
                Y ? at(B.y, c, 1, row, logn) + i : nullptr, Y ? ((const uint32_t*)B.c)[row] : 0u,
                Y ? ((const uint32_t*)B.cs)[row] : 0u, Y && B.sub != 0, coef);
}

// the tensor of K pairs at their own addresses: ciphertext c = blockIdx.z reads a[c], b[c]
__global__ void __launch_bounds__(BX) tensor_list_k(TensorListArgs A, int logn) {
    const int row = blockIdx.y, c = blockIdx.z;
    const uint32_t i = lane_word();
    const Red red(A.pr[row]);
    const size_t ro = ((size_t)row << logn) + i;
    // product c's pairs (one, or a summed range): the sums exact over any number of pairs
    const int j0 = A.sum ? A.off[c] : c, j1 = A.sum ? A.off[c + 1] : c + 1;
    Tacc s;
    for (int j = j0; j < j1; ++j) {
        const uint32_t *a = A.a[j] + ro, *b = A.b[j] + ro;
        s.mac(ld4(a), ld4(a + A.part), ld4(b), ld4(b + A.part));
    }
    uint32_t* o = A.out + c * A.ct_stride + ro;
    // the addend's words times its row's multiplier (a Shoup product; none: 1 with companion 0, each canonical word
    // unchanged)
    const uint32_t* y = A.y[c];
    const uint32_t* yk = A.yk[c];
    const uint32_t ym = yk ? yk[row] : 1u, yms = yk ? yk[A.krows + row] : 0u;
    tensor_tail(s, red, o, o + A.part, A.d2 + c * A.ct_stride + A.part + ro, false, false, A.dbl != 0,
                y ? y + ro : nullptr, y ? y + A.part + ro : nullptr, ym, yms, (A.ysub >> c) & 1u, nullptr);
}

__global__ void __launch_bounds__(BX) tensor_sum_k(TensorSumArgs A, int logn) {
    const int row = blockIdx.y, c = blockIdx.z;
    const uint32_t i = lane_word();
    const Red red(A.pr[row]);
    Tacc s;
    for (int j = 0; j < A.npairs; ++j)
        s.mac(ld4(at(A.a[j], c, 0, row, logn) + i), ld4(at(A.a[j], c, 1, row, logn) + i),
              ld4(at(A.b[j], c, 0, row, logn) + i), ld4(at(A.b[j], c, 1, row, logn) + i));
    tensor_tail(s, red, at(A.out, c, 0, row, logn) + i, at(A.out, c, 1, row, logn) + i, at(A.d2, c, 1, row, logn) + i,
                A.acc != 0, (A.acc & 2) != 0, false, nullptr, nullptr, 0u, 0u, false, nullptr);
}

// ------------------------------------------------------------------------------------------------ epilogues
// dst = f (dst + (x - t) binv) [+ k], or (TO) dst = a +- (x - t) binv
template <bool TO>
__global__ void __launch_bounds__(BX) md_epi_k(MdEpiToArgs B, int logn) {
    const MdEpiArgs& A = B.m;
    const int row = blockIdx.y, c = blockIdx.z >> 1, part = blockIdx.z & 1;
    const uint32_t i = lane_word();
    const uint32_t p = (uint32_t)A.pr[row].p;
    const uint32_t bi = ((const uint32_t*)A.binv)[row], bis = ((const uint32_t*)A.binvs)[row];
    uint32_t* d = at(A.dst, c, part, row, logn) + i;
    const W4 x = ld4(at(A.x, c, part, row, logn) + i), t = ld4(at(A.t, c, part, row, logn) + i);
    const W4 base = ld4(TO ? at(B.a, c, part, row, logn) + i : d);
    const bool addk = !TO && A.k && part == 0;
    const uint32_t kk = addk ? red_once(((const uint32_t*)A.k)[row], p) : 0u;
    W4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t v = shoup(subm(x.v[w], t.v[w], p), bi, bis, p);
        if (TO) {
            r.v[w] = B.sub ? subm(base.v[w], v, p) : addm(base.v[w], v, p);
        } else {
            uint32_t u = addm(base.v[w], v, p);
            if (A.dbl) u = addm(u, u, p);
            r.v[w] = addk ? addm(u, kk, p) : u;
        }
    }
    st4(d, r);
}

// ------------------------------------------------------------------------------------------------ weighted sums
// out[m] = sum_j w[m][j rowstride + row] src_j [+ k[m][row] on part 0] for the outputs m whose row range holds row
__global__ void __launch_bounds__(BX) wsum_k(WsumMultiArgs A, int logn) {
    const int row = blockIdx.y, c = blockIdx.z;
    const uint32_t i = lane_word();
    const uint32_t p = (uint32_t)A.pr[row].p;
    W4 r[3][2] = {};
    bool on[3];
#pragma unroll
    for (int m = 0; m < 3; ++m) on[m] = m < A.nout && row < A.n[m];
    for (int j = 0; j < A.nsrc; ++j) {
        const W4 x0 = ld4(at(A.src[j], c, 0, row, logn) + i), x1 = ld4(at(A.src[j], c, 1, row, logn) + i);
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            if (!on[m]) continue;
            const uint32_t w = ((const uint32_t*)A.w[m])[j * A.rowstride + row];
            const uint32_t ws = ((const uint32_t*)A.ws[m])[j * A.rowstride + row];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                r[m][0].v[u] = addm(r[m][0].v[u], shoup(x0.v[u], w, ws, p), p);
                r[m][1].v[u] = addm(r[m][1].v[u], shoup(x1.v[u], w, ws, p), p);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) {
        if (!on[m]) continue;
        if (A.k[m]) {
            const uint32_t kr = red_once(((const uint32_t*)A.k[m])[row], p);
#pragma unroll
            for (int u = 0; u < 4; ++u) r[m][0].v[u] = addm(r[m][0].v[u], kr, p);
        }
        st4(at(A.out[m], c, 0, row, logn) + i, r[m][0]);
        st4(at(A.out[m], c, 1, row, logn) + i, r[m][1]);
    }
}

// ------------------------------------------------------------------------------------------------ constants, tables
__global__ void __launch_bounds__(BX) add_const_k(AddConstArgs A, int logn) {
    const int row = blockIdx.y, c = blockIdx.z;
    const uint32_t p = (uint32_t)A.pr[row].p;
    uint32_t* d = at(A.x, c, 0, row, logn) + lane_word();
    const uint32_t kr = red_once(((const uint32_t*)A.k)[row], p);
    W4 x = ld4(d);
#pragma unroll
    for (int w = 0; w < 4; ++w) x.v[w] = addm(x.v[w], kr, p);
    st4(d, x);
}

// out = y op sum_j x_j t_j (MODE 0: y + s, 1: y - s, 2: s - y; Y: whether y is read); one term is mul_table / mul_add
template <int MODE, bool Y>
__global__ void __launch_bounds__(BX) mul_k(MulAddNArgs A, int logn) {
    const int row = blockIdx.y, part = blockIdx.z & 1, c = blockIdx.z >> 1;
    const uint32_t i = lane_word();
    const Red red(A.pr[row]);
    const uint32_t p = red.p;
    Acc s[4];
    for (int j = 0; j < A.nterm; ++j) {
        const W4 x = ld4(at(A.x[j], c, part, row, logn) + i);
        const W4 t = ld4((const uint32_t*)A.t[j] + ((size_t)row << logn) + i);
#pragma unroll
        for (int w = 0; w < 4; ++w) s[w].add((uint64_t)x.v[w] * t.v[w]);
    }
    W4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r.v[w] = s[w].red(red);
    if (Y) {
        const W4 y = ld4(at(A.y, c, part, row, logn) + i);
#pragma unroll
        for (int w = 0; w < 4; ++w)
            r.v[w] = MODE == 0 ? addm(y.v[w], r.v[w], p) : MODE == 1 ? subm(y.v[w], r.v[w], p) : subm(r.v[w], y.v[w], p);
    }
    st4(at(A.out, c, part, row, logn) + i, r);
}

// out[c] = in[c] t[c] on both parts (ciphertext c = blockIdx.z >> 1, its own plaintext)
__global__ void __launch_bounds__(BX) mul_pt_list_k(MulPtListArgs A, int logn) {
    const int row = blockIdx.y, part = blockIdx.z & 1, c = blockIdx.z >> 1;
    const size_t ro = ((size_t)row << logn) + lane_word();
    const Red red(A.pr[row]);
    const W4 x = ld4(A.in + c * A.ct_stride + part * A.part + ro);
    const W4 t = ld4(A.t[c] + ro);
    W4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r.v[w] = red((uint64_t)x.v[w] * t.v[w]);
    st4(A.out + c * A.ct_stride + part * A.part + ro, r);
}

// x_i = alpha_i x_i + tmp_i (rescale_combine), or out_i = alpha_i x_i + tmp_i (rescale_combine_to)
__global__ void __launch_bounds__(BX) combine_k(RescaleCombineToArgs R, int logn) {
    const RescaleCombineArgs& A = R.a;
    const int row = blockIdx.y, c = blockIdx.z >> 1, part = blockIdx.z & 1;
    const uint32_t i = lane_word();
    const uint32_t p = (uint32_t)A.pr[row].p;
    const uint32_t al = ((const uint32_t*)A.alpha)[row], als = ((const uint32_t*)A.alphas)[row];
    const W4 x = ld4(at(A.x, c, part, row, logn) + i), t = ld4(at(A.tmp, c, part, row, logn) + i);
    W4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r.v[w] = addm(shoup(x.v[w], al, als, p), t.v[w], p);
    st4(at(R.out, c, part, row, logn) + i, r);
}

// ------------------------------------------------------------------------------------------------ pointer lists
__global__ void __launch_bounds__(BX) ew_many_k(EwManyArgs A, int logn) {
    const int row = blockIdx.y, j = blockIdx.z;
    const size_t o = ((size_t)row << logn) + lane_word();
    const uint32_t p = (uint32_t)A.pr[row].p;
    W4 r = ld4((const uint32_t*)A.a[j] + o);
    if (A.b[j]) {
        const W4 y = ld4((const uint32_t*)A.b[j] + o);
#pragma unroll
        for (int w = 0; w < 4; ++w) r.v[w] = addm(r.v[w], y.v[w], p);
    }
    if (A.c[j]) {
        const W4 y = ld4((const uint32_t*)A.c[j] + o);
#pragma unroll
        for (int w = 0; w < 4; ++w) r.v[w] = addm(r.v[w], y.v[w], p);
    }
    st4((uint32_t*)A.out[j] + o, r);
}

__global__ void __launch_bounds__(BX) submul_many_k(SubMulManyArgs A, int logn) {
    const int row = blockIdx.y, j = blockIdx.z;
    const size_t o = ((size_t)row << logn) + lane_word();
    const Red red(A.pr[row]);
    const W4 x = ld4((const uint32_t*)A.a[j] + o), y = ld4((const uint32_t*)A.b[j] + o);
    const W4 t = ld4((const uint32_t*)A.t + o);
    W4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r.v[w] = red.mul(subm(x.v[w], y.v[w], red.p), t.v[w]);
    st4((uint32_t*)A.out[j] + o, r);
}

// ------------------------------------------------------------------------------------------------ BSGS plaintext dot
// res[c][j] = sum_{b < bstep} rot[c][b] pt_{bstep j + b}[prow][ptidx(i, enc)] on the row set's rows (args.cuh:184-198;
// elem.cuh:83-118): rotations and results by PolyRef plus the per-rotation / per-result strides, diagonals >= npts
// skipped; prow = y on Q rows, pt_prow + (y - nq) on special rows. 4 consecutive slots per thread, one ciphertext at a
// time, the sums exact.
//
// The register form: a thread's words of BM rotations stay in registers across the giant steps, so each rotation word
// is read from HBM once (re-reading them per giant step cost bstep x 2 rows per giant step), and each giant step
// issues all its diagonal loads before the first product. More than BM baby steps go in groups of BM: a later group's
// sums are added onto the results the earlier groups stored (the same thread's words: two result rows per giant step
// and group, against bstep rotation rows per giant step re-read). The diagonal pointers are loaded through the
// scalar cache and the words as global (not flat) loads, so no wait on one serialises the others. MODE 0: full-width
// diagonals (words i .. i + 3 in one 16-byte load); 1: compact by a shift s >= 2 (the thread's 4 words share one
// diagonal word); 2: any other index form (a load per word).
template <int BM, int MODE, bool NARROW>
__device__ __forceinline__ void pt_dot_reg_body(const PtDotArgs& A, int logn) {
    typedef const __attribute__((address_space(4))) uint64_t* ConstTab;
    typedef const __attribute__((address_space(1))) uint32_t* GPtr;
    typedef uint32_t U4 __attribute__((ext_vector_type(4)));
    const int y = blockIdx.y;
    const int row = y < A.rs.nq ? y : A.rs.qmax + (y - A.rs.nq);
    const int prow = y < A.rs.nq ? y : A.pt_prow + (y - A.rs.nq);
    const Red red(A.pr[row]);
    const uint32_t i = lane_word();
    uint32_t pi[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) pi[w] = ptidx(i + w, A.enc);
    const size_t roff = ((size_t)row << logn) + i;
    // the rotations read: b < bstep and b < npts (npts >= 1); the loads past them re-read rotation 0, never used
    const int nb = min(A.bstep, A.npts);
    const ConstTab tab = (ConstTab)A.pts;
    for (int c = 0; c < A.K; ++c)
      for (int b0 = 0; b0 < nb; b0 += BM) {
        W4 x0[BM], x1[BM];
#pragma unroll
        for (int b = 0; b < BM; ++b) {
            const uint32_t* r = (const uint32_t*)A.rot.base + c * A.rot.ct_stride +
                                (b0 + b < nb ? b0 + b : 0) * A.rot_stride + roff;
            x0[b] = ld4(r);
            x1[b] = ld4(r + A.rot.part_stride);
        }
        for (int j = 0; j < A.gstep; ++j) {
            // a missing diagonal (b0 + b >= nb or d >= npts) reads diagonal 0 and weighs 0
            uint64_t pp[BM];
#pragma unroll
            for (int b = 0; b < BM; ++b) {
                const int d = A.bstep * j + b0 + b;
                pp[b] = tab[b0 + b < nb && d < A.npts ? d : 0];
            }
            W4 pw[BM];
#pragma unroll
            for (int b = 0; b < BM; ++b) {
                const int d = A.bstep * j + b0 + b;
                const bool ok = b0 + b < nb && d < A.npts;
                const GPtr pt = (GPtr)pp[b] + (size_t)prow * A.ptw;
                if constexpr (MODE == 0) {
                    const U4 u = *(const __attribute__((address_space(1))) U4*)(pt + i);
#pragma unroll
                    for (int w = 0; w < 4; ++w) pw[b].v[w] = u[w];
                } else if constexpr (MODE == 1) {
                    const uint32_t v = pt[pi[0]];
#pragma unroll
                    for (int w = 0; w < 4; ++w) pw[b].v[w] = v;
                } else {
#pragma unroll
                    for (int w = 0; w < 4; ++w) pw[b].v[w] = pt[pi[w]];
                }
#pragma unroll
                for (int w = 0; w < 4; ++w) pw[b].v[w] = ok ? pw[b].v[w] : 0u;
            }
            AccN<NARROW> s0[4], s1[4];
#pragma unroll
            for (int b = 0; b < BM; ++b) {
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    s0[w].mad(x0[b].v[w], pw[b].v[w]);
                    s1[w].mad(x1[b].v[w], pw[b].v[w]);
                }
            }
            W4 r0, r1;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                r0.v[w] = s0[w].red(red);
                r1.v[w] = s1[w].red(red);
            }
            uint32_t* o = (uint32_t*)A.res.base + c * A.res.ct_stride + j * A.res_stride + roff;
            if (b0 > 0) {
                // the earlier groups' sums, stored by this thread
                const W4 e0 = ld4(o), e1 = ld4(o + A.res.part_stride);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    r0.v[w] = addm(r0.v[w], e0.v[w], red.p);
                    r1.v[w] = addm(r1.v[w], e1.v[w], red.p);
                }
            }
            st4(o, r0);
            st4(o + A.res.part_stride, r1);
        }
      }
}
template <int BM, int MODE>
__global__ void __launch_bounds__(BX) pt_dot_reg_k(PtDotArgs A, int logn) {
    const int y = blockIdx.y;
    const int row = y < A.rs.nq ? y : A.rs.qmax + (y - A.rs.nq);
    // the branch is uniform over the workgroup (one row per grid row)
    if ((uint32_t)A.pr[row].p < (1u << 30)) pt_dot_reg_body<BM, MODE, true>(A, logn);
    else pt_dot_reg_body<BM, MODE, false>(A, logn);
}

// no diagonals: the rotations re-read per giant step
__global__ void __launch_bounds__(BX) pt_dot_k(PtDotArgs A, int logn) {
    const int y = blockIdx.y;
    const int row = y < A.rs.nq ? y : A.rs.qmax + (y - A.rs.nq);
    const int prow = y < A.rs.nq ? y : A.pt_prow + (y - A.rs.nq);
    const Red red(A.pr[row]);
    const uint32_t i = lane_word();
    uint32_t pi[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) pi[w] = ptidx(i + w, A.enc);
    const size_t roff = ((size_t)row << logn) + i;
    for (int c = 0; c < A.K; ++c) {
        for (int j = 0; j < A.gstep; ++j) {
            Acc s0[4], s1[4];
            for (int b = 0; b < A.bstep; ++b) {
                const int d = A.bstep * j + b;
                if (d >= A.npts) break;
                const uint32_t* pt = (const uint32_t*)A.pts[d] + (size_t)prow * A.ptw;
                const uint32_t* r = (const uint32_t*)A.rot.base + c * A.rot.ct_stride + b * A.rot_stride + roff;
                const W4 x0 = ld4(r), x1 = ld4(r + A.rot.part_stride);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t pw = pt[pi[w]];
                    s0[w].add((uint64_t)x0.v[w] * pw);
                    s1[w].add((uint64_t)x1.v[w] * pw);
                }
            }
            W4 r0, r1;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                r0.v[w] = s0[w].red(red);
                r1.v[w] = s1[w].red(red);
            }
            uint32_t* o = (uint32_t*)A.res.base + c * A.res.ct_stride + j * A.res_stride + roff;
            st4(o, r0);
            st4(o + A.res.part_stride, r1);
        }
    }
}

// ------------------------------------------------------------------------------------------------ launchers
// The reference's launchers check only the counts below (em.cuh:580-692); these also refuse null operands that the
// kernel would read (-1), pt_dot's diagonal indices outside its rows of ptw words (-1), and return 0 without a launch
// when there is no work.
template <int LOGN>
dim3 grid(int rows, int z) {
    return dim3((1u << LOGN) / (BX * 4), (unsigned)rows, (unsigned)z);
}
#define PCH_LAUNCH(kern, g, ...)                                                   \
    do {                                                                           \
        hipLaunchKernelGGL(kern, g, dim3(BX), 0, (hipStream_t)s, __VA_ARGS__);     \
        return launch_rc();                                                        \
    } while (0)

inline bool ref_ok(const PolyRef& r) { return r.base != nullptr; }

template <int LOGN>
int tensor(const TensorArgs* a, pc_stream_t s) {
    if (!a || !a->pr || !ref_ok(a->out) || !ref_ok(a->d2) || a->n < 0 || a->K < 0) return -1;
    if (a->npairs >= 1 && (!ref_ok(a->a0) || !ref_ok(a->b0))) return -1;
    if (a->npairs >= 2 && (!ref_ok(a->a1) || !ref_ok(a->b1))) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    PCH_LAUNCH(tensor_k<false>, grid<LOGN>(a->n, a->K), *a, TensorYArgs{}, LOGN);
}
template <int LOGN>
int tensor_list(const TensorListArgs* a, pc_stream_t s) {
    if (!a || !a->pr || !a->out || !a->d2 || a->n < 0 || a->K < 0 || a->K > TLIST_MAX) return -1;
    const int np = a->sum ? a->off[a->K] : a->K;
    if (a->sum) {
        if (a->off[0] != 0) return -1;
        for (int c = 0; c < a->K; ++c)
            if (a->off[c + 1] <= a->off[c] || a->off[c + 1] > TLIST_MAX) return -1;
    }
    for (int c = 0; c < np; ++c)
        if (!a->a[c] || !a->b[c]) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    PCH_LAUNCH(tensor_list_k, grid<LOGN>(a->n, a->K), *a, LOGN);
}
template <int LOGN>
int mul_pt_list(const MulPtListArgs* a, pc_stream_t s) {
    if (!a || !a->pr || !a->in || !a->out || a->n < 0 || a->K < 0 || a->K > TLIST_MAX) return -1;
    for (int c = 0; c < a->K; ++c)
        if (!a->t[c]) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    PCH_LAUNCH(mul_pt_list_k, grid<LOGN>(a->n, 2 * a->K), *a, LOGN);
}
template <int LOGN>
int tensor_y(const TensorYArgs* a, pc_stream_t s) {
    if (!a || !a->c || !a->cs || !ref_ok(a->y)) return -1;
    const TensorArgs& t = a->t;
    if (!t.pr || !ref_ok(t.out) || !ref_ok(t.d2) || t.n < 0 || t.K < 0) return -1;
    if (t.npairs >= 1 && (!ref_ok(t.a0) || !ref_ok(t.b0))) return -1;
    if (t.npairs >= 2 && (!ref_ok(t.a1) || !ref_ok(t.b1))) return -1;
    if (t.n == 0 || t.K == 0) return 0;
    PCH_LAUNCH(tensor_k<true>, grid<LOGN>(t.n, t.K), t, *a, LOGN);
}
template <int LOGN>
int tensor_sum(const TensorSumArgs* a, pc_stream_t s) {
    if (!a || a->npairs < 1 || a->npairs > PC_TSUM_MAX) return -1;
    if (!a->pr || !ref_ok(a->out) || !ref_ok(a->d2) || a->n < 0 || a->K < 0) return -1;
    for (int j = 0; j < a->npairs; ++j)
        if (!ref_ok(a->a[j]) || !ref_ok(a->b[j])) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    PCH_LAUNCH(tensor_sum_k, grid<LOGN>(a->n, a->K), *a, LOGN);
}
inline bool epi_ok(const MdEpiArgs& m) {
    return m.pr && m.binv && m.binvs && ref_ok(m.dst) && ref_ok(m.x) && ref_ok(m.t) && m.n >= 0 && m.K >= 0;
}
template <int LOGN>
int md_epilogue(const MdEpiArgs* a, pc_stream_t s) {
    if (!a || !epi_ok(*a)) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    MdEpiToArgs b{};
    b.m = *a;
    PCH_LAUNCH(md_epi_k<false>, grid<LOGN>(a->n, 2 * a->K), b, LOGN);
}
template <int LOGN>
int md_epilogue_to(const MdEpiToArgs* a, pc_stream_t s) {
    if (!a || !epi_ok(a->m) || !ref_ok(a->a)) return -1;
    if (a->m.n == 0 || a->m.K == 0) return 0;
    PCH_LAUNCH(md_epi_k<true>, grid<LOGN>(a->m.n, 2 * a->m.K), *a, LOGN);
}
inline int wsum_check(const WsumArgs& w) {
    if (w.nsrc < 0 || w.nsrc > 8 || !w.pr || !ref_ok(w.out) || w.n < 0 || w.K < 0) return -1;
    if (w.nsrc > 0 && (!w.w || !w.ws)) return -1;
    for (int j = 0; j < w.nsrc; ++j)
        if (!ref_ok(w.src[j])) return -1;
    return 0;
}
inline WsumMultiArgs wsum_one(const WsumArgs& w, const void* k) {
    WsumMultiArgs m{};
    m.out[0] = w.out;
    for (int j = 0; j < 8; ++j) m.src[j] = w.src[j];
    m.w[0] = w.w;
    m.ws[0] = w.ws;
    m.k[0] = k;
    m.pr = w.pr;
    m.nout = 1;
    m.nsrc = w.nsrc;
    m.rowstride = w.rowstride;
    m.K = w.K;
    m.n[0] = m.nmax = w.n;
    return m;
}
template <int LOGN>
int wsum(const WsumArgs* a, pc_stream_t s) {
    if (!a || wsum_check(*a)) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    PCH_LAUNCH(wsum_k, grid<LOGN>(a->n, a->K), wsum_one(*a, nullptr), LOGN);
}
template <int LOGN>
int wsum_kc(const WsumKArgs* a, pc_stream_t s) {
    if (!a || !a->k || wsum_check(a->w)) return -1;
    if (a->w.n == 0 || a->w.K == 0) return 0;
    PCH_LAUNCH(wsum_k, grid<LOGN>(a->w.n, a->w.K), wsum_one(a->w, a->k), LOGN);
}
template <int LOGN>
int wsum_multi(const WsumMultiArgs* a, pc_stream_t s) {
    if (!a || a->nsrc < 1 || a->nsrc > 8 || a->nout < 1 || a->nout > 3) return -1;
    if (!a->pr || a->K < 0 || a->nmax < 0) return -1;
    for (int m = 0; m < a->nout; ++m)
        if (!ref_ok(a->out[m]) || !a->w[m] || !a->ws[m] || a->n[m] > a->nmax) return -1;
    for (int j = 0; j < a->nsrc; ++j)
        if (!ref_ok(a->src[j])) return -1;
    if (a->nmax == 0 || a->K == 0) return 0;
    PCH_LAUNCH(wsum_k, grid<LOGN>(a->nmax, a->K), *a, LOGN);
}
template <int LOGN>
int add_const(const AddConstArgs* a, pc_stream_t s) {
    if (!a || !a->pr || !a->k || !ref_ok(a->x) || a->n < 0 || a->K < 0) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    PCH_LAUNCH(add_const_k, grid<LOGN>(a->n, a->K), *a, LOGN);
}
inline MulAddNArgs mul_one(const MulTableArgs& m, const PolyRef* y) {
    MulAddNArgs n{};
    n.out = m.out;
    if (y) n.y = *y;
    n.x[0] = m.in;
    n.t[0] = m.t;
    n.pr = m.pr;
    n.n = m.n;
    n.K = m.K;
    n.nterm = 1;
    return n;
}
inline bool mul_ok(const MulTableArgs& m) {
    return m.pr && m.t && ref_ok(m.out) && ref_ok(m.in) && m.n >= 0 && m.K >= 0;
}
template <int LOGN>
int mul_table(const MulTableArgs* a, pc_stream_t s) {
    if (!a || !mul_ok(*a)) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    PCH_LAUNCH((mul_k<0, false>), grid<LOGN>(a->n, 2 * a->K), mul_one(*a, nullptr), LOGN);
}
template <int LOGN>
int mul_add(const MulAddArgs* a, pc_stream_t s) {
    if (!a || a->sub < 0 || a->sub > 2 || !mul_ok(a->m) || !ref_ok(a->y)) return -1;
    if (a->m.n == 0 || a->m.K == 0) return 0;
    const dim3 g = grid<LOGN>(a->m.n, 2 * a->m.K);
    const MulAddNArgs n = mul_one(a->m, &a->y);
    if (a->sub == 0) PCH_LAUNCH((mul_k<0, true>), g, n, LOGN);
    if (a->sub == 1) PCH_LAUNCH((mul_k<1, true>), g, n, LOGN);
    PCH_LAUNCH((mul_k<2, true>), g, n, LOGN);
}
template <int LOGN>
int mul_add_n(const MulAddNArgs* a, pc_stream_t s) {
    if (!a || a->nterm < 1 || a->nterm > 8 || !a->pr || !ref_ok(a->out) || a->n < 0 || a->K < 0) return -1;
    for (int j = 0; j < a->nterm; ++j)
        if (!ref_ok(a->x[j]) || !a->t[j]) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    const dim3 g = grid<LOGN>(a->n, 2 * a->K);
    if (a->y.base) PCH_LAUNCH((mul_k<0, true>), g, *a, LOGN);
    PCH_LAUNCH((mul_k<0, false>), g, *a, LOGN);
}
inline bool comb_ok(const RescaleCombineArgs& c) {
    return c.pr && c.alpha && c.alphas && ref_ok(c.x) && ref_ok(c.tmp) && c.n >= 0 && c.K >= 0;
}
template <int LOGN>
int rescale_combine(const RescaleCombineArgs* a, pc_stream_t s) {
    if (!a || !comb_ok(*a)) return -1;
    if (a->n == 0 || a->K == 0) return 0;
    RescaleCombineToArgs r{};
    r.a = *a;
    r.out = a->x;
    PCH_LAUNCH(combine_k, grid<LOGN>(a->n, 2 * a->K), r, LOGN);
}
template <int LOGN>
int rescale_combine_to(const RescaleCombineToArgs* a, pc_stream_t s) {
    if (!a || !comb_ok(a->a) || !ref_ok(a->out)) return -1;
    if (a->a.n == 0 || a->a.K == 0) return 0;
    PCH_LAUNCH(combine_k, grid<LOGN>(a->a.n, 2 * a->a.K), *a, LOGN);
}
template <int LOGN>
int ew_many(const EwManyArgs* a, pc_stream_t s) {
    if (!a || a->n < 1 || a->n > PC_EWM_MAX || !a->pr || a->nrows < 0) return -1;
    for (int j = 0; j < a->n; ++j)
        if (!a->out[j] || !a->a[j]) return -1;
    if (a->nrows == 0) return 0;
    PCH_LAUNCH(ew_many_k, grid<LOGN>(a->nrows, a->n), *a, LOGN);
}
template <int LOGN>
int submul_many(const SubMulManyArgs* a, pc_stream_t s) {
    if (!a || a->n < 1 || a->n > PC_EWM_MAX || !a->pr || !a->t || a->nrows < 0) return -1;
    for (int j = 0; j < a->n; ++j)
        if (!a->out[j] || !a->a[j] || !a->b[j]) return -1;
    if (a->nrows == 0) return 0;
    PCH_LAUNCH(submul_many_k, grid<LOGN>(a->nrows, a->n), *a, LOGN);
}
// tensor_multi: each output's pair list through the tensor_sum kernel, 16 pairs per launch (a longer list continues
// with acc 2 onto the first launch's words: the sums are exact, so the words are those of one pass). The reference
// loads an operand shared by consecutive outputs once (em.cuh:125-197); here each output reads its own.
template <int LOGN>
int tensor_multi(const TensorMultiArgs* a, pc_stream_t s) {
    if (!a || a->nout < 1 || a->nout > PC_TMULTI_OUT || a->npairs < 1 || a->npairs > PC_TMULTI_PAIRS) return -1;
    if (!a->pr || a->n < 0 || a->K < 0) return -1;
    for (int o = 0; o < a->nout; ++o) {
        if (!ref_ok(a->out[o]) || !ref_ok(a->d2[o])) return -1;
        for (int j = 0; j < a->npairs; ++j)
            if (!ref_ok(a->a[o][j]) || !ref_ok(a->b[o][j])) return -1;
    }
    if (a->n == 0 || a->K == 0) return 0;
    for (int o = 0; o < a->nout; ++o)
        for (int j0 = 0; j0 < a->npairs; j0 += PC_TSUM_MAX) {
            TensorSumArgs t{};
            t.out = a->out[o];
            t.d2 = a->d2[o];
            t.npairs = a->npairs - j0 < PC_TSUM_MAX ? a->npairs - j0 : PC_TSUM_MAX;
            for (int j = 0; j < t.npairs; ++j) {
                t.a[j] = a->a[o][j0 + j];
                t.b[j] = a->b[o][j0 + j];
            }
            t.pr = a->pr;
            t.acc = j0 == 0 ? a->acc : 2;
            t.n = a->n;
            t.K = a->K;
            hipLaunchKernelGGL(tensor_sum_k, grid<LOGN>(a->n, a->K), dim3(BX), 0, (hipStream_t)s, t, LOGN);
            if (int rc = launch_rc()) return rc;
        }
    return 0;
}

// ------------------------------------------------------------------------------------------------ coeff_sum
// coeff_sum (args.cuh:906-927; host twin crates/pc-host/src/coeffrows.rs:11-80). Pass 1: scratch row (r, l) = the
// residues mod p_l of round(rows[r] scale) (half to even; a product of magnitude 9.2e18 or more becomes +-2^62 and is
// counted once per limb and coefficient). Pass 2: the forward NTT of the n L scratch rows (dense: row r L + l, prime
// l). Pass 3: out (+)= sum_r scratch(r, l) ct_r, both parts, one exact reduction per word.
__global__ void __launch_bounds__(BX) coeff_conv_k(CoeffArgs A, int logn) {
    const int l = blockIdx.y, r = blockIdx.z;
    const uint32_t k = blockIdx.x * BX + threadIdx.x;
    const uint32_t p = (uint32_t)A.pr[l].p;
    const double x = (double)A.rows[r][k] * A.scale;
    int64_t m;
    const bool ovf = !(fabs(x) < 9.2e18);
    if (!ovf) m = (int64_t)rint(x);
    else m = x < 0.0 ? -(int64_t(1) << 62) : (int64_t(1) << 62);
    const uint64_t mag = m < 0 ? (uint64_t)0 - (uint64_t)m : (uint64_t)m;
    uint32_t v = (uint32_t)(mag % p);
    if (m < 0 && v) v = p - v;
    ((uint32_t*)A.scratch)[((size_t)(r * A.L + l) << logn) + k] = v;
    if (ovf && A.overflow) atomicAdd(A.overflow, 1ull);
}

__global__ void __launch_bounds__(BX) coeff_acc_k(CoeffArgs A, int logn) {
    const int l = blockIdx.y, part = blockIdx.z;
    const uint32_t i = lane_word();
    const Red red(A.pr[l]);
    const size_t row = ((size_t)l << logn) + i;
    uint32_t* o = (uint32_t*)A.out + part * A.part_stride + row;
    Acc s[4];
    if (A.accumulate) {
        const W4 y = ld4(o);
#pragma unroll
        for (int w = 0; w < 4; ++w) s[w].add(y.v[w]);
    }
    for (int r = 0; r < A.n; ++r) {
        const W4 x = ld4((const uint32_t*)A.scratch + ((size_t)(r * A.L + l) << logn) + i);
        const W4 c = ld4((const uint32_t*)A.ct[r] + part * A.part_stride + row);
#pragma unroll
        for (int w = 0; w < 4; ++w) s[w].add((uint64_t)x.v[w] * c.v[w]);
    }
    W4 z;
#pragma unroll
    for (int w = 0; w < 4; ++w) z.v[w] = s[w].red(red);
    st4(o, z);
}

template <int LOGN>
int coeff_sum(const CoeffArgs* a, pc_stream_t s) {
    if (!a || a->n < 1 || a->n > PC_COEFF_MAXT || a->L < 1 || a->L > PC_COEFF_MAXL) return -1;
    if (!a->scratch || !a->out || !a->fw || !a->fws || !a->pr) return -2;
    for (int r = 0; r < a->n; ++r)
        if (!a->rows[r] || !a->ct[r]) return -2;
    hipLaunchKernelGGL(coeff_conv_k, dim3((1 << LOGN) / BX, a->L, a->n), dim3(BX), 0, (hipStream_t)s, *a, LOGN);
    if (int rc = launch_rc()) return rc;
    NttArgs t{};
    t.base = a->scratch;
    t.fw = a->fw;
    t.fws = a->fws;
    t.pr = a->pr;
    t.nrows = a->n * a->L;
    t.xnum = a->L;
    if (int rc = ntt_fwd_dense(LOGN, &t, s)) return rc;
    PCH_LAUNCH(coeff_acc_k, grid<LOGN>(a->L, 2), *a, LOGN);
}

template <int LOGN>
int pt_dot(const PtDotArgs* a, pc_stream_t s) {
    if (!a || a->K > 8) return -1;
    if (!a->rot.base || !a->res.base || !a->pts || !a->pr || a->K < 0 || a->bstep < 0 || a->gstep < 0) return -1;
    const int rows = a->rs.nq + a->rs.np;
    if (rows <= 0 || a->K == 0 || a->gstep == 0) return 0;
    // every diagonal index inside the row of ptw words
    const uint32_t n = 1u << LOGN;
    if (a->ptw < 1 || (a->enc == 0xFFFFFFFFu ? (uint32_t)a->ptw < n
                       : (a->enc >> 24) == 0x7Fu ? (a->enc & 0xFFu) > 31 || (uint32_t)a->ptw < (n >> (a->enc & 0xFFu))
                                                 : (uint64_t)a->ptw <= ((n - 1) & a->enc)))
        return -1;
    // the register form (baby steps in groups of 4 or 8); its diagonal loads by index form (full rows of whole 16-byte
    // groups, compact by a shift of at least 2, anything else)
    if (a->bstep >= 1 && a->npts >= 1) {
        const int mode = a->enc == 0xFFFFFFFFu && (a->ptw & 3) == 0                ? 0
                         : (a->enc >> 24) == 0x7Fu && (a->enc & 0xFFu) >= 2 ? 1
                                                                              : 2;
        const dim3 g = grid<LOGN>(rows, 1);
        if (a->bstep <= 4) {
            if (mode == 0) PCH_LAUNCH((pt_dot_reg_k<4, 0>), g, *a, LOGN);
            if (mode == 1) PCH_LAUNCH((pt_dot_reg_k<4, 1>), g, *a, LOGN);
            PCH_LAUNCH((pt_dot_reg_k<4, 2>), g, *a, LOGN);
        }
        if (mode == 0) PCH_LAUNCH((pt_dot_reg_k<8, 0>), g, *a, LOGN);
        if (mode == 1) PCH_LAUNCH((pt_dot_reg_k<8, 1>), g, *a, LOGN);
        PCH_LAUNCH((pt_dot_reg_k<8, 2>), g, *a, LOGN);
    }
    PCH_LAUNCH(pt_dot_k, grid<LOGN>(rows, 1), *a, LOGN);
}
#undef PCH_LAUNCH

}  // namespace em

#define PCH_EM_INST(L)                                                                                               \
    int tensor_##L(const TensorArgs* a, pc_stream_t s) { return em::tensor<L>(a, s); }                               \
    int tensor_y_##L(const TensorYArgs* a, pc_stream_t s) { return em::tensor_y<L>(a, s); }                          \
    int tensor_sum_##L(const TensorSumArgs* a, pc_stream_t s) { return em::tensor_sum<L>(a, s); }                    \
    int md_epilogue_##L(const MdEpiArgs* a, pc_stream_t s) { return em::md_epilogue<L>(a, s); }                      \
    int md_epilogue_to_##L(const MdEpiToArgs* a, pc_stream_t s) { return em::md_epilogue_to<L>(a, s); }              \
    int wsum_##L(const WsumArgs* a, pc_stream_t s) { return em::wsum<L>(a, s); }                                     \
    int wsum_k_##L(const WsumKArgs* a, pc_stream_t s) { return em::wsum_kc<L>(a, s); }                               \
    int wsum_multi_##L(const WsumMultiArgs* a, pc_stream_t s) { return em::wsum_multi<L>(a, s); }                    \
    int add_const_##L(const AddConstArgs* a, pc_stream_t s) { return em::add_const<L>(a, s); }                       \
    int mul_table_##L(const MulTableArgs* a, pc_stream_t s) { return em::mul_table<L>(a, s); }                       \
    int mul_add_##L(const MulAddArgs* a, pc_stream_t s) { return em::mul_add<L>(a, s); }                             \
    int mul_add_n_##L(const MulAddNArgs* a, pc_stream_t s) { return em::mul_add_n<L>(a, s); }                        \
    int rescale_combine_##L(const RescaleCombineArgs* a, pc_stream_t s) { return em::rescale_combine<L>(a, s); }     \
    int rescale_combine_to_##L(const RescaleCombineToArgs* a, pc_stream_t s) {                                       \
        return em::rescale_combine_to<L>(a, s);                                                                      \
    }                                                                                                                \
    int ew_many_##L(const EwManyArgs* a, pc_stream_t s) { return em::ew_many<L>(a, s); }                             \
    int submul_many_##L(const SubMulManyArgs* a, pc_stream_t s) { return em::submul_many<L>(a, s); }             \
    int pt_dot_##L(const PtDotArgs* a, pc_stream_t s) { return em::pt_dot<L>(a, s); }                            \
    int coeff_sum_##L(const CoeffArgs* a, pc_stream_t s) { return em::coeff_sum<L>(a, s); }                      \
    int tensor_multi_##L(const TensorMultiArgs* a, pc_stream_t s) { return em::tensor_multi<L>(a, s); }
PCH_EM_INST(12)
PCH_EM_INST(13)
PCH_EM_INST(14)
PCH_EM_INST(15)
PCH_EM_INST(16)

int mul_pt_list(int logn, const MulPtListArgs* a, pc_stream_t s) {
    switch (logn) {
        case 12: return em::mul_pt_list<12>(a, s);
        case 13: return em::mul_pt_list<13>(a, s);
        case 14: return em::mul_pt_list<14>(a, s);
        case 15: return em::mul_pt_list<15>(a, s);
        case 16: return em::mul_pt_list<16>(a, s);
        default: return -2;
    }
}

int tensor_list(int logn, const TensorListArgs* a, pc_stream_t s) {
    switch (logn) {
        case 12: return em::tensor_list<12>(a, s);
        case 13: return em::tensor_list<13>(a, s);
        case 14: return em::tensor_list<14>(a, s);
        case 15: return em::tensor_list<15>(a, s);
        case 16: return em::tensor_list<16>(a, s);
        default: return -2;
    }
}

}  // namespace pch
