// ModDown's conversion fused into the forward NTT (crates/pc-gpu/src/ks.rs:1620-1649 moddown_to_j: INTT of the P rows,
// bconv P -> Q, NTT with the epilogue (x - conv) P^-1; host twin crates/pc-host/src/bconv.rs, ntt.rs).
//
// A conversion output row is only ever read by the forward NTT's column pass, and that pass works on whole columns:
// the words j = r C + c of one column c are a contiguous set of coefficient positions of every row. So one workgroup
// takes a block of CC columns of one (ciphertext, part): it keeps the kp source words y_j of each of its positions
// in registers (kp <= 6, loaded once), and for each of its target rows t forms conv_t = sum_j y_j M[j][t] mod q_t and
// runs the column pass of prime t on it before writing. The conversion rows never reach HBM: per key switch this saves
// writing and re-reading 2 (top + 1) rows. Targets are split into groups of ntg rows per workgroup so that a launch has
// several workgroups per CU; the groups of one column block are neighbours in the XCD-aware order, so the second and
// later reads of the block's sources hit that XCD's L2.
#include "fused.h"
#include "ntt_core.h"

namespace pch {
namespace ntt {

template <int LOGN, bool H, int KP>
__global__ void __launch_bounds__(WG) md_conv_cols_k(MdcArgs A) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[2][G::COL_LDS];
    const Blk B = blk_xy();
    const int ng = gridDim.x / G::COL_WGS;
    const int grp = B.x % ng, cbk = B.x / ng;
    const size_t rb = (size_t)B.y * A.rows;  // row 0 of (ciphertext, part) B.y
    const int col = threadIdx.x % G::CC, tau = threadIdx.x / G::CC;
    const int c = cbk * G::CC + col;
    // this (ciphertext, part)'s rows through buffer resources: per-lane offsets, the row and the stride uniform
    const uint32_t span = (uint32_t)A.rows << (LOGN + 2);
    const Buf bx(A.ext + (rb << LOGN), span), bc(A.conv + (rb << LOGN), span);
    // the sources at positions (tau + TR e) C + c: the column pass's layout A
    uint32_t y[KP][E];
    const uint32_t vy = (uint32_t)(tau * G::C + c) * 4;
#pragma unroll
    for (int j = 0; j < KP; ++j) {
#pragma unroll
        for (int e = 0; e < E; ++e) y[j][e] = bx.ld(vy, (uint32_t)(((A.nq + j) << LOGN) + G::TR * e * G::C) * 4);
    }
    const uint32_t vo = (uint32_t)(E * tau * G::C + c) * 4;
    const int t0 = grp * A.ntg, t1 = min(A.top + 1, t0 + A.ntg);
    // the column pass reads twiddle entries below R only: the group's targets' tables (values, then Shoup companions)
    // staged once in LDS, shared by the workgroup's columns
    __shared__ uint32_t tw[MDC_MAX_NTG][2 * G::R];
    for (int i = threadIdx.x; i < (t1 - t0) * 2 * G::R; i += WG) {
        const int k = i / (2 * G::R), j = i % (2 * G::R);
        const size_t off = ((size_t)(t0 + k) << LOGN) + (j % G::R);
        tw[k][j] = j < G::R ? A.fw[off] : A.fws[off];
    }
    __syncthreads();
    auto base = [](int h) { return (uint32_t)(G::R / (2 * h)); };
    for (int t = t0; t < t1; ++t) {
        const Red red(A.pr[t]);
        const uint32_t p = red.p, p2 = 2 * p;
        const uint32_t r64 = shoup(red.r32, red.r32, red.r32s, p);  // 2^64 mod q_t
        uint32_t m[KP];
#pragma unroll
        for (int j = 0; j < KP; ++j) m[j] = A.mt[j * A.nq + t];
        // sum_j y_j M[j][t]: products below 2^62, three to a 64-bit sum; two sums add to 65 bits, the carry folded in
        // as 2^64 mod q_t, so one reduction per word
        uint32_t x[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            uint64_t a0 = 0, a1 = 0;
#pragma unroll
            for (int j = 0; j < KP; ++j) {
                if (j < 3) a0 += (uint64_t)y[j][e] * m[j];
                else a1 += (uint64_t)y[j][e] * m[j];
            }
            if (KP > 3) {
                const uint64_t s = a0 + a1;
                x[e] = addm(red(s), s < a0 ? r64 : 0u, p);
            } else {
                x[e] = red(a0);
            }
            // one word's conversion at a time: interleaving all 16 would hold 16 double-word sums beside the 6 x 16
            // source words (2 waves per SIMD instead of 3)
            __builtin_amdgcn_sched_barrier(0);
        }
        const uint32_t* w = tw[t - t0];
        const uint32_t* ws = tw[t - t0] + G::R;
        phase_a<true, H, G::TR>(x, w, ws, p, p2, base);
        // double-buffered transpose: one barrier per target
        uint32_t* l = lds[t & 1];
#pragma unroll
        for (int e = 0; e < E; ++e) l[tau * G::WT + col + e * G::WS] = x[e];
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = l[tau * G::RT + col + e * G::RS];
        phase_b<true, H, G::TR>(x, tau, w, ws, p, p2, base);
#pragma unroll
        for (int e = 0; e < E; ++e) bc.st(x[e], vo, (uint32_t)((t << LOGN) + e * G::C) * 4);  // lazy words
    }
}

template <int LOGN, bool H>
void mdc_launch(const MdcArgs& a, hipStream_t st) {
    using G = Geo<LOGN>;
    const int ng = (a.top + 1 + a.ntg - 1) / a.ntg;
    const dim3 grid(G::COL_WGS * ng, 2 * a.m);
    switch (a.kp) {
        case 1: hipLaunchKernelGGL((md_conv_cols_k<LOGN, H, 1>), grid, dim3(WG), 0, st, a); break;
        case 2: hipLaunchKernelGGL((md_conv_cols_k<LOGN, H, 2>), grid, dim3(WG), 0, st, a); break;
        case 3: hipLaunchKernelGGL((md_conv_cols_k<LOGN, H, 3>), grid, dim3(WG), 0, st, a); break;
        case 4: hipLaunchKernelGGL((md_conv_cols_k<LOGN, H, 4>), grid, dim3(WG), 0, st, a); break;
        case 5: hipLaunchKernelGGL((md_conv_cols_k<LOGN, H, 5>), grid, dim3(WG), 0, st, a); break;
        default: hipLaunchKernelGGL((md_conv_cols_k<LOGN, H, 6>), grid, dim3(WG), 0, st, a); break;
    }
}

template <int LOGN>
int mdc(const MdcArgs* a, pc_stream_t s) {
    if (a->lazy) mdc_launch<LOGN, true>(*a, (hipStream_t)s);
    else mdc_launch<LOGN, false>(*a, (hipStream_t)s);
    return launch_rc();
}

// The fused ModDown-rescale's preparation (both parts, rows 0..top; ciphertext blockIdx.z of K, 2 rows rows apart):
// rows top - 1 and top of x take P onto (the conversion's Q sources then hold x + P onto); rows i <= top - 2 of out
// become onto s2_i (s2 = (q_top q_{top-1})^-1 mod q_i), onto which the NTT's epilogue adds (x - conv) B^-1. k: [s2 |
// s2' | P mod q | its Shoup companion] by prime id, rows words each. 4 words per thread.
__global__ void __launch_bounds__(256) mdr_prep_k(uint32_t* x, const uint32_t* onto, uint32_t* out,
                                                  const uint32_t* k, const PrimeConst* pr, int rows, int top, int logn) {
    const int part = blockIdx.y / (top + 1), i = blockIdx.y % (top + 1);
    const uint32_t p = (uint32_t)pr[i].p;
    const size_t off = ((size_t)((2 * blockIdx.z + part) * rows + i) << logn) + (blockIdx.x * 256 + threadIdx.x) * 4;
    const uint4 v = *(const uint4*)(onto + off);
    if (i >= top - 1) {
        const uint32_t w = k[2 * rows + i], ws = k[3 * rows + i];
        uint4 a = *(const uint4*)(x + off);
        a.x = addm(a.x, shoup(v.x, w, ws, p), p);
        a.y = addm(a.y, shoup(v.y, w, ws, p), p);
        a.z = addm(a.z, shoup(v.z, w, ws, p), p);
        a.w = addm(a.w, shoup(v.w, w, ws, p), p);
        *(uint4*)(x + off) = a;
    } else {
        const uint32_t w = k[i], ws = k[rows + i];
        *(uint4*)(out + off) = make_uint4(shoup(v.x, w, ws, p), shoup(v.y, w, ws, p), shoup(v.z, w, ws, p),
                                          shoup(v.w, w, ws, p));
    }
}

}  // namespace ntt

int mdr_prep(int logn, void* x, const void* onto, void* out, const uint32_t* k, const PrimeConst* pr, int rows,
             int top, int K, pc_stream_t s) {
    if (!x || !onto || !out || !k || !pr || top < 2 || top >= rows || logn < 12 || logn > 16 || K < 1) return -1;
    const dim3 grid((1u << logn) / 1024, 2 * (top + 1), K);
    hipLaunchKernelGGL(ntt::mdr_prep_k, grid, dim3(256), 0, (hipStream_t)s, (uint32_t*)x, (const uint32_t*)onto,
                       (uint32_t*)out, k, pr, rows, top, logn);
    return launch_rc();
}

int md_conv_cols(int logn, const MdcArgs* a, pc_stream_t s) {
    if (!a || !a->ext || !a->conv || !a->mt || !a->pr || !a->fw || !a->fws) return -1;
    if (a->m < 0 || a->top < 0 || a->top >= a->nq || a->ntg < 1 || a->rows < a->nq + a->kp) return -1;
    if (a->kp < 1 || a->kp > MDC_MAX_KP || a->ntg > MDC_MAX_NTG) return -2;
    if (a->m == 0) return 0;
    switch (logn) {
        case 12: return ntt::mdc<12>(a, s);
        case 13: return ntt::mdc<13>(a, s);
        case 14: return ntt::mdc<14>(a, s);
        case 15: return ntt::mdc<15>(a, s);
        case 16: return ntt::mdc<16>(a, s);
        default: return -2;
    }
}

}  // namespace pch
