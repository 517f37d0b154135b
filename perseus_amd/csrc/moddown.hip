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
        // the target's constants through the scalar cache: a vector load here would wait for the previous target's
        // stores
        const Red red = Red::scalar(A.pr, t);
        const uint32_t p = red.p, p2 = 2 * p;
        const uint32_t r64 = shoup(red.r32, red.r32, red.r32s, p);  // 2^64 mod q_t
        uint32_t m[KP];
#pragma unroll
        for (int j = 0; j < KP; ++j) m[j] = sload(A.mt + j * A.nq + t);
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

// a.ntg target rows per workgroup, fewer (down to 1) when the launch would have under 2048 workgroups: a small
// ModDown (a C1 rotation's 2 x 12 rows at N = 2^14: 24 workgroups at 5 rows each) then spreads its targets over
// more CUs, each workgroup re-reading its column block's sources from L2
template <int LOGN>
int mdc(const MdcArgs* a, pc_stream_t s) {
    using G = Geo<LOGN>;
    MdcArgs b = *a;
    while (b.ntg > 1 && (long)G::COL_WGS * ((b.top + b.ntg) / b.ntg) * 2 * b.m < 2048) --b.ntg;
    if (b.lazy) mdc_launch<LOGN, true>(b, (hipStream_t)s);
    else mdc_launch<LOGN, false>(b, (hipStream_t)s);
    return launch_rc();
}

// Any conversion plan's jobs (bconv.hip's job records, prescaled sources, fast or exact) fused into the forward NTT's
// column pass, for source counts beyond what md_conv_cols_k keeps in registers: a ModUp digit of 16 limbs, a ModDown
// over 16 special primes, the ModDown-rescale's 18 sources. A workgroup takes one job's block of CC columns and a group
// of tpw of its targets, NTG targets at a time, and streams the sources instead of holding them: for each source the
// thread loads the 16 words of its positions (the column pass's layout A) and multiplies them into NTG double-word
// sums, so its registers hold NTG x 16 sums whatever the number of sources. The first workgroup of a column block
// reads a source from HBM, the block's other target groups (its neighbours in the XCD-aware order) from that XCD's L2.
// Each target's sum is reduced (exact jobs: less u (B mod t), u = floor(sum y_i / b_i + 1/2) from the doubles in source
// order, as bconv_k forms it), taken through the column pass of its prime and stored as fwd_cols stores it, lazy
// words in the target's row of dst; ntt_fwd_rows_only completes the transform over the same rows.
template <int LOGN, bool H, int NTG, bool EX>
__global__ void __launch_bounds__(WG, EX ? (NTG == 1 ? 3 : 2) : (NTG == 3 ? 3 : 4)) conv_cols_k(BconvArgs A, const uint32_t* fw, const uint32_t* fws, int tpw) {
    using G = Geo<LOGN>;
    __shared__ uint32_t lds[2][G::COL_LDS];
    const Blk B = blk_xy();
    const int ng = gridDim.x / G::COL_WGS;
    const int grp = B.x % ng, cbk = B.x / ng;
    const BconvJob j = A.jobs[B.y];
    const int ns = (int)j.nsrc, nt = (int)j.ntgt;
    const int t0 = grp * tpw, t1 = min(nt, t0 + tpw);
    if (t0 >= t1 || ns < 1) return;  // uniform over the workgroup, before its first barrier
    // the job's pool: src_row[ns], src_prime[ns], pre[ns], tgt_row[nt], tgt_prime[nt], M[ns][nt] (workgroup-uniform
    // reads, through the scalar cache)
    const cptr pool = (cptr)((const uint32_t*)A.pool + j.pool_off);
    const cptr trows = pool + 3 * ns, tprimes = trows + nt, mt = tprimes + nt;
    uint32_t smax = 0, maxsp = 0;
    for (int i = 0; i < ns; ++i) {
        smax = max(smax, pool[i]);
        maxsp = max(maxsp, (uint32_t)sload(&A.pr[pool[ns + i]].p));
    }
    uint32_t dmax = 0;
    for (int t = t0; t < t1; ++t) dmax = max(dmax, trows[t]);
    // the rows the job reads and the group writes, as the buffer resources' extents
    const Buf bs((const uint32_t*)A.src + ((size_t)j.src_off << LOGN), (smax + 1) << (LOGN + 2));
    const Buf bd((uint32_t*)A.dst + ((size_t)j.dst_off << LOGN), (dmax + 1) << (LOGN + 2));
    const int col = threadIdx.x % G::CC, tau = threadIdx.x / G::CC;
    const int c = cbk * G::CC + col;
    const uint32_t vy = (uint32_t)(tau * G::C + c) * 4;      // word e: position (tau + TR e) C + c
    const uint32_t vo = (uint32_t)(E * tau * G::C + c) * 4;  // after the transpose: position (E tau + e) C + c
    auto ldsrc = [&](uint32_t row, uint32_t(&y)[E]) {
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] = bs.ld(vy, ((row << LOGN) + (uint32_t)(G::TR * e * G::C)) * 4);
    };
    // EX: the launch's jobs may be exact (u (B mod t) subtracted where j.exact); without EX every job is taken as fast
    uint32_t u[EX ? E : 1];
    const double* rb = nullptr;
    const uint32_t* bmod = nullptr;
    if (EX && j.exact) {
        // rb[ns] doubles at the first 8-byte aligned word after M, then bmod[nt] (Bconv::build)
        size_t w = (size_t)j.pool_off + 3 * ns + 2 * nt + (size_t)ns * nt;
        if (w & 1) ++w;
        rb = (const double*)((const uint32_t*)A.pool + w);
        bmod = (const uint32_t*)(rb + ns);
        if (j.exact == 2) {
            // the mean-centred job: ns / 2, odd ns rounded by a hash of the coefficient index
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const uint32_t coef = (uint32_t)((tau + G::TR * e) * G::C + c);
                u[e] = ((uint32_t)ns >> 1) + (((uint32_t)ns & 1) & ((coef * 0x9E3779B1u) >> 31));
            }
        }
    }
    auto base = [](int h) { return (uint32_t)(G::R / (2 * h)); };
    int lb = 0;  // the transpose's double buffer: one barrier per target
    for (int tt = t0; tt < t1; tt += NTG) {
        const int nk = min(NTG, t1 - tt);
        uint32_t pid[NTG], trow[NTG], maxtp = 0;
#pragma unroll
        for (int k = 0; k < NTG; ++k) {
            const int t = k < nk ? tt + k : tt;
            pid[k] = tprimes[t];
            trow[k] = trows[t];
            maxtp = max(maxtp, (uint32_t)sload(&A.pr[pid[k]].p));
        }
        // g products of (max source prime - 1)(max target prime - 1) stay below 2^64, a reduced residue counting as
        // one: a sum is folded to its residue before its (g + 1)-th product
        const uint64_t pm = (uint64_t)(maxsp - 1) * (uint64_t)(maxtp - 1);
        const int g = pm == 0 ? ns : (int)min((uint64_t)ns, ~0ull / pm);
        uint32_t rq[NTG][4];  // each target's Red constants
#pragma unroll
        for (int k = 0; k < NTG; ++k) {
            const Red r = Red::scalar(A.pr, pid[k]);
            rq[k][0] = r.p, rq[k][1] = r.r32, rq[k][2] = r.r32s, rq[k][3] = r.m;
        }
        auto rd = [&](int k) { return Red(rq[k][0], rq[k][1], rq[k][2], rq[k][3]); };
        uint64_t acc[NTG][E];
#pragma unroll
        for (int k = 0; k < NTG; ++k)
#pragma unroll
            for (int e = 0; e < E; ++e) acc[k][e] = 0;
        // exact jobs form u = floor(sum_i y_i rb_i + 1/2) in the first round, from the same loads: the doubles' FMAs
        // in source order, as bconv_k forms them
        const bool vu = EX && j.exact == 1 && tt == t0;
        double v[EX ? E : 1];
        if constexpr (EX) {
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = 0.0;
        }
        int cnt = 0;
        auto step = [&](const uint32_t(&y)[E], int i) {
            if (cnt == g) {
#pragma unroll
                for (int k = 0; k < NTG; ++k)
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[k][e] = rd(k)(acc[k][e]);
                cnt = 1;
            }
            ++cnt;
#pragma unroll
            for (int k = 0; k < NTG; ++k) {
                if (k < nk) {
                    const uint32_t m = mt[i * nt + tt + k];
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[k][e] += (uint64_t)y[e] * m;
                }
            }
            if constexpr (EX) {
                if (vu) {
                    const double r = rb[i];
#pragma unroll
                    for (int e = 0; e < E; ++e) v[e] = __fma_rn((double)y[e], r, v[e]);
                }
            }
        };
        // the next source's words in flight while this one's products are formed
        uint32_t ya[E], yb[E];
        ldsrc(pool[0], ya);
        for (int i = 0; i < ns; i += 2) {
            if (i + 1 < ns) ldsrc(pool[i + 1], yb);
            step(ya, i);
            if (i + 1 >= ns) break;
            if (i + 2 < ns) ldsrc(pool[i + 2], ya);
            step(yb, i + 1);
        }
        if constexpr (EX) {
            if (vu) {
#pragma unroll
                for (int e = 0; e < E; ++e) u[e] = (uint32_t)(uint64_t)floor(v[e] + 0.5);
            }
        }
#pragma unroll
        for (int k = 0; k < NTG; ++k) {
            if (k >= nk) continue;
            const uint32_t p = rq[k][0], p2 = 2 * p;
            uint32_t x[E];
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = rd(k)(acc[k][e]);
            if (EX && j.exact) {
                // u <= ns: u (B mod t) as one Shoup product
                const uint32_t b = bmod[tt + k], bs2 = (uint32_t)(((uint64_t)b << 32) / p);
#pragma unroll
                for (int e = 0; e < E; ++e) x[e] = subm(x[e], shoup(u[e], b, bs2, p), p);
            }
            const uint32_t* w = fw + ((size_t)pid[k] << LOGN);
            const uint32_t* ws = fws + ((size_t)pid[k] << LOGN);
            phase_a<true, H, G::TR, decltype(base), true>(x, w, ws, p, p2, base);
            uint32_t* l = lds[lb];
            lb ^= 1;
#pragma unroll
            for (int e = 0; e < E; ++e) l[tau * G::WT + col + e * G::WS] = x[e];
            __syncthreads();
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = l[tau * G::RT + col + e * G::RS];
            phase_b<true, H, G::TR>(x, tau, w, ws, p, p2, base);
#pragma unroll
            for (int e = 0; e < E; ++e) bd.st(x[e], vo, ((trow[k] << LOGN) + (uint32_t)(e * G::C)) * 4);
        }
    }
}

template <int LOGN, bool H, bool EX>
void cc_launch(int ntg, dim3 grid, hipStream_t st, const BconvArgs& a, const uint32_t* fw, const uint32_t* fws, int tpw) {
    if (ntg == 1) hipLaunchKernelGGL((conv_cols_k<LOGN, H, 1, EX>), grid, dim3(WG), 0, st, a, fw, fws, tpw);
    else if (ntg == 2) hipLaunchKernelGGL((conv_cols_k<LOGN, H, 2, EX>), grid, dim3(WG), 0, st, a, fw, fws, tpw);
    else hipLaunchKernelGGL((conv_cols_k<LOGN, H, 3, EX>), grid, dim3(WG), 0, st, a, fw, fws, tpw);
}
template <int LOGN>
int cc(const BconvArgs* a, const uint32_t* fw, const uint32_t* fws, int lazy, int exact, int ntg, int tpw,
       pc_stream_t s) {
    using G = Geo<LOGN>;
    const int ng = (a->max_tgt + tpw - 1) / tpw;
    const dim3 grid(G::COL_WGS * ng, a->njobs);
    const hipStream_t st = (hipStream_t)s;
    if (lazy && exact) cc_launch<LOGN, true, true>(ntg, grid, st, *a, fw, fws, tpw);
    else if (lazy) cc_launch<LOGN, true, false>(ntg, grid, st, *a, fw, fws, tpw);
    else if (exact) cc_launch<LOGN, false, true>(ntg, grid, st, *a, fw, fws, tpw);
    else cc_launch<LOGN, false, false>(ntg, grid, st, *a, fw, fws, tpw);
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

int conv_cols(int logn, const BconvArgs* a, const uint32_t* fw, const uint32_t* fws, int lazy, int exact, int ntg,
              int tpw, pc_stream_t s) {
    if (!a || !a->src || !a->dst || !a->jobs || !a->pool || !a->pr || !fw || !fws || a->njobs < 0) return -1;
    if (a->njobs > 65535 || a->max_tgt < 1 || tpw < 1 || ntg < 1 || ntg > 3) return -1;
    if (a->njobs == 0) return 0;
    tpw = (tpw + ntg - 1) / ntg * ntg;
    switch (logn) {
        case 12: return ntt::cc<12>(a, fw, fws, lazy, exact, ntg, tpw, s);
        case 13: return ntt::cc<13>(a, fw, fws, lazy, exact, ntg, tpw, s);
        case 14: return ntt::cc<14>(a, fw, fws, lazy, exact, ntg, tpw, s);
        case 15: return ntt::cc<15>(a, fw, fws, lazy, exact, ntg, tpw, s);
        case 16: return ntt::cc<16>(a, fw, fws, lazy, exact, ntg, tpw, s);
        default: return -2;
    }
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
