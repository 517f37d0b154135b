// The fused CtS / StC stage core on gfx950: hoisted baby-step rotations of a ModUp'd ciphertext times the BSGS
// plaintext diagonals, summed per giant step in Q u P, the rotations never stored (crates/pc-kernels/kernels/cts.cuh
// cts_fused / cts_fused_regen; args.cuh CtsArgs :325-355, CtsRegenArgs :752-757; host twin crates/pc-host/src/cts.rs).
//
// One wave per workgroup owns an aligned 1024-slot chunk of output slots of one row t and one ciphertext. It keeps the
// sums of two giant steps for its 16 slots per lane in registers across all baby steps. The automorphism maps aligned
// 1024-slot chunks onto aligned chunks, so the sources of baby i are one aligned chunk too. The wave forms
// P c0 + sum_d D_d b_d and sum_d D_d a_d there in SOURCE order: a lane's 16 consecutive slots are exactly one ChaCha12
// block of the KSKA stream, so `a` is regenerated without cross-lane traffic, and D, b and c0 arrive in 64-byte
// loads. The two words per slot then move to output order through LDS with the conflict-free scatter of the key-switch
// dot, and are multiplied into the giant steps' sums with the diagonals' words at the output slots. Rejected KSKA words
// are queued in LDS and redrawn by the whole wave at once.
#include "common.h"

namespace pch {
namespace cts {

constexpr int CW = 64;          // lanes per workgroup: one wave
constexpr int CS = 16;          // slots per lane: one ChaCha12 block
constexpr int CCH = CW * CS;    // the wave's chunk of slots
constexpr int DMAX = 6;         // digits a stage reads at u32 words (cts.cuh:18-22)
constexpr int GW = 2;           // giant steps per pass: 2 parts x GW x 16 sums per lane
constexpr int QCAP = 1536;      // queued rejected words (>= 1024 free before every digit)

struct Lds {
    uint64_t ex[CCH];   // per slot: the redrawn words' products D_d a_d mod p; then the two scatter buffers
    uint32_t q[QCAP];   // rejected words: digit << 16 | offset in the source chunk
    uint32_t qn;
};

// k^-1 mod 2^32 for odd k: Newton's step x (2 - k x) doubles the correct low bits, and k k = 1 mod 8 starts at three.
__device__ __forceinline__ uint32_t inv_odd(uint32_t k) {
    uint32_t x = k;
#pragma unroll
    for (int i = 0; i < 4; ++i) x *= 2u - k * x;
    return x;
}

// crates/pc-kernels/kernels/arith.cuh:242-244: a diagonal's compact index of slot o
__device__ __forceinline__ uint32_t ptidx(uint32_t o, uint32_t enc) {
    return (enc >> 24) == 0x7Fu ? o >> (enc & 0xFFu) : o & enc;
}

// the key slot of prime id t (KskShape::slot_of): Q primes at their id, special prime nq + j at q_top + 1 + j
__device__ __forceinline__ int slot_of(const KeyTab& T, int t, int nq) {
    return (t < nq || T.q_top < 0) ? t : T.q_top + 1 + (t - nq);
}

// The 16 values of a bit-packed row of `words` words from value s0 on (bits per value; the row ends in a guard word):
// value k spans words w, w + 1 with w = (s0 + k) bits / 32, read as one 8-byte buffer load at a 32-bit offset.
__device__ __forceinline__ void ld_packed(const uint32_t* row, uint64_t words, uint32_t s0, int bits,
                                          uint32_t (&b)[CS]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)row, 0, (int)(words * 4), 0x00020000);
    const uint32_t bit0 = s0 * (uint32_t)bits;
    const uint32_t msk = bits == 32 ? 0xFFFFFFFFu : (1u << bits) - 1u;
#pragma unroll
    for (int k = 0; k < CS; ++k) {
        const uint32_t bit = bit0 + k * (uint32_t)bits;
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (bit >> 5) * 4, 0, 0);
        b[k] = __builtin_amdgcn_alignbit(v[1], v[0], bit & 31) & msk;
    }
}

struct Src {
    const uint32_t* c1;   // the ciphertext's c1 row t (own digit)
    const uint32_t* mu;   // ModUp digit 0's row t
    uint64_t mds;         // digit stride of the ModUp output
    int dt;               // the digit of row t (-1 on special rows)
    __device__ __forceinline__ const uint32_t* row(int d) const { return d == dt ? c1 : mu + d * mds; }
};

// Redraw the queued words: each lane takes items and adds D_d a_d mod p (the accepted attempt t = 1..15 at block
// + t N/16, the 16th attempt kept as is) to the slot's sum; reduced products keep the sum below ndig 2^31.
__device__ __forceinline__ void drain(Lds& L, int lane, const uint32_t (&seed)[8], const Expander& ex, const Red& red,
                                      uint32_t n16, uint32_t sc, const Src& S) {
    wave_sync();
    const uint32_t nq = L.qn;
    for (uint32_t i = lane; i < nq; i += CW) {
        const uint32_t it = L.q[i], d = it >> 16, sl = it & 0xFFFF;
        const uint32_t ctr = (sc + sl) >> 4;
        uint32_t v = 0;
        for (int tt = 1; tt < KSK_T_MAX; ++tt) {
            v = chacha12_word(seed, ctr + (uint32_t)tt * n16, d, ex.p, TAG_KSKA, (int)(sl & 15));
            if (v < ex.mp) break;
        }
        const uint32_t xd = S.row((int)d)[sc + sl];
        atomicAdd((unsigned long long*)&L.ex[sl], (unsigned long long)red((uint64_t)xd * ex.red(v)));
    }
    wave_sync();
    if (lane == 0) L.qn = 0;
    wave_sync();
}

// grid (N / 1024 chunks, rows, K ciphertexts); giant steps j0, j0 + 1 of the launch. REGEN: keys through the KeyTab
// (a regenerated for digits < nregen); WIDE: more than 4 digits (the 64-bit sums reduced every 3 digits).
template <bool REGEN, bool WIDE>
__global__ void __launch_bounds__(CW, 2) cts_k(CtsRegenArgs RA, int logn, int j0) {
    __shared__ Lds L;
    const CtsArgs& A = RA.cts;
    const KeyTab& T = RA.key;
    const int lane = threadIdx.x, c = blockIdx.z;
    const int t = (int)A.rows[blockIdx.y];
    const PrimeConst& q = A.pr[t];
    const uint32_t p = (uint32_t)q.p;
    const Red red(q);
    const Expander ex(p);
    const uint32_t n16 = (1u << logn) >> 4, mask2n = (2u << logn) - 1;
    const bool isq = t < A.nq;
    const int prow = isq ? t : A.pt_prow + (t - A.nq);
    const uint32_t pm = isq ? ((const uint32_t*)A.pmod)[t] : 0, pms = isq ? ((const uint32_t*)A.pmods)[t] : 0;
    const size_t roff = (size_t)t << logn;
    const uint32_t* X = (const uint32_t*)A.x + c * A.ct_stride + roff;  // c0 row t; c1 at + part_stride
    const Src S{X + A.part_stride, (const uint32_t*)A.modup + c * A.mu_ct_stride + roff, A.mu_digit_stride,
                isq ? A.digit_of[t] : -1};
    const uint32_t oc0 = blockIdx.x * CCH;
    const uint32_t o0 = oc0 + lane * CS;  // the lane's output slots o0 .. o0 + 15
    const int gn = min(GW, A.G - j0);
    const int ndig = A.ndig;
    const int slot = REGEN ? slot_of(T, t, A.nq) : t;
    const int nreg = REGEN ? min(ndig, T.nregen) : 0;
    const bool pt16 = A.enc == 0xFFFFFFFFu && (A.ptw & 3) == 0;
    uint32_t acc0[GW][CS], acc1[GW][CS];
#pragma unroll
    for (int j = 0; j < GW; ++j)
#pragma unroll
        for (int k = 0; k < CS; ++k) acc0[j][k] = acc1[j][k] = 0;

    for (int i = 0; i < A.B; ++i) {
        uint32_t w0[CS], w1[CS];
        if (i == 0) {
            if (A.x0) {
                const uint32_t* x0 = (const uint32_t*)A.x0 + c * A.ct_stride + roff + o0;
                ld16(x0, w0);
                ld16(x0 + A.part_stride, w1);
            } else if (isq) {
                ld16(X + o0, w0);
                ld16(X + A.part_stride + o0, w1);
#pragma unroll
                for (int k = 0; k < CS; ++k) {
                    w0[k] = shoup(w0[k], pm, pms, p);
                    w1[k] = shoup(w1[k], pm, pms, p);
                }
            } else {
#pragma unroll
                for (int k = 0; k < CS; ++k) w0[k] = w1[k] = 0;
            }
        } else {
            // baby i: sources s = automorph_slot(g, o) of the chunk's outputs, one aligned chunk from sc on; the
            // products scatter back to the outputs by g^-1
            const uint32_t g = A.kinv[i - 1];
            const uint32_t kx = inv_odd(g) & mask2n;
            const uint32_t sc = automorph_slot(g, oc0, logn) & ~(uint32_t)(CCH - 1);
            const uint32_t s0 = sc + lane * CS;
            uint32_t seed[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (REGEN && nreg > 0) {
                const uint32_t* sp = T.seed[i - 1];
#pragma unroll
                for (int k = 0; k < 8; ++k) seed[k] = sp[k];
            }
            if (REGEN) {
#pragma unroll
                for (int k = 0; k < CS; ++k) L.ex[lane * CS + k] = 0;
                if (lane == 0) L.qn = 0;
                wave_sync();
            }
            uint32_t* l0 = (uint32_t*)L.ex;  // the scatter buffers of the two parts (over ex, once it is read)
            uint32_t* l1 = l0 + CCH;
            const int sh = logn - 9;
            const uint32_t bs0 = brev_n(s0, logn);
            const uint32_t cbh = (((2 * bs0 + 1) * kx) & mask2n) >> sh;
            const uint32_t sth = ((kx << (logn - 3)) & mask2n) >> sh;
            // part 1 first, sum_d D_d a_d (the regeneration and the redraws), then part 0, P c0 + sum_d D_d b_d: one
            // array of 64-bit sums at a time (D is read twice, the second time from L2)
            uint64_t z[CS];
            uint32_t part[WIDE ? CS : 1];
            uint32_t v[CS];
#pragma unroll
            for (int k = 0; k < CS; ++k) z[k] = 0;
#pragma unroll
            for (int k = 0; k < (WIDE ? CS : 1); ++k) part[k] = 0;
            for (int d = 0; d < ndig; ++d) {
                uint32_t a[CS], x[CS];
                if (REGEN && d < nreg) {
                    chacha12(seed, s0 >> 4, (uint32_t)d, p, TAG_KSKA, a);
                    uint32_t rej = 0;
#pragma unroll
                    for (int j = 0; j < CS; ++j) rej |= (uint32_t)(a[j] >= ex.mp) << j;
                    if (rej) {
                        // queued: the slot's sum gets D_d a_d when the wave drains the queue; counts as 0 here
                        uint32_t m = rej, qi = atomicAdd(&L.qn, (uint32_t)__builtin_popcount(rej));
                        while (m) {
                            const int j = __builtin_ctz(m);
                            m &= m - 1;
                            L.q[qi++] = (uint32_t)d << 16 | (uint32_t)(lane * CS + j);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < CS; ++j) a[j] = (rej >> j) & 1 ? 0 : ex.red(a[j]);
                } else {
                    ld16((const uint32_t*)A.ka[i - 1] + d * A.key_digit_stride + roff + s0, a);
                }
                ld16(S.row(d) + s0, x);
#pragma unroll
                for (int k = 0; k < CS; ++k) z[k] += (uint64_t)x[k] * a[k];
                if (WIDE && d % 3 == 2 && d + 1 < ndig) {
#pragma unroll
                    for (int k = 0; k < CS; ++k) {
                        part[k] = addm(part[k], red(z[k]), p);
                        z[k] = 0;
                    }
                }
                if (REGEN) {
                    // room for a whole digit's words before the next one (qn is shared: the test is wave-uniform)
                    wave_sync();
                    if (L.qn > (uint32_t)(QCAP - CCH)) drain(L, lane, seed, ex, red, n16, sc, S);
                }
            }
            if (REGEN) drain(L, lane, seed, ex, red, n16, sc, S);
#pragma unroll
            for (int k = 0; k < CS; ++k) {
                const uint64_t e = REGEN ? L.ex[lane * CS + k] : 0;
                // WIDE: <= 3 products per sum; else <= 4 products of (p - 1)^2 plus <= 4 words below p: < 2^64
                v[k] = WIDE ? addm(addm(part[k], red(z[k]), p), red(e), p) : red(z[k] + e);
            }
            // to output order: source s0 + k goes to output automorph_slot(g^-1, s0 + k) of chunk oc0
            wave_sync();
#pragma unroll
            for (int k = 0; k < CS; ++k) l1[scat_addr((cbh + brev4(k) * sth) & (CCH - 1))] = v[k];
#pragma unroll
            for (int k = 0; k < CS; ++k) z[k] = 0;
#pragma unroll
            for (int k = 0; k < (WIDE ? CS : 1); ++k) part[k] = 0;
            for (int d = 0; d < ndig; ++d) {
                uint32_t b[CS], x[CS];
                if (REGEN) {
                    const uint32_t* kr = (const uint32_t*)T.kb[i - 1] + (size_t)(d * T.srows + slot) * T.row_words;
                    if (T.bits == 0) ld16(kr + s0, b);
                    else ld_packed(kr, T.row_words, s0, T.bits, b);
                } else {
                    ld16((const uint32_t*)A.kb[i - 1] + d * A.key_digit_stride + roff + s0, b);
                }
                ld16(S.row(d) + s0, x);
#pragma unroll
                for (int k = 0; k < CS; ++k) z[k] += (uint64_t)x[k] * b[k];
                if (WIDE && d % 3 == 2 && d + 1 < ndig) {
#pragma unroll
                    for (int k = 0; k < CS; ++k) {
                        part[k] = addm(part[k], red(z[k]), p);
                        z[k] = 0;
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < CS; ++k) v[k] = WIDE ? addm(part[k], red(z[k]), p) : red(z[k]);
            if (isq) {
                uint32_t cz[CS];
                ld16(X + s0, cz);
#pragma unroll
                for (int k = 0; k < CS; ++k) v[k] = addm(v[k], shoup(cz[k], pm, pms, p), p);
            }
#pragma unroll
            for (int k = 0; k < CS; ++k) l0[scat_addr((cbh + brev4(k) * sth) & (CCH - 1))] = v[k];
            wave_sync();
            const uint32_t rb = scat_addr(__brev((uint32_t)lane) >> 26);
#pragma unroll
            for (int j = 0; j < CS; ++j) {
                w0[j] = l0[rb + 32 * brev4(j)];
                w1[j] = l1[rb + 32 * brev4(j)];
            }
            wave_sync();
        }
        // the giant steps' sums: acc_j += rot_i pt_{B j + i} at the lane's outputs
#pragma unroll
        for (int jj = 0; jj < GW; ++jj) {
            if (jj >= gn) break;
            const int dg = A.B * (j0 + jj) + i;
            if (dg >= A.npts) continue;
            const uint32_t* pt = (const uint32_t*)A.pts[dg] + (size_t)prow * A.ptw;
            uint32_t w[CS];
            if (pt16 && ((uintptr_t)pt & 15) == 0) {
                ld16(pt + o0, w);
            } else {
                const Buf bp(pt, (uint32_t)A.ptw * 4);
#pragma unroll
                for (int k = 0; k < CS; ++k) w[k] = bp.ld(ptidx(o0 + k, A.enc) * 4, 0);
            }
#pragma unroll
            for (int k = 0; k < CS; ++k) {
                acc0[jj][k] = red((uint64_t)w0[k] * w[k] + acc0[jj][k]);
                acc1[jj][k] = red((uint64_t)w1[k] * w[k] + acc1[jj][k]);
            }
        }
    }
#pragma unroll
    for (int jj = 0; jj < GW; ++jj) {
        if (jj >= gn) break;
        const int j = j0 + jj;
        const size_t at = A.pair_cts > 0 ? (size_t)(j >> 1) * A.pair_cts + (j & 1) : (size_t)c * A.G + j;
        uint32_t* r = (uint32_t*)A.res + at * A.ct_stride + roff + o0;
        st16(r, acc0[jj]);
        st16(r + A.part_stride, acc1[jj]);
    }
}

// The checks of the reference's launchers (cts.cuh:480-524: giant steps above 2, or above 4 in the K = 1 regen form
// with pair_cts; more than 6 digits; pair_cts outside that form; more than 64 baby steps in the regen form; x0 in the
// four-giant-step form or with ciphertext groups off the regen form: -1), then this kernel's own range: row strides
// of whole 16-byte groups (-2), and diagonals' compact indices inside ptw words (-1).
template <int LOGN, bool REGEN>
int launch(const CtsRegenArgs& R, pc_stream_t s) {
    static_assert((1 << LOGN) >= CCH, "ring of at least 1024 slots");
    const CtsArgs& a = R.cts;
    const int km = a.kmax <= 1 ? 1 : a.kmax <= 2 ? 2 : a.kmax <= 4 ? 4 : 8;
    const bool g4 = REGEN && km == 1 && a.K == 1 && a.pair_cts > 0;
    if (a.G > (g4 ? 4 : 2) || a.ndig > DMAX) return -1;
    if (a.pair_cts > 0 && !g4) return -1;
    if (REGEN && a.B > 64) return -1;
    if (a.x0 && (REGEN ? g4 : km != 1)) return -1;
    if (a.K < 0 || a.nrows < 0 || a.G < 0 || a.ndig < 0 || a.npts < 0) return -1;
    if (a.K == 0 || a.nrows == 0 || a.G <= 0) return 0;
    if (!a.rows || !a.pr || !a.x || !a.res || !a.digit_of || !a.pmod || !a.pmods) return -1;
    if (a.B > 0 && a.npts > 0 && !a.pts) return -1;
    if (a.B > 1) {
        if (!a.kinv || (a.ndig > 0 && !a.modup)) return -1;
        if (REGEN) {
            if (a.ndig > 0 && !R.key.kb) return -1;
            if (R.key.nregen > 0 && !R.key.seed) return -1;
            if (a.ndig > R.key.nregen && !a.ka) return -1;
        } else if (a.ndig > 0 && (!a.kb || !a.ka)) {
            return -1;
        }
    }
    const uint32_t n = 1u << LOGN;
    if (a.enc == 0xFFFFFFFFu ? (uint32_t)a.ptw < n
        : (a.enc >> 24) == 0x7Fu ? (a.enc & 0xFFu) > 31 || (uint32_t)a.ptw < (n >> (a.enc & 0xFFu))
                                 : (uint64_t)a.ptw <= ((n - 1) & a.enc))
        return -1;
    if ((a.ct_stride | a.part_stride | a.mu_ct_stride | a.mu_digit_stride | a.key_digit_stride) & 3) return -2;
    if (REGEN && R.key.bits == 0 && (R.key.row_words & 3)) return -2;
    const dim3 grid(n / CCH, a.nrows, a.K);
    hipStream_t st = (hipStream_t)s;
    for (int j0 = 0; j0 < a.G; j0 += GW) {
        if (a.ndig > 4) hipLaunchKernelGGL((cts_k<REGEN, true>), grid, dim3(CW), 0, st, R, LOGN, j0);
        else hipLaunchKernelGGL((cts_k<REGEN, false>), grid, dim3(CW), 0, st, R, LOGN, j0);
    }
    return launch_rc();
}

template <int LOGN>
int cts_fused(const CtsArgs* a, pc_stream_t s) {
    if (!a) return -1;
    CtsRegenArgs r{};
    r.cts = *a;
    return launch<LOGN, false>(r, s);
}

template <int LOGN>
int cts_fused_regen(const CtsRegenArgs* a, pc_stream_t s) {
    if (!a) return -1;
    if (a->key.bits < 0 || a->key.bits > 32 || a->cts.ndig > DMAX) return -1;
    return launch<LOGN, true>(*a, s);
}

}  // namespace cts

#define PCH_CTS(L)                                                                                               \
    int cts_fused_##L(const CtsArgs* a, pc_stream_t s) { return cts::cts_fused<L>(a, s); }                       \
    int cts_fused_regen_##L(const CtsRegenArgs* a, pc_stream_t s) { return cts::cts_fused_regen<L>(a, s); }
PCH_CTS(12)
PCH_CTS(13)
PCH_CTS(14)
PCH_CTS(15)
PCH_CTS(16)

}  // namespace pch
