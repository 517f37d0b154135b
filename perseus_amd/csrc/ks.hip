// Hybrid key switching on gfx950: the key inner product with the seeded half of each key regenerated in-kernel, the
// KSKA expander, key generation and packed-key expansion. Semantics: crates/pc-kernels/kernels/args.cuh KsArgs
// (:197-228), KeyTab (:284-294), KsKeyArgs (:997-1003), KskExpandArgs (:309-325), KskGenArgs (:817-833),
// KskUnpackArgs (:836-842); host twins crates/pc-host/src/ks.rs, keys.rs.
//
// The dot. A workgroup (4 waves) owns 1024 consecutive slots of one row t of Q u P and a group of keys. It stages the
// chunk's digit operands D_d (c1 itself on the rows of digit d, else the ModUp output) and c0 in LDS once; every key
// of the group reuses them, so the ModUp output is read once per batch instead of once per key. Each wave takes one
// key at a time; a lane owns 16 consecutive slots, exactly one ChaCha12 block of the KSKA stream (16 words per
// block), so the regeneration of a needs no cross-lane traffic. Per digit the lane reads its 16 words of b (dense, or
// from the bit-packed stream), regenerates a, and accumulates D b and D a in 64 bits (P c0 folded in). Rejected ChaCha
// words (v >= floor((2^32-1)/p) p, up to a few percent at 31-bit primes) go to a wave-local LDS queue that the whole
// wave redraws at once, their products added to the slot's sum with 64-bit LDS atomics, so a rare retry does not
// stall the wave. The output is scattered by sigma_k: in the bit-reversed order the high bits of automorph_slot(k, i)
// depend only on the high bits of i, so the chunk's 1024 slots land in one aligned 1024-slot chunk of the output,
// permuted; the permutation goes through LDS and the stores stay coalesced.
#include "common.h"
#include <type_traits>

#include "fused.h"

namespace pch {
namespace ks {

constexpr int DBX = 64;          // lanes per workgroup (one wave)
constexpr int DS = 16;           // slots per lane (one ChaCha block)
constexpr int DCH = DBX * DS;    // slots per workgroup

__device__ __forceinline__ int slot_of(const KeyTab& T, int t, int nq) {
    return (t < nq || T.q_top < 0) ? t : T.q_top + 1 + (t - nq);
}

// The 16 KSKA values of slots [s0, s0 + 16) of (seed, digit d, prime p) (crates/pc-core/src/keys.rs:466-498): block
// s0/16 of the ChaCha12 stream with state words (counter, d, p, tag); a rejected word is redrawn from block
// s0/16 + t N/16 (t = 1..15), the 16th attempt kept as is; value v mod p. The tag is "KSKA" for switching keys and
// "ENCA" (with d = the nonce) for an encryption's a (args.cuh:614-617).
__device__ __forceinline__ void kska16(const uint32_t (&seed)[8], uint32_t s0, uint32_t d, const Expander& ex,
                                       uint32_t n16, uint32_t (&a)[DS], uint32_t tag = TAG_KSKA) {
    const uint32_t ctr = s0 >> 4;
    uint32_t o[16];
    chacha12(seed, ctr, d, ex.p, tag, o);
    uint32_t rej = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) rej |= (uint32_t)(o[j] >= ex.mp) << j;
    while (rej) {
        const int j = __builtin_ctz(rej);
        rej &= rej - 1;
        uint32_t v = 0;
        for (int t = 1; t < KSK_T_MAX; ++t) {
            v = chacha12_word(seed, ctr + (uint32_t)t * n16, d, ex.p, tag, j);
            if (v < ex.mp) break;
        }
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) o[jj] = jj == j ? v : o[jj];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) a[j] = ex.red(o[j]);
}

constexpr int KW = 4;               // waves per workgroup: each takes one key at a time
constexpr int KBX = DBX * KW;       // threads per workgroup
constexpr int MAXD = 3;             // digits staged in LDS (more are read from global memory)
constexpr int QCAP = 1536;          // rejected-word queue entries per wave (>= 1024 free before every digit)

// D and c0 rows are staged with 4 words of padding after every 16 (a lane's 16 words start 20 words after its
// neighbour's), so the lanes' 16-byte LDS reads fall on distinct banks.
constexpr int PADW = DCH + DCH / 4;
__device__ __forceinline__ int padw(int i) { return i + (i >> 4) * 4; }

struct DotLds {
    uint32_t D[MAXD][PADW];  // the chunk's digit operands D_d (shared by every key), padded rows
    uint32_t c0[PADW];       // the chunk's c0 (mode 1: times P mod q_t; mode 2: added), padded
    struct Wave {
        uint64_t ex[DCH];    // D_d a_d of the redrawn words (64-bit LDS atomics); then the scatter buffers
        uint32_t q[QCAP];    // rejected words: digit << 16 | slot
        uint32_t qn;
    } w[KW];
};

struct DotCtx {
    const KsArgs* A;
    int c, dt, t;
    size_t trow;
    uint32_t chunk0;
    __device__ __forceinline__ const uint32_t* dptr(int d) const {
        return d == dt ? (const uint32_t*)A->c1 + c * A->ct_stride + trow
                       : (const uint32_t*)A->modup + c * A->mu_ct_stride + d * A->mu_digit_stride + trow;
    }
};

// The redraw sums' slot s lives at (s mod 16) 64 + s / 16: a lane's 16 slots are 64 entries apart, so the 64 lanes'
// clears and reads of one k touch consecutive words (bank-conflict free)
__device__ __forceinline__ uint32_t ex_slot(uint32_t s) { return (s & 15u) * DBX + (s >> 4); }

// Redraw the queued words of one wave: item = digit << 16 | slot; each lane takes items and adds D_d a_d mod p (the
// accepted attempt of the word, attempts t = 1..15 at block + t N/16) to the slot's 64-bit sum. Reduced products keep
// the sum below ndig 2^31 however many of a slot's digits were redrawn.
__device__ __forceinline__ void drain(DotLds& L, DotLds::Wave& W, const DotCtx& X, int lane, const uint32_t (&seed)[8],
                                      const Expander& ex, const Red& red, uint32_t n16) {
    wave_sync();
    const uint32_t nq = W.qn;
    for (uint32_t i = lane; i < nq; i += DBX) {
        const uint32_t it = W.q[i], d = it >> 16, sl = it & 0xFFFF;
        const uint32_t ctr = (X.chunk0 + sl) >> 4;
        uint32_t v = 0;
        for (int tt = 1; tt < KSK_T_MAX; ++tt) {
            v = chacha12_word(seed, ctr + (uint32_t)tt * n16, d, ex.p, TAG_KSKA, (int)(sl & 15));
            if (v < ex.mp) break;
        }
        const uint32_t xd = d < (uint32_t)MAXD ? L.D[d][padw(sl)] : X.dptr((int)d)[X.chunk0 + sl];
        atomicAdd((unsigned long long*)&W.ex[ex_slot(sl)], (unsigned long long)red((uint64_t)xd * ex.red(v)));
    }
    wave_sync();
    if (lane == 0) W.qn = 0;
    wave_sync();
}

// mode 0: ks_dot (dense kb / ka per key, [digit][prime id][N]); mode 1: ks_dot_key (KeyTab). WIDE: more than 4 digits
// (the 64-bit sums reduced every 3 digits). grid (N / 1024, rows, key groups), KW waves; each workgroup stages its
// chunk's D and c0 once, then wave w takes the group's keys w, w + KW, ...
template <bool WIDE>
__global__ void __launch_bounds__(KBX) dot_k(KsArgs A, KeyTab T, int logn, int mode) {
    __shared__ DotLds L;
    const int lane = threadIdx.x & (DBX - 1), wv = threadIdx.x / DBX;
    const int t = (int)A.rows[blockIdx.y];
    const PrimeConst& q = A.pr[t];
    const uint32_t p = (uint32_t)q.p;
    const Red red(q);
    const Expander ex(p);
    const uint32_t n16 = (1u << logn) >> 4;
    const uint32_t mask2n = (2u << logn) - 1;
    const uint32_t chunk0 = blockIdx.x * DCH;
    const uint32_t s0 = chunk0 + lane * DS;
    const int slot = mode == 1 ? slot_of(T, t, A.nq) : t;
    const int m0 = A.c0_mode & 3;
    const bool acc_out = (A.c0_mode & PC_KS_ACC) != 0;
    const int ndig = A.ndig;
    const int kpg = (A.R + (int)gridDim.z - 1) / (int)gridDim.z;
    const int r_lo = blockIdx.z * kpg, r_hi = min(A.R, r_lo + kpg);
    const bool pc0 = m0 == 1 && t < A.nq;
    const bool fold_c0 = pc0 && ndig <= 3;  // ndig + 1 products of (p - 1)^2 < 2^62 stay below 2^64
    const uint32_t pm = pc0 ? ((const uint32_t*)A.pmod)[t] : 0;
    const uint32_t pms = pc0 ? ((const uint32_t*)A.pmods)[t] : 0;
    const uint32_t bs0 = brev_n(s0, logn);
    DotLds::Wave& W = L.w[wv];
    DotCtx X{&A, 0, t < A.nq ? A.digit_of[t] : -1, t, (size_t)t << logn, chunk0};
    for (int c = 0; c < A.K; ++c) {
        X.c = c;
        __syncthreads();
        // stage D_d (d < MAXD) and c0 of the chunk: coalesced 16-byte loads by the whole workgroup
        for (int d = 0; d < min(ndig, MAXD); ++d) {
            const uint4* D = (const uint4*)(X.dptr(d) + chunk0);
            for (int i = threadIdx.x; i < DCH / 4; i += KBX) ((uint4*)L.D[d])[i + (i >> 2)] = D[i];
        }
        if (m0) {
            const uint4* C0 = (const uint4*)((const uint32_t*)A.c0 + c * A.ct_stride + X.trow + chunk0);
            for (int i = threadIdx.x; i < DCH / 4; i += KBX) ((uint4*)L.c0)[i + (i >> 2)] = C0[i];
        }
        __syncthreads();
        for (int r = r_lo + wv; r < r_hi; r += KW) {
            uint32_t seed[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (mode == 1 && T.nregen > 0) {
                const gptr sp = as_global(T.seed[r]);
#pragma unroll
                for (int i = 0; i < 8; ++i) seed[i] = sp[i];
            }
#pragma unroll
            for (int k = 0; k < DS; ++k) W.ex[k * DBX + lane] = 0;
            if (lane == 0) W.qn = 0;
            wave_sync();
            uint64_t s0a[DS], s1a[DS];
            uint32_t part0[WIDE ? DS : 1], part1[WIDE ? DS : 1];
#pragma unroll
            for (int k = 0; k < (WIDE ? DS : 1); ++k) part0[k] = part1[k] = 0;
            if (fold_c0) {
#pragma unroll
                for (int k = 0; k < DS; ++k) s0a[k] = (uint64_t)L.c0[padw(lane * DS) + k] * pm;
            } else {
#pragma unroll
                for (int k = 0; k < DS; ++k) s0a[k] = 0;
            }
#pragma unroll
            for (int k = 0; k < DS; ++k) s1a[k] = 0;
            for (int d = 0; d < ndig; ++d) {
                uint32_t b[DS], a[DS];
                if (mode == 0) {
                    ld16(as_global(A.kb[r]) + d * A.key_digit_stride + X.trow + s0, b);
                } else if (T.bits == 0) {
                    ld16(as_global(T.kb[r]) + (size_t)(d * T.srows + slot) * T.row_words + s0, b);
                } else {
                    // packed b: the lane's 16 values sit in words [bit0 / 32, bit0 / 32 + 16] of the row's stream
                    const gptr row = as_global(T.kb[r]) + (size_t)(d * T.srows + slot) * T.row_words;
                    const uint32_t bit0 = s0 * (uint32_t)T.bits;
                    const uint32_t msk = T.bits == 32 ? 0xFFFFFFFFu : (1u << T.bits) - 1u;
#pragma unroll
                    for (int k = 0; k < DS; ++k) {
                        const uint32_t bit = bit0 + k * (uint32_t)T.bits;
                        const uint32_t w = bit >> 5;
                        b[k] = __builtin_amdgcn_alignbit(row[w + 1], row[w], bit & 31) & msk;
                    }
                }
                if (mode == 1 && d < T.nregen) {
                    chacha12(seed, s0 >> 4, (uint32_t)d, p, TAG_KSKA, a);
                    uint32_t rej = 0;
#pragma unroll
                    for (int j = 0; j < 16; ++j) rej |= (uint32_t)(a[j] >= ex.mp) << j;
                    if (rej) {
                        // queued (the slot's sum gets D_d a_d when the wave drains the queue); counts as 0 here
                        uint32_t m = rej, i = atomicAdd(&W.qn, (uint32_t)__builtin_popcount(rej));
                        while (m) {
                            const int j = __builtin_ctz(m);
                            m &= m - 1;
                            W.q[i++] = (uint32_t)d << 16 | (lane * DS + j);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j) a[j] = (rej >> j) & 1 ? 0 : ex.red(a[j]);
                } else {
                    ld16(as_global(A.ka[r]) + d * A.key_digit_stride + X.trow + s0, a);
                }
                uint32_t x[DS];
                if (d < MAXD) ld16(L.D[d] + padw(lane * DS), x);
                else ld16(X.dptr(d) + s0, x);
#pragma unroll
                for (int k = 0; k < DS; ++k) {
                    s0a[k] += (uint64_t)x[k] * b[k];
                    s1a[k] += (uint64_t)x[k] * a[k];
                }
                if (WIDE && d % 3 == 2 && d + 1 < ndig) {
#pragma unroll
                    for (int k = 0; k < DS; ++k) {
                        part0[k] = addm(part0[k], red(s0a[k]), p);
                        part1[k] = addm(part1[k], red(s1a[k]), p);
                        s0a[k] = s1a[k] = 0;
                    }
                }
                // room for a whole digit's words before the next one (wave-uniform: qn is shared)
                wave_sync();
                if (W.qn > (uint32_t)(QCAP - DCH)) drain(L, W, X, lane, seed, ex, red, n16);
            }
            drain(L, W, X, lane, seed, ex, red, n16);
            uint32_t r0[DS], r1[DS];
#pragma unroll
            for (int k = 0; k < DS; ++k) {
                const uint64_t e = W.ex[k * DBX + lane];
                if (WIDE) {
                    r0[k] = addm(part0[k], red(s0a[k]), p);
                    r1[k] = addm(addm(part1[k], red(s1a[k]), p), red(e), p);
                } else {
                    r0[k] = red(s0a[k]);
                    r1[k] = red(s1a[k] + e);  // ndig <= 4 products of (p - 1)^2 plus ndig words below p: < 2^64
                }
            }
            if ((pc0 && !fold_c0) || m0 == 2) {
#pragma unroll
                for (int k = 0; k < DS; ++k) {
                    const uint32_t cz = L.c0[padw(lane * DS) + k];
                    r0[k] = addm(r0[k], m0 == 2 ? cz : shoup(cz, pm, pms, p), p);
                }
            }
            const uint32_t kexp = A.autok[r];
            uint32_t* o0 = (uint32_t*)A.out0 + c * A.out_ct_stride + r * A.out_rot_stride + X.trow;
            uint32_t* o1 = (uint32_t*)A.out1 + c * A.out_ct_stride + r * A.out_rot_stride + X.trow;
            if (kexp == 1 && !acc_out) {
                st16(o0 + s0, r0);
                st16(o1 + s0, r1);
                continue;
            }
            // sigma_k on the way out, through the conflict-free scatter addresses (scat_addr above)
            uint32_t* l0 = (uint32_t*)W.ex;
            uint32_t* l1 = l0 + DCH;
            wave_sync();
            const int sh = logn - 9;
            const uint32_t cbh = (((2 * bs0 + 1) * kexp) & mask2n) >> sh;
            const uint32_t sth = ((kexp << (logn - 3)) & mask2n) >> sh;
#pragma unroll
            for (int k = 0; k < DS; ++k) {
                const uint32_t o = scat_addr((cbh + brev4(k) * sth) & (DCH - 1));
                l0[o] = r0[k];
                l1[o] = r1[k];
            }
            wave_sync();
            const uint32_t ob = (automorph_slot(kexp, chunk0, logn) & ~(uint32_t)(DCH - 1)) + lane * DS;
            const uint32_t rb = scat_addr(__brev((uint32_t)lane) >> 26);
            uint32_t v0[DS], v1[DS];
#pragma unroll
            for (int j = 0; j < DS; ++j) {
                v0[j] = l0[rb + 32 * brev4(j)];
                v1[j] = l1[rb + 32 * brev4(j)];
            }
            if (acc_out) {
                uint32_t e0[DS], e1[DS];
                ld16(o0 + ob, e0);
                ld16(o1 + ob, e1);
#pragma unroll
                for (int k = 0; k < DS; ++k) {
                    v0[k] = addm(v0[k], e0[k], p);
                    v1[k] = addm(v1[k], e1[k], p);
                }
            }
            st16(o0 + ob, v0);
            st16(o1 + ob, v1);
            wave_sync();
        }
    }
}

// The hot case of the dot, specialised: one ciphertext, dense b through a KeyTab, every digit's a regenerated, NDIG
// (<= 3) live digits unrolled. D and c0 are staged once per workgroup as in dot_k. A lane that meets rejected ChaCha
// words appends them to its wave's queue (slot and digit; the queue position of each digit's first entry is kept),
// and leaves their products out of its sums; the whole wave then redraws the queued words at once, writing each
// accepted value back into its queue entry. The output goes through one 1024-word scatter buffer per wave, one part at
// a time; each owner adds D_d a_d of its redrawn words into its slots there, after the scatter write of s1. A wave
// needs 8 KB of LDS, so three workgroups fit on a CU.
constexpr int FQCAP = DCH;  // queue entries per wave

struct FastWave {
    uint32_t buf[DCH];  // scatter buffer
    uint32_t q[FQCAP];  // rejected words: (digit << 16 | slot), then the redrawn value
    uint32_t qn;
};
// KW waves (one key each) share the chunk's D and c0 staged in LDS; a launch with fewer keys than KW runs one-wave
// workgroups that read D and c0 straight from memory (their LDS holds the wave's buffers only), so the chip keeps
// enough waves in flight on a single key
struct FastLds {
    uint32_t D[MAXD][PADW];
    uint32_t c0[PADW];
    FastWave w[KW];
};
struct FastLds1 {
    FastWave w[1];
};


// KSKA value of an accepted word v < floor((2^32-1)/p) p. MU2: floor((2^32-1)/p) = 2 (every p > (2^32-1)/3), where
// v < 2p needs one conditional subtraction.
template <bool MU2>
__device__ __forceinline__ uint32_t kska_value(const Expander& ex, uint32_t v) {
    return MU2 ? min(v, v - ex.p) : ex.red(v);
}

struct FastCtx {
    const KsArgs* A;
    const KeyTab* T;
    const uint32_t* D[MAXD];  // the chunk's D_d words (LDS, padded; or memory), this lane's at lp
    const uint32_t* c0;
    gptr c0b;  // c0 mode 3: the chunk's words of the second part (memory), this lane's at 16 lane
    FastWave* W;
    int lane, lp, slot, logn, m0;
    bool acc_out, pc0;
    size_t oct;  // this workgroup's ciphertext's output offset (words)
    uint32_t p, pm, n16, mask2n, chunk0, s0, bs0, rb;
    size_t trow;
};

// wave-wide exclusive prefix over lanes of a count below 32 (five ballots)
__device__ __forceinline__ uint32_t lane_prefix(uint32_t cnt, int lane) {
    const uint64_t below = (1ull << lane) - 1;
    uint32_t pre = 0;
#pragma unroll
    for (int b = 0; b < 5; ++b) pre += (uint32_t)__popcll(__ballot((cnt >> b) & 1) & below) << b;
    return pre;
}

// The 16 values of slots [s0, s0 + 16) of a bit-packed key row (value i at bits [i BITS, (i + 1) BITS) of the row's
// little-endian stream, crates/pc-gpu/src/keys.rs:54-58): the lane's words w0 .. w0 + 16, read as four 16-byte loads
// and one word (the row's guard word keeps w0 + 16 inside the row). With s0 a multiple of 16 the first value starts
// at bit 0 of w0 (even BITS) or at bit 0 or 16 (odd BITS, by the lane's parity): the window is realigned by that shift
// once, so every value's position is a compile-time constant.
template <int BITS>
__device__ __forceinline__ void ldpk16(gptr row, uint32_t s0, uint32_t (&out)[DS]) {
    const uint32_t bit0 = s0 * BITS;
    const gptr p = row + (bit0 >> 5);
    uint32_t w[17];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const gu4a4 v = *(const __attribute__((address_space(1))) gu4a4*)(p + 4 * i);
        w[4 * i] = v.x, w[4 * i + 1] = v.y, w[4 * i + 2] = v.z, w[4 * i + 3] = v.w;
    }
    w[16] = p[16];
    if (BITS & 1) {
        const uint32_t sh = bit0 & 31;
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], sh);
    }
    constexpr uint32_t mask = BITS == 32 ? 0xFFFFFFFFu : (1u << BITS) - 1u;
#pragma unroll
    for (int k = 0; k < DS; ++k) {
        const int pos = k * BITS, wi = pos >> 5, off = pos & 31;
        const uint32_t v = off + BITS <= 32 ? w[wi] >> off : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], off);
        out[k] = v & mask;
    }
}

// PATCH: the retry values come from the key group's table (P) instead of the wave's redraw. PK: key b bit-packed at
// PK bits (0: dense words). F: c0 mode 3 handled (the one-wave form; its second-part words held through the ChaCha
// blocks)
// RES: digits >= KeyTab.nregen read the key's resident dense `a` (KsArgs.ka[r] + d key_digit_stride, prime-id rows:
// the reference's keys with a stored `a`, crates/pc-gpu/src/ks.rs:1259-1262), the others regenerated
template <int NDIG, bool MU2, bool PATCH, int PK, bool F, bool RES = false>
__device__ __forceinline__ void dot_fast_key(const FastCtx& C, const Red& red, const Expander& ex, int r,
                                             const PatchTab& P) {
    const KsArgs& A = *C.A;
    const KeyTab& T = *C.T;
    FastWave& W = *C.W;
    const int lane = C.lane, lp = C.lp;
    const uint32_t p = C.p, s0 = C.s0;
    // the key's tables (row pointer, seed, automorphism exponent, retry-list offsets) are uniform over the wave and
    // read-only: scalar loads, whose waits do not include the vector memory counter (the previous key's stores)
    const gptr kb = as_global(sload(T.kb + r)) + (size_t)C.slot * T.row_words + (PK ? 0 : s0);
    const size_t dstride = (size_t)T.srows * T.row_words;
    uint32_t seed[8];
    const uint32_t* sp = sload(T.seed + r);
#pragma unroll
    for (int i = 0; i < 8; ++i) seed[i] = sload(sp + i);
    const uint32_t kexp = sload(A.autok + r);
    if (lane == 0) W.qn = 0;
    wave_sync();
    // PATCH: this chunk's retry values of each digit, loaded now (two per lane) and stored to the queue after the
    // ChaCha blocks; a digit whose list would overflow the queue is read from the table when the words are patched
    const int nreg = RES ? T.nregen : NDIG;
    uint32_t poff[PATCH ? NDIG : 1], pn[PATCH ? NDIG : 1], pv[PATCH ? NDIG : 1][2];
    if constexpr (PATCH) {
        const uint32_t chunks = (1u << C.logn) / DCH;
        uint32_t tot = 0, i1[NDIG];
        // every digit's offsets first (one wait for all)
#pragma unroll
        for (int d = 0; d < NDIG; ++d) {
            const size_t ix = (((size_t)r * P.ndig + d) * P.rows + C.slot) * chunks + C.chunk0 / DCH;
            poff[d] = sload(P.idx + ix);
            i1[d] = sload(P.idx + ix + 1);
        }
#pragma unroll
        for (int d = 0; d < NDIG; ++d) {
            if (RES && d >= nreg) {
                // a resident digit: no retry values
                poff[d] = pn[d] = pv[d][0] = pv[d][1] = 0;
                continue;
            }
            pn[d] = i1[d] - poff[d];
            if (tot + pn[d] > (uint32_t)FQCAP) pn[d] = 0xFFFFFFFFu;  // read from memory when patched
            else tot += pn[d];
            const bool ok = pn[d] != 0xFFFFFFFFu;
            pv[d][0] = ok && (uint32_t)lane < pn[d] ? P.val[poff[d] + lane] : 0;
            pv[d][1] = ok && (uint32_t)lane + DBX < pn[d] ? P.val[poff[d] + lane + DBX] : 0;
        }
    }
    // s1 = sum_d D_d a_d, a regenerated (one ChaCha12 block per lane and digit); rejected words contribute later
    uint64_t acc[DS];
#pragma unroll
    for (int k = 0; k < DS; ++k) acc[k] = 0;
    uint32_t rejd[NDIG], based[NDIG];
    uint32_t pbase = 0;
#pragma unroll
    for (int d = 0; d < NDIG; ++d) {
        uint32_t a[DS];
        uint32_t rej = 0;
        uint32_t base = 0;
        if (RES && d >= nreg) {
            // canonical words: kska_value leaves them as they are
            ld16(as_global(((const void* const*)A.ka)[r]) + (size_t)d * A.key_digit_stride + C.trow + s0, a);
        } else {
            chacha12(seed, s0 >> 4, (uint32_t)d, p, TAG_KSKA, a);
            if constexpr (MU2) {
                // reduced at once: z = min(v, v - p) is v mod p for v < 2p, and z >= p exactly when v >= 2p (rejected:
                // 0 here, its bit in rej, built by shifts)
#pragma unroll
                for (int j = 15; j >= 0; --j) {
                    const uint32_t z = min(a[j], a[j] - p);
                    const bool bad = z >= p;
                    rej = rej << 1 | (uint32_t)bad;
                    a[j] = bad ? 0u : z;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) rej |= (uint32_t)(a[j] >= ex.mp) << j;
            }
            if constexpr (PATCH) {
                // the table lists this chunk's rejected words in slot order: this lane's come after the lower lanes'.
                // A list that does not fit the queue is read from the table in memory (top bit of base)
                const uint32_t pre = lane_prefix(__builtin_popcount(rej), lane);
                if (pn[d] != 0xFFFFFFFFu) {
                    base = pbase + pre;
                    pbase += pn[d];
                } else {
                    base = poff[d] + pre;
                }
            } else if (rej) {
                const uint32_t cnt = __builtin_popcount(rej);
                base = atomicAdd(&W.qn, cnt);
                if (base + cnt <= (uint32_t)FQCAP) {
                    uint32_t m = rej, i = base;
#pragma unroll 1
                    while (m) {
                        const int j = __builtin_ctz(m);
                        m &= m - 1;
                        W.q[i++] = (uint32_t)d << 16 | (lane * DS + j);
                    }
                } else {
                    // the queue is full (rejection rates far above any prime of this path's): redraw in the lane
                    uint32_t m = rej;
                    while (m) {
                        const int j = __builtin_ctz(m);
                        m &= m - 1;
                        uint32_t v = 0;
                        for (int tt = 1; tt < KSK_T_MAX; ++tt) {
                            v = chacha12_word(seed, (s0 >> 4) + (uint32_t)tt * C.n16, (uint32_t)d, p, TAG_KSKA, j);
                            if (v < ex.mp) break;
                        }
                        const uint32_t nv = MU2 ? kska_value<true>(ex, v) : v;
#pragma unroll
                        for (int jj = 0; jj < 16; ++jj) a[jj] = jj == j ? nv : a[jj];
                    }
                    rej = 0;
                }
            }
        }
        rejd[d] = rej;
        based[d] = base;
        uint32_t x[DS];
        ld16(C.D[d] + lp, x);
#pragma unroll
        for (int k = 0; k < DS; ++k) acc[k] += (uint64_t)x[k] * (MU2 ? a[k] : (rej >> k) & 1 ? 0 : ex.red(a[k]));
        // materialise the sums here: this digit's a words die before the next block is computed
#pragma unroll
        for (int k = 0; k < DS; ++k) asm volatile("" : "+v"(acc[k]));
    }
    // c0 mode 3 (F): + P c0' (the second part's words, loaded with b, added at s1's reduction): ndig + 1 <= 4 products
    // of (p - 1)^2 < 2^62
    uint32_t cw1[F ? DS : 1];
    const bool f3 = F && C.m0 == 3 && C.pc0;
    if constexpr (F) {
        if (f3) ld16(C.c0b + lane * DS, cw1);
    }
    // the key's b rows: they arrive while the queued words are redrawn and s1 goes out, and are consumed last
    uint32_t b[NDIG][DS];
#pragma unroll
    for (int d = 0; d < NDIG; ++d) {
        if constexpr (PK == 0) ld16(kb + d * dstride, b[d]);
        else ldpk16<PK>(kb + d * dstride, s0, b[d]);
    }
    // redraw the queued words: entry <- accepted value mod p (PATCH: the table's values into the queue)
    wave_sync();
    uint32_t nq = 0;
    if constexpr (PATCH) {
        uint32_t b0 = 0;
#pragma unroll
        for (int d = 0; d < NDIG; ++d) {
            if (pn[d] == 0xFFFFFFFFu) continue;
            if ((uint32_t)lane < pn[d]) W.q[b0 + lane] = pv[d][0];
            if ((uint32_t)lane + DBX < pn[d]) W.q[b0 + lane + DBX] = pv[d][1];
            for (uint32_t i = lane + 2 * DBX; i < pn[d]; i += DBX) W.q[b0 + i] = P.val[poff[d] + i];
            b0 += pn[d];
        }
    } else {
        nq = min(W.qn, (uint32_t)FQCAP);
    }
    for (uint32_t i = lane; i < nq; i += DBX) {
        const uint32_t it = W.q[i], d = it >> 16, sl = it & 0xFFFF;
        const uint32_t ctr = (C.chunk0 + sl) >> 4;
        uint32_t v = 0;
        for (int tt = 1; tt < KSK_T_MAX; ++tt) {
            v = chacha12_word(seed, ctr + (uint32_t)tt * C.n16, d, p, TAG_KSKA, (int)(sl & 15));
            if (v < ex.mp) break;
        }
        W.q[i] = ex.red(v);
    }
    uint32_t* o0 = (uint32_t*)A.out0 + C.oct + r * A.out_rot_stride + C.trow;
    uint32_t* o1 = (uint32_t*)A.out1 + C.oct + r * A.out_rot_stride + C.trow;
    // W_k = top 10 bits of (cb + brev4(k) step) mod 2N; step's low logn - 3 bits are zero, so the sum's top bits are
    // (cb >> sh) + brev4(k) (step >> sh) modulo 1024
    const int sh = C.logn - 9;
    const uint32_t cbh = (((2 * C.bs0 + 1) * kexp) & C.mask2n) >> sh;
    const uint32_t sth = ((kexp << (C.logn - 3)) & C.mask2n) >> sh;
    const uint32_t ob = (automorph_slot(kexp, C.chunk0, C.logn) & ~(uint32_t)(DCH - 1)) + lane * DS;
    uint32_t* buf = W.buf;
    // out one part through the scatter buffer: v[j] = the word of output offset 16 lane + j
    auto emit = [&](uint32_t (&v)[DS], uint32_t* o) {
        wave_sync();
#pragma unroll
        for (int j = 0; j < DS; ++j) v[j] = buf[C.rb + 32 * brev4(j)];
        o += ob;
        if (C.acc_out) {
            uint32_t e[DS];
            ld16(o, e);
#pragma unroll
            for (int k = 0; k < DS; ++k) v[k] = addm(v[k], e[k], p);
        }
        st16(o, v);
        wave_sync();
    };
    {
        // s1 first (its registers free before s0's): reduce, scatter, add D_d a_d of this lane's redrawn words
        uint32_t v[DS];
#pragma unroll
        for (int k = 0; k < DS; ++k) {
            uint64_t x = acc[k];
            if constexpr (F) x += f3 ? (uint64_t)cw1[k] * C.pm : 0;
            buf[scat_addr((cbh + brev4(k) * sth) & (DCH - 1))] = red(x);
        }
#pragma unroll
        for (int d = 0; d < NDIG; ++d) {
            // the values from the queue in LDS, or (a list too long for it: uniform over the wave) from the table in
            // memory; two loops, so that the LDS one waits for no memory load
            auto patch = [&](auto value) {
                uint32_t m = rejd[d], i = based[d];
#pragma unroll 1
                while (m) {
                    const uint32_t j = __builtin_ctz(m);
                    m &= m - 1;
                    const uint32_t add = red.mul(C.D[d][lp + j], value(i++));
                    const uint32_t o = scat_addr((cbh + brev4(j) * sth) & (DCH - 1));
                    buf[o] = addm(buf[o], add, p);
                }
            };
            if (PATCH && __builtin_amdgcn_readfirstlane(pn[PATCH ? d : 0]) == 0xFFFFFFFFu)
                patch([&](uint32_t i) { return P.val[i]; });
            else
                patch([&](uint32_t i) { return W.q[i]; });
        }
        emit(v, o1);
    }
    // s0 = sum_d D_d b_d (+ P c0 folded in: ndig + 1 <= 4 products of (p - 1)^2 < 2^62)
    uint32_t cw[DS];
    if (C.m0) ld16(C.c0 + lp, cw);
#pragma unroll
    for (int k = 0; k < DS; ++k) acc[k] = (C.m0 == 2 || !C.pc0) ? 0 : (uint64_t)cw[k] * C.pm;
#pragma unroll
    for (int d = 0; d < NDIG; ++d) {
        uint32_t x[DS];
        ld16(C.D[d] + lp, x);
#pragma unroll
        for (int k = 0; k < DS; ++k) acc[k] += (uint64_t)x[k] * b[d][k];
    }
    {
        uint32_t v[DS];
#pragma unroll
        for (int k = 0; k < DS; ++k) {
            uint32_t r0 = red(acc[k]);
            if (C.m0 == 2) r0 = addm(r0, cw[k], p);
            buf[scat_addr((cbh + brev4(k) * sth) & (DCH - 1))] = r0;
        }
        emit(v, o0);
    }
}

// NW: waves per workgroup (KW: staged D and c0, one key per wave; 1: read from memory)
template <int NDIG, bool PATCH, int NW, int PK = 0, bool RES = false>
__global__ void __launch_bounds__(DBX * NW, 3) dot_fast(KsArgs A, KeyTab T, PatchTab P, int logn) {
    static_assert(NDIG >= 1 && NDIG <= MAXD, "digits staged in LDS");
    static_assert(NW == KW || NW == 1, "staged (KW waves) or direct (one wave)");
    static_assert(3 * sizeof(FastLds) <= 160 * 1024, "three workgroups per CU");
    using Lds = typename std::conditional<NW == KW, FastLds, FastLds1>::type;
    __shared__ Lds L;
    // the wave index is uniform across the wave: in scalar registers, so are its key, seed and row pointers
    const int lane = threadIdx.x & (DBX - 1), wv = __builtin_amdgcn_readfirstlane(threadIdx.x / DBX);
    const int t = (int)A.rows[blockIdx.y];
    const PrimeConst& q = A.pr[t];
    FastCtx C;
    C.A = &A;
    C.T = &T;
    C.W = &L.w[wv];
    C.lane = lane;
    C.slot = slot_of(T, t, A.nq);
    C.logn = logn;
    C.m0 = A.c0_mode & 3;
    C.acc_out = (A.c0_mode & PC_KS_ACC) != 0;
    C.pc0 = (C.m0 == 1 || C.m0 == 3) && t < A.nq;
    C.p = (uint32_t)q.p;
    C.pm = C.pc0 ? ((const uint32_t*)A.pmod)[t] : 0;
    C.n16 = (1u << logn) >> 4;
    C.mask2n = (2u << logn) - 1;
    C.chunk0 = blockIdx.x * DCH;
    C.s0 = C.chunk0 + lane * DS;
    C.bs0 = brev_n(C.s0, logn);
    C.rb = scat_addr(__brev((uint32_t)lane) >> 26);  // read base of output offsets 16 lane + j
    C.trow = (size_t)t << logn;
    const Red red(q);
    const Expander ex(C.p);
    // grid z: K ciphertexts x key groups
    const int ng = (int)gridDim.z / A.K, cix = (int)blockIdx.z / ng, kg = (int)blockIdx.z % ng;
    const int kpg = (A.R + ng - 1) / ng;
    int r_lo = kg * kpg, r_hi = min(A.R, r_lo + kpg);
    if (P.diag) r_lo = cix, r_hi = cix + 1;  // ciphertext cix under key cix alone
    C.oct = (size_t)cix * A.out_ct_stride;
    DotCtx X{&A, cix, t < A.nq ? A.digit_of[t] : -1, t, C.trow, C.chunk0};
    const uint32_t* c0row = (const uint32_t*)A.c0 + (size_t)cix * A.ct_stride + C.trow + C.chunk0;
    C.c0b = C.m0 == 3 ? as_global(c0row + A.ct_stride / 2) : nullptr;
    if constexpr (NW == KW) {
        C.lp = padw(lane * DS);  // this lane's 16 words in the padded rows
#pragma unroll
        for (int d = 0; d < NDIG; ++d) {
            const uint4* D = (const uint4*)(X.dptr(d) + C.chunk0);
            for (int i = threadIdx.x; i < DCH / 4; i += KBX) ((uint4*)L.D[d])[i + (i >> 2)] = D[i];
            C.D[d] = L.D[d];
        }
        if (C.m0) {
            const uint4* C0 = (const uint4*)c0row;
            for (int i = threadIdx.x; i < DCH / 4; i += KBX) ((uint4*)L.c0)[i + (i >> 2)] = C0[i];
        }
        C.c0 = L.c0;
        __syncthreads();
    } else {
        C.lp = lane * DS;
#pragma unroll
        for (int d = 0; d < NDIG; ++d) C.D[d] = X.dptr(d) + C.chunk0;
        C.c0 = C.m0 ? c0row : nullptr;
    }
    if (ex.mu == 2) {
        for (int r = r_lo + wv; r < r_hi; r += NW) dot_fast_key<NDIG, true, PATCH, PK, NW == 1, RES>(C, red, ex, r, P);
    } else {
        for (int r = r_lo + wv; r < r_hi; r += NW) dot_fast_key<NDIG, false, PATCH, PK, NW == 1, RES>(C, red, ex, r, P);
    }
}

// the fast dot's launch: one-wave direct workgroups when the launch has fewer keys than a staged workgroup's waves
template <int NDIG, bool PATCH, int PK = 0, bool RES = false>
void dot_fast_launch(dim3 grid, const KsArgs& a, const KeyTab& key, const PatchTab& P, int logn, hipStream_t st) {
    if (P.diag || a.R < KW) {
        grid.z = P.diag ? a.K : a.R * a.K;
        hipLaunchKernelGGL((dot_fast<NDIG, PATCH, 1, PK, RES>), grid, dim3(DBX), 0, st, a, key, P, logn);
    } else {
        hipLaunchKernelGGL((dot_fast<NDIG, PATCH, KW, PK, RES>), grid, dim3(KBX), 0, st, a, key, P, logn);
    }
}
// the fast dot's packed-b widths (the reference's PackedSeeded keys store b at the widest prime's bits)
template <int PK>
void dot_fast_pk(int ndig, dim3 grid, const KsArgs& a, const KeyTab& key, int logn, hipStream_t st) {
    const PatchTab none = {};
    if (ndig == 1) dot_fast_launch<1, false, PK>(grid, a, key, none, logn, st);
    if (ndig == 2) dot_fast_launch<2, false, PK>(grid, a, key, none, logn, st);
    if (ndig == 3) dot_fast_launch<3, false, PK>(grid, a, key, none, logn, st);
}

template <int LOGN>
int dot_launch(const KsArgs& a, const KeyTab& key, int mode, pc_stream_t s) {
    static_assert((1 << LOGN) >= DCH, "ring of at least 1024 slots");
    if (a.nrows < 0 || a.R < 0 || a.K < 0 || a.ndig < 0) return -1;
    if (a.nrows == 0 || a.R == 0 || a.K == 0) return 0;
    if (!a.rows || !a.pr || !a.c1 || !a.out0 || !a.out1 || !a.autok || !a.digit_of) return -1;
    if (a.ndig > 0 && !a.modup) return -1;
    if ((a.c0_mode & 3) == 1 && (!a.c0 || !a.pmod || !a.pmods)) return -1;
    if ((a.c0_mode & 3) == 2 && !a.c0) return -1;
    if ((a.c0_mode & 3) == 3) return -1;
    // key groups: enough workgroups to fill the chip, each group sharing one staging of D
    const int chunks = (1 << LOGN) / DCH;
    int groups = 1;
    while (groups < a.R && (long)chunks * a.nrows * groups < 2048) ++groups;
    dim3 grid(chunks, a.nrows, groups);
    const bool pk_fast = key.bits == 0 || key.bits == 30 || key.bits == 31;
    const bool fast = mode == 1 && a.K <= 4 && pk_fast && key.nregen >= a.ndig && a.ndig >= 1 && a.ndig <= 3;
    if (fast) {
        // the fast dot takes the K ciphertexts through grid z (K x its key groups)
        int gf = 1;
        while (gf < a.R && (long)chunks * a.nrows * gf * a.K < 2048) ++gf;
        const dim3 g(chunks, a.nrows, gf * a.K);
        if (key.bits == 0) dot_fast_pk<0>(a.ndig, g, a, key, LOGN, (hipStream_t)s);
        if (key.bits == 30) dot_fast_pk<30>(a.ndig, g, a, key, LOGN, (hipStream_t)s);
        if (key.bits == 31) dot_fast_pk<31>(a.ndig, g, a, key, LOGN, (hipStream_t)s);
    } else if (a.ndig > 4) hipLaunchKernelGGL(dot_k<true>, grid, dim3(KBX), 0, (hipStream_t)s, a, key, LOGN, mode);
    else hipLaunchKernelGGL(dot_k<false>, grid, dim3(KBX), 0, (hipStream_t)s, a, key, LOGN, mode);
    return launch_rc();
}

// the fast dot with a retry-value table (driver-internal; the table entry ks_dot_key redraws)
template <int LOGN>
int dot_patched(const KsKeyArgs* g, const PatchTab* P, pc_stream_t s) {
    if (!g || !P || !P->idx || !P->val) return -1;
    const KsArgs& a = g->ks;
    const KeyTab& key = g->key;
    // digits >= nregen: the keys' resident dense `a` (full layout)
    const bool res = key.nregen < a.ndig;
    if (a.K < 1 || a.K > (P->diag ? 8 : 4) || key.bits != 0 || key.nregen < 0 || a.ndig < 1 || a.ndig > 3 ||
        a.ndig > P->ndig || key.q_top >= 0 || key.srows != P->rows || (P->diag && (a.R != a.K || (a.c0_mode & 3) == 3)) ||
        (res && (!a.ka || a.key_digit_stride < (uint64_t)key.srows << LOGN)))
        return -2;
    if (a.nrows < 0 || a.R < 0) return -1;
    if (a.nrows == 0 || a.R == 0) return 0;
    if (!a.rows || !a.pr || !a.c1 || !a.out0 || !a.out1 || !a.autok || !a.digit_of || !a.modup) return -1;
    if ((a.c0_mode & 3) != 0 && (a.c0_mode & 3) != 2 && (!a.c0 || !a.pmod || !a.pmods)) return -1;
    if ((a.c0_mode & 3) == 2 && !a.c0) return -1;
    if ((a.c0_mode & 3) == 3 && ((a.ct_stride & 1) || a.R >= KW)) return -2;  // mode 3: the one-wave form only
    if (!key.kb || !key.seed) return -1;
    const int chunks = (1 << LOGN) / DCH;
    int groups = 1;
    while (groups < a.R && (long)chunks * a.nrows * groups * a.K < 2048) ++groups;
    const dim3 grid(chunks, a.nrows, groups * a.K);
    hipStream_t st = (hipStream_t)s;
    if (res) {
        if (a.ndig == 1) dot_fast_launch<1, true, 0, true>(grid, a, key, *P, LOGN, st);
        if (a.ndig == 2) dot_fast_launch<2, true, 0, true>(grid, a, key, *P, LOGN, st);
        if (a.ndig == 3) dot_fast_launch<3, true, 0, true>(grid, a, key, *P, LOGN, st);
        return launch_rc();
    }
    if (a.ndig == 1) dot_fast_launch<1, true>(grid, a, key, *P, LOGN, st);
    if (a.ndig == 2) dot_fast_launch<2, true>(grid, a, key, *P, LOGN, st);
    if (a.ndig == 3) dot_fast_launch<3, true>(grid, a, key, *P, LOGN, st);
    return launch_rc();
}

// The retry table's two passes: one wave per (chunk, row, key x digit) regenerates the chunk's KSKA blocks, counts
// its rejected words, then (fill) writes their redrawn values in slot order.
template <bool FILL>
__global__ void __launch_bounds__(DBX) patch_k(const uint32_t* const* seeds, const PrimeConst* pr, int ndig, int rows,
                                              int logn, uint32_t* counts, const uint32_t* idx, uint32_t* val) {
    const int lane = threadIdx.x, t = blockIdx.y, r = blockIdx.z / ndig, d = blockIdx.z % ndig;
    const uint32_t chunks = (1u << logn) / DCH;
    const size_t ix = (((size_t)r * ndig + d) * rows + t) * chunks + blockIdx.x;
    const uint32_t p = (uint32_t)pr[t].p;
    const Expander ex(p);
    uint32_t seed[8];
    const uint32_t* sp = seeds[r];
#pragma unroll
    for (int i = 0; i < 8; ++i) seed[i] = sp[i];
    const uint32_t s0 = blockIdx.x * DCH + lane * DS, n16 = (1u << logn) >> 4;
    uint32_t a[DS];
    chacha12(seed, s0 >> 4, (uint32_t)d, p, TAG_KSKA, a);
    uint32_t rej = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) rej |= (uint32_t)(a[j] >= ex.mp) << j;
    const uint32_t cnt = __builtin_popcount(rej);
    if (!FILL) {
        const uint32_t tot = __popcll(__ballot(cnt & 1)) + 2 * __popcll(__ballot(cnt & 2)) +
                             4 * __popcll(__ballot(cnt & 4)) + 8 * __popcll(__ballot(cnt & 8)) +
                             16 * __popcll(__ballot(cnt & 16));
        if (lane == 0) counts[ix] = tot;
        return;
    }
    uint32_t o = idx[ix] + lane_prefix(cnt, lane);
    while (rej) {
        const int j = __builtin_ctz(rej);
        rej &= rej - 1;
        uint32_t v = 0;
        for (int tt = 1; tt < KSK_T_MAX; ++tt) {
            v = chacha12_word(seed, (s0 >> 4) + (uint32_t)tt * n16, (uint32_t)d, p, TAG_KSKA, j);
            if (v < ex.mp) break;
        }
        val[o++] = ex.red(v);
    }
}

// ks_dot: K <= 8 ciphertexts x R keys stored dense (crates/pc-host/src/ks.rs:139-162: KS_SUM -3, K > 8 -1)
template <int LOGN>
int ks_dot(const KsArgs* a, pc_stream_t s) {
    if (!a) return -1;
    if (a->c0_mode & PC_KS_SUM) return -3;
    if (a->K > 8) return -1;
    if (!a->kb || !a->ka) return -1;
    KeyTab none = {};
    return dot_launch<LOGN>(*a, none, 0, s);
}

// ks_dot_key: keys through a KeyTab (crates/pc-host/src/ks.rs:164-200: bits outside 0..=32 -1, K > 4 -2); the summed
// rotations (KS_SUM) run the gather-form kernel.
template <int LOGN>
int ks_dot_key(const KsKeyArgs* g, pc_stream_t s) {
    if (!g) return -1;
    if (g->key.bits < 0 || g->key.bits > 32) return -1;
    if (g->ks.K > 4) return -2;
    if (g->ks.c0_mode & PC_KS_SUM) return ks_dot_key_sum(LOGN, g, s);
    if (!g->key.kb || (g->key.nregen > 0 && !g->key.seed)) return -1;
    if (g->ks.ndig > g->key.nregen && !g->ks.ka) return -1;
    if (g->key.bits > 0 && (g->key.row_words % 4 != 0)) return -1;
    return dot_launch<LOGN>(g->ks, g->key, 1, s);
}

// ------------------------------------------------------------------------------------------------ expander
__global__ void __launch_bounds__(DBX) expand_k(KskExpandArgs A, int logn) {
    const int m = blockIdx.y, z = blockIdx.z;
    const int id = A.prime_ids[m];
    const uint32_t p = (uint32_t)A.pr[id].p;
    const Expander ex(p);
    uint32_t seed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) seed[i] = A.seed[i];
    const uint32_t s0 = blockIdx.x * DCH + threadIdx.x * DS;
    uint32_t a[DS];
    kska16(seed, s0, (uint32_t)(A.d0 + z), ex, (1u << logn) >> 4, a);
    st16((uint32_t*)A.out + (((size_t)z * A.nmod + m) << logn) + s0, a);
}

template <int LOGN>
int ksk_expand(const KskExpandArgs* a, pc_stream_t s) {
    if (!a || !a->out || !a->seed || !a->prime_ids || !a->pr) return -1;
    if (a->d0 < 0 || a->d0 >= a->dnum || a->nmod < 0) return -1;
    if (a->nmod == 0) return 0;
    hipLaunchKernelGGL(expand_k, dim3((1 << LOGN) / DCH, a->nmod, a->dnum - a->d0), dim3(DBX), 0, (hipStream_t)s, *a,
                       LOGN);
    return launch_rc();
}

// ------------------------------------------------------------------------------------------------ encryption
// Secret-key encryption in the evaluation domain, limb l = prime id l (args.cuh:613-628; encrypt.cuh:10-31): a from the
// "ENCA" expander lane (w13 = nonce), c0 = e + m - a s, c1 = a when c1 is set. One ChaCha block per lane; e (and m) may
// alias c0: a lane reads its 16 words before it writes them.
__global__ void __launch_bounds__(DBX) encrypt_k(EncryptArgs A, int logn) {
    const int l = blockIdx.y;
    const Red red(A.pr[l]);
    const Expander ex(red.p);
    uint32_t seed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) seed[i] = A.seed[i];
    const uint32_t s0 = blockIdx.x * DCH + threadIdx.x * DS;
    uint32_t a[DS];
    kska16(seed, s0, A.nonce, ex, (1u << logn) >> 4, a, TAG_ENCA);
    const size_t off = ((size_t)l << logn) + s0;
    uint32_t sv[DS], e[DS], m[DS];
    ld16((const uint32_t*)A.s + off, sv);
    ld16((const uint32_t*)A.e + off, e);
    if (A.m) {
        ld16((const uint32_t*)A.m + off, m);
    } else {
#pragma unroll
        for (int j = 0; j < DS; ++j) m[j] = 0;
    }
#pragma unroll
    for (int j = 0; j < DS; ++j) e[j] = subm(addm(e[j], m[j], red.p), red.mul(a[j], sv[j]), red.p);
    st16((uint32_t*)A.c0 + off, e);
    if (A.c1) st16((uint32_t*)A.c1 + off, a);
}

template <int LOGN>
int encrypt(const EncryptArgs* a, pc_stream_t s) {
    if (!a || !a->c0 || !a->s || !a->e || !a->seed || !a->pr || a->nl < 0) return -1;
    if (a->nl == 0) return 0;
    hipLaunchKernelGGL(encrypt_k, dim3((1 << LOGN) / DCH, a->nl), dim3(DBX), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}

// ------------------------------------------------------------------------------------------------ subring switch
// pack_split / pack_dot (args.cuh:230-259; ks.cuh:909-963; host twin crates/pc-host/src/ks.rs:355-405): the split
// of c1 into sub coefficient classes (4 consecutive coefficients per thread, one 16-byte store per digit), and the dot
// of the digits against the pack key with the sum of the sub <= 16 products carried exactly.
constexpr int PBX = 256;

__global__ void __launch_bounds__(PBX) pack_split_k(PackSplitArgs A, int logn) {
    const int y = blockIdx.y, c = blockIdx.z;
    const uint32_t i = (blockIdx.x * PBX + threadIdx.x) * 4;
    const uint32_t* src = y < A.nq ? (const uint32_t*)A.q + c * A.q_stride + ((size_t)y << logn)
                                   : (const uint32_t*)A.p + c * A.p_stride + ((size_t)(y - A.nq) << logn);
    const uint4 v = *(const uint4*)(src + i);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t* o = (uint32_t*)A.out + c * A.out_stride + ((size_t)y << logn) + i;
    const size_t js = (size_t)A.nrows << logn;
    for (int j = 0; j < A.sub; ++j) {
        uint32_t r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = (int)((i + k) & (A.sub - 1)) == j ? w[k] : 0u;
        *(uint4*)(o + j * js) = make_uint4(r[0], r[1], r[2], r[3]);
    }
}

__global__ void __launch_bounds__(PBX) pack_dot_k(PackDotArgs A, int logn) {
    const int y = blockIdx.y, c = blockIdx.z;
    const uint32_t t = A.rows[y];
    const Red red(A.pr[t]);
    const uint32_t i = (blockIdx.x * PBX + threadIdx.x) * 4;
    const size_t koff = ((size_t)y << logn) + i, js = (size_t)A.nrows << logn;
    const uint32_t* dg = (const uint32_t*)A.dig + c * A.dig_stride + koff;
    uint64_t l0[4] = {0, 0, 0, 0}, l1[4] = {0, 0, 0, 0};
    uint32_t h0[4] = {0, 0, 0, 0}, h1[4] = {0, 0, 0, 0};
    for (int j = 0; j < A.sub; ++j) {
        const uint4 x = *(const uint4*)(dg + j * js);
        const uint4 b = *(const uint4*)((const uint32_t*)A.kb + koff + j * js);
        const uint4 a = *(const uint4*)((const uint32_t*)A.ka + koff + j * js);
        const uint32_t xv[4] = {x.x, x.y, x.z, x.w}, bv[4] = {b.x, b.y, b.z, b.w}, av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint64_t p0 = (uint64_t)xv[k] * bv[k], p1 = (uint64_t)xv[k] * av[k];
            l0[k] += p0;
            h0[k] += l0[k] < p0;
            l1[k] += p1;
            h1[k] += l1[k] < p1;
        }
    }
    const size_t roff = ((size_t)t << logn) + i;
    uint32_t r0[4], r1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        r0[k] = red.red96(l0[k], h0[k]);
        r1[k] = red.red96(l1[k], h1[k]);
    }
    if (y < A.nq) {
        const uint32_t pm = ((const uint32_t*)A.pmod)[t], pms = ((const uint32_t*)A.pmods)[t];
        const uint4 z = *(const uint4*)((const uint32_t*)A.c0 + c * A.ct_stride + roff);
        const uint32_t zv[4] = {z.x, z.y, z.z, z.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) r0[k] = addm(r0[k], shoup(zv[k], pm, pms, red.p), red.p);
    }
    *(uint4*)((uint32_t*)A.out0 + c * A.out_ct_stride + roff) = make_uint4(r0[0], r0[1], r0[2], r0[3]);
    *(uint4*)((uint32_t*)A.out1 + c * A.out_ct_stride + roff) = make_uint4(r1[0], r1[1], r1[2], r1[3]);
}

// the reference's checks (ks.cuh:949-963): sub a power of two in 2..16, 0 <= nq <= nrows, K >= 1
inline bool pack_ok(int sub, int nq, int nrows, int K) {
    return sub >= 2 && sub <= 16 && !(sub & (sub - 1)) && nq >= 0 && nq <= nrows && K >= 1;
}
template <int LOGN>
int pack_split(const PackSplitArgs* a, pc_stream_t s) {
    if (!a || !pack_ok(a->sub, a->nq, a->nrows, a->K)) return -1;
    if (!a->out || (a->nq > 0 && !a->q) || (a->nrows > a->nq && !a->p)) return -1;
    if (a->nrows == 0) return 0;
    hipLaunchKernelGGL(pack_split_k, dim3((1 << LOGN) / (PBX * 4), a->nrows, a->K), dim3(PBX), 0, (hipStream_t)s, *a,
                       LOGN);
    return launch_rc();
}
template <int LOGN>
int pack_dot(const PackDotArgs* a, pc_stream_t s) {
    if (!a || !pack_ok(a->sub, a->nq, a->nrows, a->K)) return -1;
    if (!a->dig || !a->kb || !a->ka || !a->out0 || !a->out1 || !a->rows || !a->pr) return -1;
    if (a->nq > 0 && (!a->c0 || !a->pmod || !a->pmods)) return -1;
    if (a->nrows == 0) return 0;
    hipLaunchKernelGGL(pack_dot_k, dim3((1 << LOGN) / (PBX * 4), a->nrows, a->K), dim3(PBX), 0, (hipStream_t)s, *a,
                       LOGN);
    return launch_rc();
}

// ------------------------------------------------------------------------------------------------ key generation
// b = e - a s_new + [id < nq and digit_of[id] == d] (P mod q_id) s_old' (s_old' = s_old^2 when sq), a from the KSKA
// expander; b dense or bit-packed (the little-endian value stream, the guard words past N bits / 32 zeroed).
__global__ void __launch_bounds__(DBX) kskgen_k(KskGenArgs A, int logn) {
    __shared__ uint32_t lv[DCH];
    const int m = blockIdx.y, d = blockIdx.z;
    const int id = A.ids[m];
    const PrimeConst& q = A.pr[id];
    const uint32_t p = (uint32_t)q.p;
    const Red red(q);
    const Expander ex(p);
    uint32_t seed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) seed[i] = A.seed[i];
    const uint32_t n = 1u << logn;
    const uint32_t chunk0 = blockIdx.x * DCH;
    const uint32_t s0 = chunk0 + threadIdx.x * DS;
    uint32_t a[DS], e[DS], sn[DS], r[DS];
    kska16(seed, s0, (uint32_t)d, ex, n >> 4, a);
    const size_t row = (size_t)d * A.nrows + m;
    ld16((const uint32_t*)A.e + (row << logn) + s0, e);
    ld16((const uint32_t*)A.s_new + ((size_t)id << logn) + s0, sn);
    const bool in_digit = id < A.nq && A.digit_of[id] == d;
    uint32_t so[DS];
    uint32_t pm = 0, pms = 0;
    if (in_digit) {
        ld16((const uint32_t*)A.s_old + ((size_t)id << logn) + s0, so);
        pm = ((const uint32_t*)A.pmod)[id];
        pms = ((const uint32_t*)A.pmods)[id];
    }
#pragma unroll
    for (int k = 0; k < DS; ++k) {
        uint32_t x = e[k];
        if (in_digit) {
            uint32_t tv = so[k];
            if (A.sq) tv = red.mul(tv, tv);
            x = addm(x, shoup(tv, pm, pms, p), p);
        }
        r[k] = subm(x, red.mul(a[k], sn[k]), p);
    }
    if (A.a) st16((uint32_t*)A.a + (row << logn) + s0, a);
    if (A.bits == 0) {
        st16((uint32_t*)A.b + (row << logn) + s0, r);
        return;
    }
#pragma unroll
    for (int k = 0; k < DS; ++k) lv[threadIdx.x * DS + k] = r[k];
    __syncthreads();
    const int bits = A.bits;
    const uint32_t mask = bits == 32 ? 0xFFFFFFFFu : (1u << bits) - 1u;
    const int nw = DCH / 32 * bits;
    uint32_t* out = (uint32_t*)A.b + row * A.row_words + chunk0 / 32 * (uint32_t)bits;
    for (int w = threadIdx.x; w < nw; w += DBX) {
        const uint32_t bit0 = (uint32_t)w * 32u;
        uint32_t k = bit0 / bits;
        const uint32_t o = bit0 - k * bits;
        uint64_t acc = (uint64_t)(lv[k] & mask) >> o;
        for (uint32_t filled = bits - o; filled < 32 && k + 1 < (uint32_t)DCH; filled += bits)
            acc |= (uint64_t)(lv[++k] & mask) << filled;
        out[w] = (uint32_t)acc;
    }
    if (blockIdx.x == gridDim.x - 1) {
        uint32_t* rowp = (uint32_t*)A.b + row * A.row_words;
        for (uint64_t g = (uint64_t)n * bits / 32 + threadIdx.x; g < A.row_words; g += DBX) rowp[g] = 0;
    }
}

template <int LOGN>
int ksk_gen(const KskGenArgs* a, pc_stream_t s) {
    if (!a || !a->b || !a->e || !a->s_new || !a->seed || !a->ids || !a->pr) return -1;
    if (a->bits < 0 || a->bits > 32 || a->nrows < 0 || a->ndig < 0) return -1;
    if (a->bits > 0 && (a->row_words < (uint64_t)(1 << LOGN) * a->bits / 32 + 1)) return -1;
    if (a->nrows == 0 || a->ndig == 0) return 0;
    if (!a->digit_of || !a->s_old || !a->pmod || !a->pmods) return -1;
    hipLaunchKernelGGL(kskgen_k, dim3((1 << LOGN) / DCH, a->nrows, a->ndig), dim3(DBX), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}

__global__ void unpack_k(KskUnpackArgs A, int logn) {
    const int r = blockIdx.y;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t* in = A.in + (size_t)r * A.row_words;
    const uint64_t bit = (uint64_t)i * A.bits;
    const uint32_t w = (uint32_t)(bit >> 5), off = (uint32_t)(bit & 31);
    const uint64_t v = ((uint64_t)in[w + 1] << 32 | in[w]) >> off;
    const uint32_t mask = A.bits == 32 ? 0xFFFFFFFFu : (1u << A.bits) - 1u;
    ((uint32_t*)A.out)[((size_t)r << logn) + i] = (uint32_t)v & mask;
}

template <int LOGN>
int ksk_unpack(const KskUnpackArgs* a, pc_stream_t s) {
    if (!a || !a->out || !a->in || a->bits < 1 || a->bits > 32 || a->nrows < 0) return -1;
    if (a->row_words < (uint64_t)(1 << LOGN) * a->bits / 32 + 1) return -1;
    if (a->nrows == 0) return 0;
    hipLaunchKernelGGL(unpack_k, dim3((1 << LOGN) / 256, a->nrows), dim3(256), 0, (hipStream_t)s, *a, LOGN);
    return launch_rc();
}

// ------------------------------------------------------------------------------------------------ tensor_seeded
// tensor_seeded (args.cuh:407-436; host twin crates/pc-host/src/elem.rs:345-404). The table's argument struct is
// 25 KiB, beyond a kernel's argument space, so the launcher runs it in chunks of TS_OUT outputs x TS_PAIRS pairs:
// each chunk reduces its sums exactly and the chunks after a group's first add onto its outputs (acc 3), which gives
// the words of one sum.
constexpr int TS_OUT = 4, TS_PAIRS = 32, TS_BX = 64;
constexpr uint32_t TAG_CTSA = 0x43545341u;  // "CTSA" (keys.rs:580-582)
constexpr int CTS_T_MAX = 32;               // attempts per word (keys.rs:585-587)
struct TsChunk {
    PolyRef out[TS_OUT], d2[TS_OUT];
    PolyRef b[TS_PAIRS];
    const uint32_t* a[TS_OUT][TS_PAIRS];
    const PrimeConst* pr;
    uint64_t seed_off;
    int nout, npairs, acc, packed;
};

// 16 consecutive c1 words (slots s0 .. s0 + 15, s0 a multiple of 16) of a regenerable ciphertext's row with prime p:
// ChaCha12 block s0 / 16 of (seed, w13 = 0, p, "CTSA"), a rejected word redrawn from block s0 / 16 + t N / 16
// (t < 32, the last draw kept), then mod p
__device__ __forceinline__ void cts16(const uint32_t (&seed)[8], uint32_t s0, const Expander& ex, uint32_t n16,
                                      uint32_t (&a)[16]) {
    const uint32_t ctr = s0 >> 4;
    uint32_t o[16];
    chacha12(seed, ctr, 0, ex.p, TAG_CTSA, o);
    uint32_t rej = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) rej |= (uint32_t)(o[j] >= ex.mp) << j;
    while (rej) {
        const int j = __builtin_ctz(rej);
        rej &= rej - 1;
        uint32_t v = 0;
        for (int t = 1; t < CTS_T_MAX; ++t) {
            v = chacha12_word(seed, ctr + (uint32_t)t * n16, 0, ex.p, TAG_CTSA, j);
            if (v < ex.mp) break;
        }
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) o[jj] = jj == j ? v : o[jj];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) a[j] = ex.red(o[j]);
}

// one thread: 16 slots (one ChaCha block) of one row, every output and pair of the chunk
__global__ void __launch_bounds__(TS_BX) tseed_k(TsChunk A, int logn) {
    const int row = blockIdx.y;
    const uint32_t s0 = (blockIdx.x * TS_BX + threadIdx.x) * 16;
    const uint32_t n = 1u << logn, n16 = n >> 4;
    const Red red(A.pr[row]);
    const Expander ex(red.p);
    const uint32_t p = red.p;
    const size_t roff = ((size_t)row << logn) + s0;
    const uint32_t roww = (n * PC_PACK_BITS + 31) / 32;
    for (int o = 0; o < A.nout; ++o) {
        uint32_t s0v[16], s1v[16], s2v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) s0v[k] = s1v[k] = s2v[k] = 0;
        for (int j = 0; j < A.npairs; ++j) {
            const uint32_t* base = A.a[o][j];
            uint32_t x0[16], x1[16], y0[16], y1[16];
            if (A.packed) {
                // 16 words of 28 bits = 14 words of the row's bit stream, word-aligned at slot s0
                const uint32_t* w = base + (size_t)row * roww + (s0 / 16) * 14;
                uint32_t u[15];
#pragma unroll
                for (int k = 0; k < 14; ++k) u[k] = w[k];
                u[14] = 0;
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const int bit = 28 * k, wi = bit >> 5, sh = bit & 31;
                    const uint64_t v = ((uint64_t)u[wi + 1] << 32) | u[wi];
                    x0[k] = (uint32_t)(v >> sh) & ((1u << PC_PACK_BITS) - 1u);
                }
            } else {
                ld16(base + roff, x0);
            }
            uint32_t seed[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) seed[k] = base[A.seed_off + 8 * (size_t)row + k];
            cts16(seed, s0, ex, n16, x1);
            const uint32_t* b0 = (const uint32_t*)A.b[j].base + roff;
            ld16(b0, y0);
            ld16(b0 + A.b[j].part_stride, y1);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                s0v[k] = red((uint64_t)s0v[k] + (uint64_t)x0[k] * y0[k]);
                s1v[k] = red((uint64_t)s1v[k] + (uint64_t)x0[k] * y1[k]);
                s1v[k] = red((uint64_t)s1v[k] + (uint64_t)x1[k] * y0[k]);
                s2v[k] = red((uint64_t)s2v[k] + (uint64_t)x1[k] * y1[k]);
            }
        }
        uint32_t* o0 = (uint32_t*)A.out[o].base + roff;
        uint32_t* o1 = o0 + A.out[o].part_stride;
        uint32_t* d2 = (uint32_t*)A.d2[o].base + A.d2[o].part_stride + roff;
        if (A.acc) {
            uint32_t v0[16], v1[16];
            ld16(o0, v0);
            ld16(o1, v1);
#pragma unroll
            for (int k = 0; k < 16; ++k) s0v[k] = addm(s0v[k], v0[k], p), s1v[k] = addm(s1v[k], v1[k], p);
        }
        if (A.acc & 2) {
            uint32_t v2[16];
            ld16(d2, v2);
#pragma unroll
            for (int k = 0; k < 16; ++k) s2v[k] = addm(s2v[k], v2[k], p);
        }
        st16(o0, s0v);
        st16(o1, s1v);
        st16(d2, s2v);
    }
}

template <int LOGN>
int tensor_seeded(const TensorSeededArgs* a, pc_stream_t s) {
    if (!a || !a->pr || a->nq < 1 || a->nq > PC_TSEED_Q || a->nout < 1 || a->nout > PC_TSEED_OUT || a->npairs < 1 ||
        a->npairs > PC_TSEED_PAIRS || a->nq * a->nout > PC_TSEED_QOUT || a->n < 0)
        return -1;
    for (int j = 0; j < a->npairs; ++j) {
        if (!a->b[j].base) return -1;
        for (int q = 1; q < a->nq; ++q)
            if (!a->bq[q - 1][j]) return -1;
        for (int o = 0; o < a->nout; ++o)
            if (!a->a[o][j]) return -1;
    }
    for (int m = 0; m < a->nq * a->nout; ++m)
        if (!a->out[m].base || !a->d2[m].base) return -1;
    if (a->n == 0) return 0;
    const dim3 grid((1u << LOGN) / 16 / TS_BX, a->n);
    for (int q = 0; q < a->nq; ++q)
        for (int o0 = 0; o0 < a->nout; o0 += TS_OUT)
            for (int j0 = 0; j0 < a->npairs; j0 += TS_PAIRS) {
                TsChunk c{};
                c.nout = std::min(TS_OUT, a->nout - o0);
                c.npairs = std::min(TS_PAIRS, a->npairs - j0);
                for (int k = 0; k < c.nout; ++k) {
                    c.out[k] = a->out[q * a->nout + o0 + k];
                    c.d2[k] = a->d2[q * a->nout + o0 + k];
                    for (int j = 0; j < c.npairs; ++j) c.a[k][j] = (const uint32_t*)a->a[o0 + k][j0 + j];
                }
                for (int j = 0; j < c.npairs; ++j) {
                    c.b[j] = a->b[j0 + j];
                    if (q > 0) c.b[j].base = const_cast<void*>(a->bq[q - 1][j0 + j]);
                }
                c.pr = a->pr;
                c.seed_off = a->seed_off;
                c.acc = j0 == 0 ? a->acc : 3;
                c.packed = a->packed;
                hipLaunchKernelGGL(tseed_k, grid, dim3(TS_BX), 0, (hipStream_t)s, c, LOGN);
                if (int rc = launch_rc()) return rc;
            }
    return 0;
}

}  // namespace ks

#define PCH_KS_INST(L)                                                                                        \
    int ks_dot_##L(const KsArgs* a, pc_stream_t s) { return ks::ks_dot<L>(a, s); }                          \
    int ks_dot_key_##L(const KsKeyArgs* a, pc_stream_t s) { return ks::ks_dot_key<L>(a, s); }                \
    int ksk_expand_##L(const KskExpandArgs* a, pc_stream_t s) { return ks::ksk_expand<L>(a, s); }            \
    int encrypt_##L(const EncryptArgs* a, pc_stream_t s) { return ks::encrypt<L>(a, s); }                     \
    int pack_split_##L(const PackSplitArgs* a, pc_stream_t s) { return ks::pack_split<L>(a, s); }            \
    int pack_dot_##L(const PackDotArgs* a, pc_stream_t s) { return ks::pack_dot<L>(a, s); }                  \
    int ksk_gen_##L(const KskGenArgs* a, pc_stream_t s) { return ks::ksk_gen<L>(a, s); }                     \
    int ksk_unpack_##L(const KskUnpackArgs* a, pc_stream_t s) { return ks::ksk_unpack<L>(a, s); }            \
    int tensor_seeded_##L(const TensorSeededArgs* a, pc_stream_t s) { return ks::tensor_seeded<L>(a, s); }
PCH_KS_INST(12)
PCH_KS_INST(13)
PCH_KS_INST(14)
PCH_KS_INST(15)
PCH_KS_INST(16)

int ks_dot_patched(int logn, const KsKeyArgs* g, const PatchTab* P, pc_stream_t s) {
    switch (logn) {
        case 12: return ks::dot_patched<12>(g, P, s);
        case 13: return ks::dot_patched<13>(g, P, s);
        case 14: return ks::dot_patched<14>(g, P, s);
        case 15: return ks::dot_patched<15>(g, P, s);
        case 16: return ks::dot_patched<16>(g, P, s);
        default: return -2;
    }
}
static int patch_launch(bool fill, int logn, const uint32_t* const* seeds, const PrimeConst* pr, int nkeys, int ndig,
                        int rows, uint32_t* counts, const uint32_t* idx, uint32_t* val, pc_stream_t s) {
    if (!seeds || !pr || nkeys < 1 || ndig < 1 || ndig > 4 || rows < 1 || logn < 10 || logn > 17) return -1;
    if (fill ? (!idx || !val) : !counts) return -1;
    const dim3 grid((1u << logn) / ks::DCH, rows, nkeys * ndig);
    if (fill) hipLaunchKernelGGL(ks::patch_k<true>, grid, dim3(ks::DBX), 0, (hipStream_t)s, seeds, pr, ndig, rows, logn,
                                 counts, idx, val);
    else hipLaunchKernelGGL(ks::patch_k<false>, grid, dim3(ks::DBX), 0, (hipStream_t)s, seeds, pr, ndig, rows, logn,
                            counts, idx, val);
    return launch_rc();
}
int kska_patch_count(int logn, const uint32_t* const* seeds, const PrimeConst* pr, int nkeys, int ndig, int rows,
                     uint32_t* counts, pc_stream_t s) {
    return patch_launch(false, logn, seeds, pr, nkeys, ndig, rows, counts, nullptr, nullptr, s);
}
int kska_patch_fill(int logn, const uint32_t* const* seeds, const PrimeConst* pr, int nkeys, int ndig, int rows,
                    const uint32_t* idx, uint32_t* val, pc_stream_t s) {
    return patch_launch(true, logn, seeds, pr, nkeys, ndig, rows, nullptr, idx, val, s);
}

}  // namespace pch
