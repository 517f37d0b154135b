// Key products gathered in output order, on gfx950: the fused CtS / StC stage core, the summed rotations of a key
// group, and the relinearisation dot with a regenerated key.
//   cts_fused / cts_fused_regen: hoisted baby-step rotations of a ModUp'd ciphertext times the BSGS plaintext
//     diagonals, summed per giant step in Q u P, the rotations never stored (crates/pc-kernels/kernels/cts.cuh;
//     args.cuh CtsArgs :325-355, CtsRegenArgs :748-758; host twin crates/pc-host/src/cts.rs);
//   ks_dot_key with KS_SUM: the R rotations of a key group summed into one output (ks.cuh ks_dot_seg /
//     ks_dot_key_sum; host twin crates/pc-host/src/ks.rs:226-265);
//   ks_dot_regen: one key, `a` regenerated from the args' seed, no automorphism, optionally through the fused ModDown
//     epilogue (ks.cuh:129-212; args.cuh KsRegenArgs :292-304, EpiArgs; host twin crates/pc-host/src/ks.rs:267-340).
//
// One wave per workgroup owns an aligned 512-slot chunk of output slots of one row t and one ciphertext, 8 slots per
// lane, and keeps its sums in registers across all keys (for the CtS stage: up to four giant steps, both parts), so a
// launch regenerates each key once for all its sums. The automorphism maps aligned chunks onto aligned chunks, so the
// sources of a rotation are one aligned 512-slot chunk too, and the wave works there in SOURCE order:
//   1. stage_a: the chunk's KSKA words, 32 ChaCha12 blocks per regenerated digit, one whole block per lane and item, go
//      to LDS (a rejected word is queued and redrawn by the wave, the accepted value written over it);
//   2. products: each lane forms C0 + sum_d D_d b_d and sum_d D_d a_d for its 8 consecutive source slots (32-byte
//      loads of D and b, `a` from LDS);
//   3. to_output: the two words per slot move to output order through LDS with a conflict-free scatter (below);
//   4. the kernel adds them into its sums (the CtS stage: times the diagonals' words at the lane's output slots).
#include "common.h"

namespace pch {
namespace cts {

constexpr int CW = 64;          // lanes per workgroup: one wave
constexpr int CS = 8;           // slots per lane
constexpr int CCH = CW * CS;    // the wave's chunk of slots
constexpr int NBLK = CCH / 16;  // ChaCha12 blocks per digit and chunk
constexpr int DMAX = 6;         // digits a stage reads at u32 words (cts.cuh:18-22)
constexpr int GW = 4;           // CtS giant steps per pass: 2 parts x GW x 8 sums per lane
constexpr int QCAP = 512;       // queued rejected words (a lane whose word does not fit redraws it itself)
constexpr int APAD = CCH + CCH / 4;  // one digit's words in LDS: 4 padding words after every 16 (80-byte blocks)

// LDS of one wave (dynamic: nreg digits of `a`, at least the two scatter buffers' 1024 words, then the queue)
__host__ __device__ constexpr int a_words(int nreg) { return nreg * APAD > 2 * CCH ? nreg * APAD : 2 * CCH; }
__host__ __device__ constexpr int lds_bytes(int nreg) { return 4 * (a_words(nreg) + QCAP + 1); }
__device__ __forceinline__ uint32_t apad(uint32_t s) { return s + (s >> 4) * 4; }

// k^-1 mod 2^32 for odd k: Newton's step x (2 - k x) doubles the correct low bits, and k k = 1 mod 8 starts at three.
__device__ __forceinline__ uint32_t inv_odd(uint32_t k) {
    uint32_t x = k;
#pragma unroll
    for (int i = 0; i < 4; ++i) x *= 2u - k * x;
    return x;
}

// the key slot of prime id t (KskShape::slot_of): Q primes at their id, special prime nq + j at q_top + 1 + j
__device__ __forceinline__ int slot_of(const KeyTab& T, int t, int nq) {
    return (t < nq || T.q_top < 0) ? t : T.q_top + 1 + (t - nq);
}

// Scatter inside a 512-slot chunk. For source slot s0 + k (s0 = chunk + 8 lane) and W = the top 9 bits of
// V = ((2 brev(s) + 1) k) mod 2N (k the scatter exponent), the output's offset in its chunk is brev9(W), and
// W = C + k (64 brev3(j) + brev6(lane)) mod 512 is affine in the lane. Storing at rotr1(W) (a 9-bit rotate right) puts
// the 32 lanes of each half wave on 32 distinct banks, for the writes of one word and for the reads of output offsets
// 8 lane + j, which sit at rotr1(brev6(lane)) + 32 brev3(j).
__device__ __forceinline__ uint32_t scat9(uint32_t w) { return (w >> 1) | ((w & 1) << 8); }
__device__ __forceinline__ uint32_t brev3(uint32_t j) { return __brev(j) >> 29; }

__device__ __forceinline__ void ld8(const uint32_t* p, uint32_t (&v)[CS]) {
    const uint4 a = ((const uint4*)p)[0], b = ((const uint4*)p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
__device__ __forceinline__ void ld8(gptr p, uint32_t (&v)[CS]) {
    const __attribute__((address_space(1))) gu4* q = (const __attribute__((address_space(1))) gu4*)p;
    const gu4 a = q[0], b = q[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
// a stream read once per launch (a key's b row, a diagonal): non-temporal, so that it does not push the rows read
// again out of L2 (the ModUp digits, which every baby of the chunk's row reads at another source chunk)
__device__ __forceinline__ void ld8_once(gptr p, uint32_t (&v)[CS]) {
    const __attribute__((address_space(1))) gu4* q = (const __attribute__((address_space(1))) gu4*)p;
    const gu4 a = __builtin_nontemporal_load(q), b = __builtin_nontemporal_load(q + 1);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
__device__ __forceinline__ void st8(uint32_t* p, const uint32_t (&v)[CS]) {
    ((uint4*)p)[0] = make_uint4(v[0], v[1], v[2], v[3]);
    ((uint4*)p)[1] = make_uint4(v[4], v[5], v[6], v[7]);
}

// The 8 values of a bit-packed row of `words` words from value s0 on (bits per value; the row ends in a guard word):
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

// w's Shoup companion floor(w 2^32 / p) for w < p, from m = floor(2^64 / p) = mhi 2^32 + mlo: (w m) >> 32 =
// w mhi + umulhi(w, mlo) is exact or one low, and w 2^32 - ws p (in [0, 2p), so its low word) tells which
__device__ __forceinline__ uint32_t shoup_of(uint32_t w, uint32_t p, uint32_t mhi, uint32_t mlo) {
    const uint32_t ws = w * mhi + __umulhi(w, mlo);
    return (0u - ws * p) >= p ? ws + 1 : ws;
}

// the accepted attempt t = 1..15 of a rejected word (block ctr + t N/16; the 16th attempt kept as is), reduced
__device__ __forceinline__ uint32_t redraw(const uint32_t (&seed)[8], uint32_t ctr, uint32_t d, const Expander& ex,
                                           uint32_t n16, int w) {
    uint32_t v = 0;
    for (int tt = 1; tt < KSK_T_MAX; ++tt) {
        v = chacha12_word(seed, ctr + (uint32_t)tt * n16, d, ex.p, TAG_KSKA, w);
        if (v < ex.mp) break;
    }
    return ex.red(v);
}

// What the steps need of one (row t, ciphertext): the prime's arithmetic, the ModUp digits' row t (D_d = c1 on the
// rows of digit d), the c0 term (0 none, 1 P c0, 2 c0 as is) and the wave's LDS.
struct Row {
    uint32_t p;
    Red red;
    Expander ex;
    uint32_t n16, mask2n;
    int logn, ndig, nreg, dt, c0m;
    const uint32_t *c0, *c1, *mu;  // row t of c0, c1 and ModUp digit 0
    uint64_t mds;                  // digit stride of the ModUp output
    uint32_t pm, pms;              // P mod q_t and its Shoup companion (c0m 1)
    uint32_t *la, *lq, *lqn;       // LDS: [nreg][APAD] of `a` (then the scatter buffers), the queue, its count
    __device__ __forceinline__ const uint32_t* drow(int d) const { return d == dt ? c1 : mu + d * mds; }
};

// A key's rows at row t: b of digit d at kb + d bstride (dense: plus the slot; packed: bits per value, rows of bwords
// words), resident a of digit d >= nreg at ka + d astride, the seed of the regenerated digits.
struct KeyRow {
    gptr kb;
    uint64_t bstride, bwords;
    int bits;
    gptr ka;
    uint64_t astride;
    const uint32_t* seed;  // read with scalar loads (uniform, read-only)
};

__device__ __forceinline__ Row make_row(const PrimeConst& q, int logn, uint32_t* lds, int nreg) {
    Row R{(uint32_t)q.p, Red(q), Expander((uint32_t)q.p)};
    R.n16 = (1u << logn) >> 4;
    R.mask2n = (2u << logn) - 1;
    R.logn = logn;
    R.nreg = nreg;
    R.la = lds;
    R.lq = lds + a_words(nreg);
    R.lqn = R.lq + QCAP;
    return R;
}

// 1. The KSKA words of digits d < nreg at the source chunk [sc, sc + 512) into la[d][apad(s - sc)].
__device__ __forceinline__ void stage_a(const Row& R, const uint32_t* sp, uint32_t sc, int lane) {
    uint32_t seed[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) seed[k] = sload(sp + k);
    if (lane == 0) *R.lqn = 0;
    wave_sync();
    // item = digit d, block b (slots sc + 16 b ..), one per lane and round
    for (int it = lane; it < R.nreg * NBLK; it += CW) {
        const uint32_t d = (uint32_t)it / NBLK, b = (uint32_t)it % NBLK;
        uint32_t o[16];
        chacha12(seed, (sc >> 4) + b, d, R.p, TAG_KSKA, o);
        uint32_t rej = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) rej |= (uint32_t)(o[j] >= R.ex.mp) << j;
#pragma unroll
        for (int j = 0; j < 16; ++j) o[j] = R.ex.red(o[j]);
        if (rej) {
            uint32_t m = rej, qi = atomicAdd(R.lqn, (uint32_t)__builtin_popcount(rej));
            while (m) {
                const int j = __builtin_ctz(m);
                m &= m - 1;
                if (qi < (uint32_t)QCAP) {
                    R.lq[qi] = d << 16 | (16 * b + j);
                } else {
                    // the queue is full: this lane redraws the word itself
                    const uint32_t v = redraw(seed, (sc >> 4) + b, d, R.ex, R.n16, j);
#pragma unroll
                    for (int jj = 0; jj < 16; ++jj) o[jj] = jj == j ? v : o[jj];
                }
                ++qi;
            }
        }
        uint4* dst = (uint4*)(R.la + d * APAD + 20 * b);
#pragma unroll
        for (int m = 0; m < 4; ++m) dst[m] = make_uint4(o[4 * m], o[4 * m + 1], o[4 * m + 2], o[4 * m + 3]);
    }
    wave_sync();
    const uint32_t nq = min(*R.lqn, (uint32_t)QCAP);
    for (uint32_t k = lane; k < nq; k += CW) {
        const uint32_t e = R.lq[k], d = e >> 16, sl = e & 0xFFFF;
        R.la[d * APAD + apad(sl)] = redraw(seed, (sc + sl) >> 4, d, R.ex, R.n16, (int)(sl & 15));
    }
    wave_sync();
}

// 2. v0 = C0 + sum_d D_d b_d and v1 = sum_d D_d a_d at source slots s0 .. s0 + 7 (s0 - chunk = 8 lane), canonical.
// WIDE: more than 4 digits (the 64-bit sums reduced every 3 digits).
template <bool WIDE>
__device__ __forceinline__ void products(const Row& R, const KeyRow& K, uint32_t s0, int lane, uint32_t (&v0)[CS],
                                         uint32_t (&v1)[CS]) {
    const uint32_t p = R.p;
    uint64_t z0[CS], z1[CS];
    uint32_t q0[WIDE ? CS : 1], q1[WIDE ? CS : 1];
#pragma unroll
    for (int k = 0; k < CS; ++k) z0[k] = z1[k] = 0;
#pragma unroll
    for (int k = 0; k < (WIDE ? CS : 1); ++k) q0[k] = q1[k] = 0;
    for (int d = 0; d < R.ndig; ++d) {
        uint32_t a[CS], b[CS], x[CS];
        if (d < R.nreg) {
            const uint4* src = (const uint4*)(R.la + d * APAD + apad(lane * CS));
            const uint4 u = src[0], v = src[1];
            a[0] = u.x, a[1] = u.y, a[2] = u.z, a[3] = u.w, a[4] = v.x, a[5] = v.y, a[6] = v.z, a[7] = v.w;
        } else {
            ld8(K.ka + d * K.astride + s0, a);
        }
        if (K.bits == 0) ld8_once(K.kb + d * K.bstride + s0, b);
        else ld_packed((const uint32_t*)(K.kb + d * K.bstride), K.bwords, s0, K.bits, b);
        ld8(R.drow(d) + s0, x);
#pragma unroll
        for (int k = 0; k < CS; ++k) {
            z0[k] += (uint64_t)x[k] * b[k];
            z1[k] += (uint64_t)x[k] * a[k];
        }
        if (WIDE && d % 3 == 2 && d + 1 < R.ndig) {
#pragma unroll
            for (int k = 0; k < CS; ++k) {
                q0[k] = addm(q0[k], R.red(z0[k]), p);
                q1[k] = addm(q1[k], R.red(z1[k]), p);
                z0[k] = z1[k] = 0;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < CS; ++k) {
        // WIDE: <= 3 products per sum; else <= 4 products of (p - 1)^2 < 2^64
        v0[k] = WIDE ? addm(q0[k], R.red(z0[k]), p) : R.red(z0[k]);
        v1[k] = WIDE ? addm(q1[k], R.red(z1[k]), p) : R.red(z1[k]);
    }
    if (R.c0m) {
        uint32_t cz[CS];
        ld8(R.c0 + s0, cz);
#pragma unroll
        for (int k = 0; k < CS; ++k) v0[k] = addm(v0[k], R.c0m == 1 ? shoup(cz[k], R.pm, R.pms, p) : cz[k], p);
    }
}

// 3. Source slot s0 + k to output automorph_slot(kx, s0 + k) of the output chunk, read back at the lane's 8 output
// slots (8 lane + j of the chunk).
__device__ __forceinline__ void to_output(const Row& R, uint32_t kx, uint32_t s0, int lane, const uint32_t (&v0)[CS],
                                          const uint32_t (&v1)[CS], uint32_t (&w0)[CS], uint32_t (&w1)[CS]) {
    uint32_t* l0 = R.la;
    uint32_t* l1 = R.la + CCH;
    const int sh = R.logn - 8;
    const uint32_t cbh = (((2 * brev_n(s0, R.logn) + 1) * kx) & R.mask2n) >> sh;
    const uint32_t sth = ((kx << (R.logn - 2)) & R.mask2n) >> sh;
    wave_sync();  // every lane has read its `a` words
#pragma unroll
    for (int k = 0; k < CS; ++k) {
        const uint32_t o = scat9((cbh + brev3(k) * sth) & (CCH - 1));
        l0[o] = v0[k];
        l1[o] = v1[k];
    }
    wave_sync();
    const uint32_t rb = scat9(__brev((uint32_t)lane) >> 26);
#pragma unroll
    for (int j = 0; j < CS; ++j) {
        w0[j] = l0[rb + 32 * brev3(j)];
        w1[j] = l1[rb + 32 * brev3(j)];
    }
    wave_sync();  // before the next key's blocks overwrite the buffers
}

// One rotation's words at the lane's output slots: the key switch of source chunk sc (gather exponent g) scattered by
// kx = g^-1 to output chunk oc0.
template <bool WIDE>
__device__ __forceinline__ void rotation(const Row& R, const KeyRow& K, uint32_t g, uint32_t kx, uint32_t oc0,
                                         int lane, uint32_t (&w0)[CS], uint32_t (&w1)[CS]) {
    const uint32_t sc = automorph_slot(g, oc0, R.logn) & ~(uint32_t)(CCH - 1);
    if (R.nreg > 0) stage_a(R, K.seed, sc, lane);
    uint32_t v0[CS], v1[CS];
    products<WIDE>(R, K, sc + lane * CS, lane, v0, v1);
    to_output(R, kx, sc + lane * CS, lane, v0, v1, w0, w1);
}

// The block's (chunk, row index) in an XCD-aware order: each XCD takes a contiguous range of the row-major
// (row, chunk) blocks, so that a row's chunks run on one XCD. A rotation's sources are the automorphism's image of the
// output chunk, spread over the whole row: kept on one XCD, a row's digit and key words are fetched into that XCD's
// L2 once instead of once per XCD. (The summed rotations' kernel keeps the plain order: there the K ciphertexts of a
// launch share each key row, and the plain order measured faster.)
__device__ __forceinline__ uint2 chunk_row() {
    const uint32_t l = xcd_block(blockIdx.y * gridDim.x + blockIdx.x, gridDim.x * gridDim.y);
    return make_uint2(l % gridDim.x, l / gridDim.x);
}

// ------------------------------------------------------------------------------------------------ CtS stage
// grid (N / 512 chunks, rows, K ciphertexts); giant steps j0 .. j0 + 3 of the launch. REGEN: keys through the KeyTab
// (a regenerated for digits < nregen).
template <bool REGEN, bool WIDE>
__global__ void __launch_bounds__(CW, 3) cts_k(CtsRegenArgs RA, int logn, int j0) {
    extern __shared__ uint32_t lds[];
    const CtsArgs& A = RA.cts;
    const KeyTab& T = RA.key;
    const int lane = threadIdx.x, c = blockIdx.z;
    const uint2 cr = chunk_row();
    const int t = (int)A.rows[cr.y];
    const PrimeConst& q = A.pr[t];
    const bool isq = t < A.nq;
    Row R = make_row(q, logn, lds, REGEN ? min(A.ndig, T.nregen) : 0);
    const uint32_t p = R.p;
    const uint32_t mhi = (uint32_t)(q.mu_lo >> 32), mlo = (uint32_t)q.mu_lo;  // floor(2^64 / p)
    const size_t roff = (size_t)t << logn;
    R.ndig = A.ndig;
    R.dt = isq ? A.digit_of[t] : -1;
    R.c0m = isq ? 1 : 0;
    R.c0 = (const uint32_t*)A.x + c * A.ct_stride + roff;
    R.c1 = R.c0 + A.part_stride;
    R.mu = (const uint32_t*)A.modup + c * A.mu_ct_stride + roff;
    R.mds = A.mu_digit_stride;
    R.pm = isq ? ((const uint32_t*)A.pmod)[t] : 0;
    R.pms = isq ? ((const uint32_t*)A.pmods)[t] : 0;
    const int prow = isq ? t : A.pt_prow + (t - A.nq);
    const int slot = REGEN ? slot_of(T, t, A.nq) : t;
    const uint32_t oc0 = cr.x * CCH;
    const uint32_t o0 = oc0 + lane * CS;  // the lane's output slots o0 .. o0 + 7
    const int gn = min(GW, A.G - j0);
    const bool pt8 = A.enc == 0xFFFFFFFFu && (A.ptw & 3) == 0;
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
                ld8(x0, w0);
                ld8(x0 + A.part_stride, w1);
            } else if (isq) {
                ld8(R.c0 + o0, w0);
                ld8(R.c1 + o0, w1);
#pragma unroll
                for (int k = 0; k < CS; ++k) {
                    w0[k] = shoup(w0[k], R.pm, R.pms, p);
                    w1[k] = shoup(w1[k], R.pm, R.pms, p);
                }
            } else {
#pragma unroll
                for (int k = 0; k < CS; ++k) w0[k] = w1[k] = 0;
            }
        } else {
            // baby i: sources s = automorph_slot(g, o) of the chunk's outputs, scattered back by g^-1
            const uint32_t g = sload(A.kinv + (i - 1));
            KeyRow K;
            if (REGEN) {
                K.kb = as_global(sload(T.kb + (i - 1))) + (size_t)slot * T.row_words;
                K.bstride = (uint64_t)T.srows * T.row_words;
                K.bwords = T.row_words;
                K.bits = T.bits;
                K.seed = R.nreg > 0 ? sload(T.seed + (i - 1)) : nullptr;
            } else {
                K.kb = as_global(sload(A.kb + (i - 1))) + roff;
                K.bstride = A.key_digit_stride;
                K.bwords = 0;
                K.bits = 0;
                K.seed = nullptr;  // no regenerated digit: never read
            }
            K.ka = R.nreg < A.ndig ? as_global(sload(A.ka + (i - 1))) + roff : K.kb;  // (K.kb: never read)
            K.astride = A.key_digit_stride;
            rotation<WIDE>(R, K, g, inv_odd(g) & R.mask2n, oc0, lane, w0, w1);
        }
        // 4. the giant steps' sums: acc_j += rot_i pt_{B j + i} at the lane's outputs
#pragma unroll
        for (int jj = 0; jj < GW; ++jj) {
            if (jj >= gn) break;
            const int dg = A.B * (j0 + jj) + i;
            if (dg >= A.npts) continue;
            const uint32_t* pt = (const uint32_t*)A.pts[dg] + (size_t)prow * A.ptw;
            uint32_t w[CS];
            if (pt8 && ((uintptr_t)pt & 15) == 0) {
                ld8_once(as_global(pt) + o0, w);
            } else {
                const Buf bp(pt, (uint32_t)A.ptw * 4);
#pragma unroll
                for (int k = 0; k < CS; ++k) w[k] = bp.ld(ptidx(o0 + k, A.enc) * 4, 0);
            }
            // Shoup products by the diagonal's word (its companion made once for both parts), added mod p: the sums
            // stay single words
#pragma unroll
            for (int k = 0; k < CS; ++k) {
                const uint32_t ws = shoup_of(w[k], p, mhi, mlo);
                acc0[jj][k] = addm(acc0[jj][k], shoup(w0[k], w[k], ws, p), p);
                acc1[jj][k] = addm(acc1[jj][k], shoup(w1[k], w[k], ws, p), p);
            }
        }
    }
#pragma unroll
    for (int jj = 0; jj < GW; ++jj) {
        if (jj >= gn) break;
        const int j = j0 + jj;
        const size_t at = A.pair_cts > 0 ? (size_t)(j >> 1) * A.pair_cts + (j & 1) : (size_t)c * A.G + j;
        uint32_t* r = (uint32_t*)A.res + at * A.ct_stride + roff + o0;
        st8(r, acc0[jj]);
        st8(r + A.part_stride, acc1[jj]);
    }
}

// The checks of the reference's launchers (cts.cuh:480-524: giant steps above 2, or above 4 in the K = 1 regen form
// with pair_cts; more than 6 digits; pair_cts outside that form; more than 64 baby steps in the regen form; x0 in the
// four-giant-step form or with ciphertext groups off the regen form: -1), then this kernel's own range: row strides
// of whole 16-byte groups (-2), and diagonals' compact indices inside ptw words (-1).
template <int LOGN, bool REGEN>
int launch(const CtsRegenArgs& R, pc_stream_t s) {
    static_assert((1 << LOGN) >= CCH, "ring of at least 512 slots");
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
    const int nreg = REGEN ? std::max(0, std::min(a.ndig, R.key.nregen)) : 0;
    const dim3 grid(n / CCH, a.nrows, a.K);
    const size_t lb = lds_bytes(nreg);
    hipStream_t st = (hipStream_t)s;
    for (int j0 = 0; j0 < a.G; j0 += GW) {
        if (a.ndig > 4) hipLaunchKernelGGL((cts_k<REGEN, true>), grid, dim3(CW), lb, st, R, LOGN, j0);
        else hipLaunchKernelGGL((cts_k<REGEN, false>), grid, dim3(CW), lb, st, R, LOGN, j0);
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

// ------------------------------------------------------------------------------------------------ KS_SUM
// ks_dot_key with KS_SUM: out[c] (rotation 0's output) = sum_r sigma_r(dot_r) (+ out with KS_ACC), each rotation's c0
// term applied before its automorphism (crates/pc-host/src/ks.rs:226-265). grid (N / 512 chunks, rows, K).
template <bool WIDE>
__global__ void __launch_bounds__(CW, 3) ksum_k(KsKeyArgs G, int logn) {
    extern __shared__ uint32_t lds[];
    const KsArgs& A = G.ks;
    const KeyTab& T = G.key;
    const int lane = threadIdx.x, c = blockIdx.z;
    const int t = (int)A.rows[blockIdx.y];
    const bool isq = t < A.nq;
    Row R = make_row(A.pr[t], logn, lds, max(0, min(A.ndig, T.nregen)));
    const uint32_t p = R.p;
    const size_t roff = (size_t)t << logn;
    const int m0 = A.c0_mode & 3;
    R.ndig = A.ndig;
    R.dt = isq ? A.digit_of[t] : -1;
    R.c0m = m0 == 1 ? (isq ? 1 : 0) : m0 == 2 ? 2 : 0;
    R.c1 = (const uint32_t*)A.c1 + c * A.ct_stride + roff;
    R.c0 = R.c0m ? (const uint32_t*)A.c0 + c * A.ct_stride + roff : R.c1;  // (R.c1: never read)
    R.mu = (const uint32_t*)A.modup + c * A.mu_ct_stride + roff;
    R.mds = A.mu_digit_stride;
    R.pm = R.c0m == 1 ? ((const uint32_t*)A.pmod)[t] : 0;
    R.pms = R.c0m == 1 ? ((const uint32_t*)A.pmods)[t] : 0;
    const int slot = slot_of(T, t, A.nq);
    const uint32_t oc0 = blockIdx.x * CCH;
    const uint32_t o0 = oc0 + lane * CS;
    uint32_t acc0[CS], acc1[CS];
#pragma unroll
    for (int k = 0; k < CS; ++k) acc0[k] = acc1[k] = 0;
    for (int r = 0; r < A.R; ++r) {
        KeyRow K;
        K.kb = as_global(sload(T.kb + r)) + (size_t)slot * T.row_words;
        K.bstride = (uint64_t)T.srows * T.row_words;
        K.bwords = T.row_words;
        K.bits = T.bits;
        K.seed = R.nreg > 0 ? sload(T.seed + r) : nullptr;
        K.ka = R.nreg < A.ndig ? as_global(sload(A.ka + r)) + roff : K.kb;  // (K.kb: never read)
        K.astride = A.key_digit_stride;
        const uint32_t kx = sload(A.autok + r) & R.mask2n;  // the scatter exponent; its inverse gathers
        uint32_t w0[CS], w1[CS];
        rotation<WIDE>(R, K, inv_odd(kx) & R.mask2n, kx, oc0, lane, w0, w1);
#pragma unroll
        for (int k = 0; k < CS; ++k) {
            acc0[k] = addm(acc0[k], w0[k], p);
            acc1[k] = addm(acc1[k], w1[k], p);
        }
    }
    uint32_t* out0 = (uint32_t*)A.out0 + c * A.out_ct_stride + roff + o0;
    uint32_t* out1 = (uint32_t*)A.out1 + c * A.out_ct_stride + roff + o0;
    if (A.c0_mode & PC_KS_ACC) {
        uint32_t e0[CS], e1[CS];
        ld8(out0, e0);
        ld8(out1, e1);
#pragma unroll
        for (int k = 0; k < CS; ++k) {
            acc0[k] = addm(acc0[k], e0[k], p);
            acc1[k] = addm(acc1[k], e1[k], p);
        }
    }
    st8(out0, acc0);
    st8(out1, acc1);
}

// ------------------------------------------------------------------------------------------------ ks_dot_regen
// One key (b from key 0 of the KeyTab when key.kb is set, else the dense prime-id rows of ks.kb[0]; `a` regenerated
// from the args' seed for every digit), K <= 4 ciphertexts, no automorphism, no c0 term; out0 / out1, or through the
// fused epilogue: dst = f (alpha dst + (dot - conv) binv) [+ k on part 0] [+ add]. grid (N / 512 chunks, rows).
template <bool WIDE, bool EPI>
__global__ void __launch_bounds__(CW, 3) regen_k(KsRegenArgs G, int logn) {
    extern __shared__ uint32_t lds[];
    const KsArgs& A = G.ks;
    const KeyTab& T = G.key;
    const EpiArgs& E = G.epi;
    const int lane = threadIdx.x;
    const int t = (int)A.rows[blockIdx.y];
    Row R = make_row(A.pr[t], logn, lds, A.ndig);
    const uint32_t p = R.p;
    const size_t roff = (size_t)t << logn;
    R.ndig = A.ndig;
    R.dt = t < A.nq ? A.digit_of[t] : -1;
    R.c0m = 0;
    R.c0 = (const uint32_t*)A.c1;  // no c0 term: never read
    R.mds = A.mu_digit_stride;
    R.pm = R.pms = 0;
    KeyRow K;
    if (T.kb) {
        K.kb = as_global(T.kb[0]) + (size_t)slot_of(T, t, A.nq) * T.row_words;
        K.bstride = (uint64_t)T.srows * T.row_words;
        K.bwords = T.row_words;
        K.bits = T.bits;
    } else {
        K.kb = as_global(A.kb[0]) + roff;
        K.bstride = A.key_digit_stride;
        K.bwords = 0;
        K.bits = 0;
    }
    K.ka = K.kb;  // every digit regenerates: never read
    K.astride = 0;
    K.seed = G.seed;
    const uint32_t s0 = blockIdx.x * CCH + lane * CS;  // no automorphism: source and output slots coincide
    if (R.nreg > 0) stage_a(R, G.seed, blockIdx.x * CCH, lane);
    for (int c = 0; c < A.K; ++c) {
        R.c1 = (const uint32_t*)A.c1 + c * A.ct_stride + roff;
        R.mu = (const uint32_t*)A.modup + c * A.mu_ct_stride + roff;
        uint32_t v0[CS], v1[CS];
        products<WIDE>(R, K, s0, lane, v0, v1);
        const size_t ob = c * A.out_ct_stride + roff + s0;
        if (!EPI) {
            st8((uint32_t*)A.out0 + ob, v0);
            st8((uint32_t*)A.out1 + ob, v1);
            continue;
        }
        const uint32_t bi = ((const uint32_t*)E.binv)[t], bis = ((const uint32_t*)E.binvs)[t];
        uint32_t kk = E.k ? ((const uint32_t*)E.k)[t] : 0;
        kk = kk >= p ? kk - p : kk;
        // alpha = 1 when absent: its Shoup companion floor(2^32 / p) makes the product exact
        const uint32_t ai = E.alpha ? ((const uint32_t*)E.alpha)[t] : 1u;
        const uint32_t ais = E.alpha ? ((const uint32_t*)E.alphas)[t] : (uint32_t)((1ull << 32) / p);
        const uint32_t fm = E.dbl ? 2u : 1u;  // the doubling as one more addition of r
        for (int part = 0; part < 2; ++part) {
            const size_t off = ob + part * E.part_stride;
            uint32_t* dp = (uint32_t*)E.dst + off;
            uint32_t cv[CS], dv[CS], av[CS];
            ld8((const uint32_t*)E.conv + off, cv);
            ld8(dp, dv);
#pragma unroll
            for (int k = 0; k < CS; ++k) av[k] = 0;
            if (G.add) ld8((const uint32_t*)G.add + off, av);
            const uint32_t kp = part == 0 ? kk : 0u;
#pragma unroll
            for (int k = 0; k < CS; ++k) {
                const uint32_t x = part ? v1[k] : v0[k];
                uint32_t r = addm(shoup(dv[k], ai, ais, p), shoup(subm(x, cv[k], p), bi, bis, p), p);
                r = addm(r, fm == 2u ? r : 0u, p);
                dv[k] = addm(addm(r, kp, p), av[k], p);
            }
            st8(dp, dv);
        }
    }
}

// ks_dot_regen (crates/pc-host/src/ks.rs:267-280: a packed width outside 0..=32 -1, `add` without the epilogue -1,
// K > 4 -2), then this kernel's range: more than 6 digits -1, row strides of whole 16-byte groups (-2).
template <int LOGN>
int ks_dot_regen(const KsRegenArgs* g, pc_stream_t s) {
    static_assert((1 << LOGN) >= CCH, "ring of at least 512 slots");
    if (!g) return -1;
    const KsArgs& a = g->ks;
    if (g->key.kb && (g->key.bits < 0 || g->key.bits > 32)) return -1;
    if (g->add && !g->use_epi) return -1;
    if (a.K > 4) return -2;
    if (a.nrows < 0 || a.K < 0 || a.ndig < 0 || a.ndig > DMAX) return -1;
    if (a.nrows == 0 || a.K == 0) return 0;
    if (!a.rows || !a.pr || !a.c1 || !a.digit_of || !g->seed) return -1;
    if (a.ndig > 0 && (!a.modup || (!g->key.kb && !a.kb))) return -1;
    if (g->use_epi) {
        if (!g->epi.dst || !g->epi.conv || !g->epi.binv || !g->epi.binvs) return -1;
        if (g->epi.alpha && !g->epi.alphas) return -1;
        if (g->epi.part_stride & 3) return -2;
    } else if (!a.out0 || !a.out1) {
        return -1;
    }
    if ((a.ct_stride | a.mu_ct_stride | a.mu_digit_stride | a.out_ct_stride | a.key_digit_stride) & 3) return -2;
    if (g->key.kb && g->key.bits == 0 && (g->key.row_words & 3)) return -2;
    const dim3 grid((1u << LOGN) / CCH, a.nrows);
    const size_t lb = lds_bytes(a.ndig);
    hipStream_t st = (hipStream_t)s;
    const bool wide = a.ndig > 4;
    if (g->use_epi) {
        if (wide) hipLaunchKernelGGL((regen_k<true, true>), grid, dim3(CW), lb, st, *g, LOGN);
        else hipLaunchKernelGGL((regen_k<false, true>), grid, dim3(CW), lb, st, *g, LOGN);
    } else {
        if (wide) hipLaunchKernelGGL((regen_k<true, false>), grid, dim3(CW), lb, st, *g, LOGN);
        else hipLaunchKernelGGL((regen_k<false, false>), grid, dim3(CW), lb, st, *g, LOGN);
    }
    return launch_rc();
}

}  // namespace cts

// The summed rotations of ks_dot_key (KS_SUM), its argument checks done by the caller except this kernel's range:
// more than 6 digits -1, row strides of whole 16-byte groups -2.
int ks_dot_key_sum(int logn, const KsKeyArgs* g, pc_stream_t s) {
    using namespace cts;
    const KsArgs& a = g->ks;
    if (a.nrows < 0 || a.R < 0 || a.K < 0 || a.ndig < 0 || a.ndig > DMAX) return -1;
    if (a.nrows == 0 || a.K == 0) return 0;
    if (!a.rows || !a.pr || !a.c1 || !a.out0 || !a.out1 || !a.digit_of || (a.R > 0 && !a.autok)) return -1;
    if (a.ndig > 0 && !a.modup) return -1;
    if ((a.c0_mode & 3) == 1 && (!a.c0 || !a.pmod || !a.pmods)) return -1;
    if ((a.c0_mode & 3) == 2 && !a.c0) return -1;
    if ((a.c0_mode & 3) == 3) return -1;
    if (a.R > 0 && (!g->key.kb || (g->key.nregen > 0 && !g->key.seed))) return -1;
    if (a.R > 0 && a.ndig > g->key.nregen && !a.ka) return -1;
    if ((a.ct_stride | a.mu_ct_stride | a.mu_digit_stride | a.out_ct_stride | a.key_digit_stride) & 3) return -2;
    if (g->key.bits == 0 && (g->key.row_words & 3)) return -2;
    if (logn < 12 || logn > 16) return -2;
    const int nreg = std::max(0, std::min(a.ndig, g->key.nregen));
    const dim3 grid((1u << logn) / CCH, a.nrows, a.K);
    hipStream_t st = (hipStream_t)s;
    if (a.ndig > 4) hipLaunchKernelGGL(ksum_k<true>, grid, dim3(CW), lds_bytes(nreg), st, *g, logn);
    else hipLaunchKernelGGL(ksum_k<false>, grid, dim3(CW), lds_bytes(nreg), st, *g, logn);
    return launch_rc();
}

#define PCH_CTS(L)                                                                                               \
    int cts_fused_##L(const CtsArgs* a, pc_stream_t s) { return cts::cts_fused<L>(a, s); }                       \
    int cts_fused_regen_##L(const CtsRegenArgs* a, pc_stream_t s) { return cts::cts_fused_regen<L>(a, s); }      \
    int ks_dot_regen_##L(const KsRegenArgs* a, pc_stream_t s) { return cts::ks_dot_regen<L>(a, s); }
PCH_CTS(12)
PCH_CTS(13)
PCH_CTS(14)
PCH_CTS(15)
PCH_CTS(16)

}  // namespace pch
