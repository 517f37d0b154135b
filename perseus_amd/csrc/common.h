// Device helpers of the gfx950 kernels: 32-bit modular arithmetic on the VALU, the ChaCha12 block, the bit-reversed
// automorphism index, launch helpers. Residues are canonical words in [0, p) with p < 2^31 (the u32 word's limit,
// crates/pc-core/src/modmul.rs:376-383).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pc_hip.h"

namespace pch {

// ------------------------------------------------------------------------------------------------ modular words
__device__ __forceinline__ uint32_t addm(uint32_t a, uint32_t b, uint32_t p) {
    const uint32_t s = a + b;  // < 2^32 since a, b < p < 2^31
    return s >= p ? s - p : s;
}
__device__ __forceinline__ uint32_t subm(uint32_t a, uint32_t b, uint32_t p) {
    const uint32_t d = a - b;
    return a >= b ? d : d + p;
}
// Shoup product a w mod p with ws = floor(w 2^32 / p): exact for any a < 2^32, w < p < 2^31. The unreduced form is in
// [0, 2p).
__device__ __forceinline__ uint32_t shoup_lz(uint32_t a, uint32_t w, uint32_t ws, uint32_t p) {
    return a * w - __umulhi(a, ws) * p;
}
__device__ __forceinline__ uint32_t shoup(uint32_t a, uint32_t w, uint32_t ws, uint32_t p) {
    const uint32_t r = shoup_lz(a, w, ws, p);
    return r >= p ? r - p : r;
}

// u mod p for any u < 2^32 with m = floor(2^32 / p): the quotient estimate is low by at most 1
__device__ __forceinline__ uint32_t red32(uint32_t u, uint32_t p, uint32_t m) {
    const uint32_t b = u - __umulhi(u, m) * p;
    return b >= p ? b - p : b;
}

// Reduction of any 64-bit x mod p (p < 2^31) from 32-bit products: x = hi 2^32 + lo, hi (2^32 mod p) as a Shoup
// product by the constant r32 = 2^32 mod p (companion r32s), lo mod p by m = floor(2^32 / p); each part below 2p
// before its guard. PrimeConst.split holds (r32, r32s), the high word of mu_lo is m (args.cuh:38-49).
struct Red {
    uint32_t p, r32, r32s, m;
    __device__ __forceinline__ explicit Red(const PrimeConst& c)
        : p((uint32_t)c.p), r32((uint32_t)c.split), r32s((uint32_t)(c.split >> 32)), m((uint32_t)(c.mu_lo >> 32)) {}
    __device__ __forceinline__ Red(uint32_t p_, uint32_t r32_, uint32_t r32s_, uint32_t m_)
        : p(p_), r32(r32_), r32s(r32s_), m(m_) {}
    // the constants of prime table entry i read with scalar loads (i uniform over the wave)
    __device__ __forceinline__ static Red scalar(const PrimeConst* pr, uint32_t i);
    __device__ __forceinline__ uint32_t operator()(uint64_t x) const {
        const uint32_t hi = (uint32_t)(x >> 32), lo = (uint32_t)x;
        uint32_t a = shoup(hi, r32, r32s, p);
        uint32_t b = lo - __umulhi(lo, m) * p;
        b = b >= p ? b - p : b;
        return addm(a, b, p);
    }
    // x = c 2^64 + v (a 96-bit sum of products, c small): c 2^64 = c (2^32 mod p)^2
    __device__ __forceinline__ uint32_t red96(uint64_t v, uint32_t c) const {
        uint32_t r = (*this)(v);
        if (c) {
            const uint32_t r64 = shoup(r32, r32, r32s, p);  // 2^64 mod p
            r = addm(r, (*this)((uint64_t)c * r64), p);
        }
        return r;
    }
    __device__ __forceinline__ uint32_t mul(uint32_t a, uint32_t b) const { return (*this)((uint64_t)a * b); }
};

// ------------------------------------------------------------------------------------------------ bit tricks
// A BSGS diagonal's compact index of output slot o (crates/pc-kernels/kernels/arith.cuh:242-244): o >> (enc & 0xFF)
// when enc >> 24 == 0x7F (a block-constant diagonal), else o & enc (0xFFFFFFFF: the full row)
__device__ __forceinline__ uint32_t ptidx(uint32_t o, uint32_t enc) {
    return (enc >> 24) == 0x7Fu ? o >> (enc & 0xFFu) : o & enc;
}
__device__ __forceinline__ uint32_t brev_n(uint32_t x, int logn) { return __brev(x) >> (32 - logn); }
// FIDESlib automorph_slot (crates/pc-kernels/kernels/arith.cuh:233-239; crates/pc-core/src/galois.rs:105-112): the
// slot of sigma_k's source for output `slot` in the bit-reversed evaluation order. Scatter by k = gather by k^-1.
__device__ __forceinline__ uint32_t automorph_slot(uint32_t k, uint32_t slot, int logn) {
    const uint32_t j = brev_n(slot, logn);
    const uint32_t r = (((j << 1) + 1) * k & ((2u << logn) - 1)) >> 1;
    return brev_n(r, logn);
}

// Scatter addresses of the automorphism inside a 1024-slot chunk. With V = ((2 brev(s) + 1) k) mod 2N for source slot
// s, the output slot's offset in its chunk is brev10 of W = the top 10 bits of V, and W is affine in the lane:
// W = C + k (brev6(lane) + 64 brev4(j)) mod 1024 for the lane's word j. Storing the word at rotr1(W) (a 10-bit rotate
// right) makes both the 64 lanes' writes of one j and the reads of output offsets 16 lane + j fall on 32 distinct
// banks per half wave; the offset 16 lane + j is read back from rotr1(64 brev4(j) + brev6(lane)).
__device__ __forceinline__ uint32_t scat_addr(uint32_t w) { return (w >> 1) | ((w & 1) << 9); }
__device__ __forceinline__ uint32_t brev4(uint32_t j) { return __brev(j) >> 28; }

// Wave-level ordering of LDS traffic between the lanes of one wave (no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------------------------------------------------ ChaCha12
constexpr uint32_t TAG_KSKA = 0x4b534b41u;  // "KSKA" (crates/pc-core/src/keys.rs:460)
constexpr uint32_t TAG_ENCA = 0x454e4341u;  // "ENCA" (args.cuh:615)
constexpr int KSK_T_MAX = 16;

__device__ __forceinline__ uint32_t rotl(uint32_t x, int r) { return __builtin_rotateleft32(x, r); }
#define PCH_QR(a, b, c, d)          \
    a += b;                         \
    d = rotl(d ^ a, 16);            \
    c += d;                         \
    b = rotl(b ^ c, 12);            \
    a += b;                         \
    d = rotl(d ^ a, 8);             \
    c += d;                         \
    b = rotl(b ^ c, 7);

// One ChaCha12 block (crates/pc-core/src/keys.rs:29-49 with 12 rounds): state words 12..15 = (w12, w13, w14, w15),
// the key in words 4..11, the feed-forward add; 16 output words in registers.
__device__ __forceinline__ void chacha12(const uint32_t (&k)[8], uint32_t w12, uint32_t w13, uint32_t w14, uint32_t w15,
                                         uint32_t (&o)[16]) {
    uint32_t x0 = 0x61707865u, x1 = 0x3320646eu, x2 = 0x79622d32u, x3 = 0x6b206574u;
    uint32_t x4 = k[0], x5 = k[1], x6 = k[2], x7 = k[3], x8 = k[4], x9 = k[5], x10 = k[6], x11 = k[7];
    uint32_t x12 = w12, x13 = w13, x14 = w14, x15 = w15;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        PCH_QR(x0, x4, x8, x12)
        PCH_QR(x1, x5, x9, x13)
        PCH_QR(x2, x6, x10, x14)
        PCH_QR(x3, x7, x11, x15)
        PCH_QR(x0, x5, x10, x15)
        PCH_QR(x1, x6, x11, x12)
        PCH_QR(x2, x7, x8, x13)
        PCH_QR(x3, x4, x9, x14)
    }
    o[0] = x0 + 0x61707865u;
    o[1] = x1 + 0x3320646eu;
    o[2] = x2 + 0x79622d32u;
    o[3] = x3 + 0x6b206574u;
    o[4] = x4 + k[0];
    o[5] = x5 + k[1];
    o[6] = x6 + k[2];
    o[7] = x7 + k[3];
    o[8] = x8 + k[4];
    o[9] = x9 + k[5];
    o[10] = x10 + k[6];
    o[11] = x11 + k[7];
    o[12] = x12 + w12;
    o[13] = x13 + w13;
    o[14] = x14 + w14;
    o[15] = x15 + w15;
}
// Only word w of a block (a retry draws one word).
__device__ __forceinline__ uint32_t chacha12_word(const uint32_t (&k)[8], uint32_t w12, uint32_t w13, uint32_t w14,
                                                  uint32_t w15, int w) {
    uint32_t o[16];
    chacha12(k, w12, w13, w14, w15, o);
    uint32_t v = o[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) v = (w == i) ? o[i] : v;
    return v;
}

// The KSKA expander's acceptance bound and reduction (crates/pc-host/src/chacha.rs:96-110): accept v < mp =
// floor((2^32-1)/p) p, value v - umulhi(v, floor((2^32-1)/p)) p with one guard (= v mod p for every v < 2^32).
struct Expander {
    uint32_t p, mu, mp;
    __device__ __forceinline__ explicit Expander(uint32_t p_) : p(p_), mu(0xFFFFFFFFu / p_), mp(mu * p_) {}
    __device__ __forceinline__ uint32_t red(uint32_t v) const {
        const uint32_t r = v - __umulhi(v, mu) * p;
        return r >= p ? r - p : r;
    }
};

// ------------------------------------------------------------------------------------------------ vector access
// A pointer read from a table in memory (a key's rows, a seed), unlike one passed as a kernel argument, is generic to
// the compiler: loads through it become flat loads, which also count against the LDS / scalar-load counter, so the next
// wait for an LDS access waits for them too. These views make such loads global loads.
typedef const __attribute__((address_space(1))) uint32_t* gptr;
typedef uint32_t gu4 __attribute__((ext_vector_type(4)));
typedef uint32_t gu4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ gptr as_global(const void* p) { return (gptr)p; }
// A read of read-only memory at an address uniform over the wave, through the constant address space: a scalar load
// (kept by the scalar cache, counted by lgkmcnt, not by the vector memory counter)
template <class T>
__device__ __forceinline__ T sload(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}
__device__ __forceinline__ Red Red::scalar(const PrimeConst* pr, uint32_t i) {
    const uint64_t p = sload(&pr[i].p), split = sload(&pr[i].split), mu = sload(&pr[i].mu_lo);
    return Red((uint32_t)p, (uint32_t)split, (uint32_t)(split >> 32), (uint32_t)(mu >> 32));
}
__device__ __forceinline__ void ld16(gptr p, uint32_t (&v)[16]) {
    const __attribute__((address_space(1))) gu4* q = (const __attribute__((address_space(1))) gu4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const gu4 x = q[i];
        v[4 * i] = x.x;
        v[4 * i + 1] = x.y;
        v[4 * i + 2] = x.z;
        v[4 * i + 3] = x.w;
    }
}
__device__ __forceinline__ void ld16(const uint32_t* p, uint32_t (&v)[16]) {
    const uint4* q = (const uint4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 x = q[i];
        v[4 * i] = x.x;
        v[4 * i + 1] = x.y;
        v[4 * i + 2] = x.z;
        v[4 * i + 3] = x.w;
    }
}
__device__ __forceinline__ void st16(uint32_t* p, const uint32_t (&v)[16]) {
    uint4* q = (uint4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = make_uint4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

// A raw buffer over [base, base + bytes): 32-bit loads and stores at a per-lane byte offset plus a uniform one kept in
// a scalar register, so a thread's strided accesses need one address register instead of one 64-bit address each;
// accesses past `bytes` read 0 and write nothing.
struct Buf {
    __amdgpu_buffer_rsrc_t r;
    // the base must be the same in every lane (a row of the workgroup); read through the first lane, so the compiler
    // keeps the resource in scalar registers instead of looping over lanes
    __device__ __forceinline__ static void* uniform(const void* p) {
        const uint64_t v = (uint64_t)p;
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
        return (void*)(((uint64_t)hi << 32) | lo);
    }
    __device__ __forceinline__ Buf(const void* base, uint32_t bytes)
        : r(__builtin_amdgcn_make_buffer_rsrc(uniform(base), 0, (int)bytes, 0x00020000)) {}
    __device__ __forceinline__ uint32_t ld(uint32_t voff, uint32_t soff) const {
        return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
    __device__ __forceinline__ void st(uint32_t v, uint32_t voff, uint32_t soff) const {
        __builtin_amdgcn_raw_buffer_store_b32(v, r, voff, soff, 0);
    }
};

// Workgroups of a launch are dispatched round-robin over the 8 XCDs (workgroup i to XCD i mod 8), each XCD with its own
// L2. Renumbering so that XCD k runs the contiguous range of logical blocks [k q + min(k, r), ...) (q, r = nblocks
// div / mod 8) keeps neighbouring blocks, which share cache lines and twiddle tables, on one L2.
__device__ __forceinline__ uint32_t xcd_block(uint32_t bid, uint32_t nblocks) {
    const uint32_t xcd = bid & 7, slot = bid >> 3, q = nblocks >> 3, r = nblocks & 7;
    return xcd * q + (xcd < r ? xcd : r) + slot;
}

inline int launch_rc() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}

}  // namespace pch
