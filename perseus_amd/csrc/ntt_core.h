// Device building blocks of the gfx950 NTT passes (the geometry, lazy butterflies, stage loops over registers, the
// wave-private LDS transposes, the XCD-aware block order), shared by the plain transforms (ntt.hip) and the passes
// that fuse a base conversion into the NTT (moddown.hip). The pass structure is described in ntt.hip.
#pragma once
#include "common.h"

namespace pch {
namespace ntt {

constexpr int E = 16;     // words per thread
constexpr int WG = 256;   // threads per workgroup

template <int LOGN>
struct Geo {
    static constexpr int LR = LOGN / 2, LC = LOGN - LR;
    static constexpr int N = 1 << LOGN, R = 1 << LR, C = 1 << LC;
    static constexpr int TR = R / E, TC = C / E;   // threads per column / row sub-transform
    static constexpr int CC = WG / TR;             // columns per column-pass workgroup
    static constexpr int BB = WG / TC;             // blocks per row-pass workgroup
    static constexpr int COL_WGS = C / CC;         // column-pass workgroups per row
    static constexpr int ROW_WGS = R / BB;         // row-pass workgroups per row
    // The column pass's transpose writes rows tau + TR j and reads rows E tau + j of a CC-wide tile. At CC = 16 one
    // padding row after every 16 rows puts the four rows a wave touches at once in four distinct 16-bank blocks on
    // both sides (a single padding word per row cannot serve both: the writes want an even row stride, the reads an
    // odd one); at CC >= 32 a wave touches at most two rows of 32 or more words, which unpadded rows serve.
    // Word j of thread (tau, col) is written at tau WT + col + j WS (row tau + TR j) and read at tau RT + col + j RS
    // (row E tau + j): with the padding row, row r sits at (r + r / 16) 16.
    static constexpr int COL_LDS = CC == 16 ? (R + R / 16) * 16 : R * CC;
    static constexpr int WT = CC == 16 ? 16 : CC, WS = CC == 16 ? 17 * 16 : TR * CC;
    static constexpr int RT = CC == 16 ? 17 * 16 : E * CC, RS = CC;
    static constexpr int ROW_LDS = BB * (C + C / E);
    static_assert(TR >= 2 && TC >= 2 && TR <= E && TC <= E, "sub-transforms of 32 to 256 points");
};

// ------------------------------------------------------------------------------------------------ butterflies
// Two VALU instructions the compiler does not form from this arithmetic by itself:
// v_sad_u32: a - b + c in one instruction, for b <= a < 2^31 (d = |a - b| + c);
// v_mad_u64_u32: a b + c mod 2^64; only the low word is used below, so c's high word is free and the Shoup product's
// subtraction of floor(a ws / 2^32) p folds into a multiply-add by 2^32 - p.
__device__ __forceinline__ uint32_t sub_add(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t d;
    asm("v_sad_u32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
// Shoup product a w mod p in [0, 2p) (as shoup_lz) in three instructions: a w as a 64-bit product, the quotient
// estimate, then a w + q (2^32 - p) mod 2^32
__device__ __forceinline__ uint32_t shoup3(uint32_t a, uint32_t w, uint32_t ws, uint32_t p) {
    uint64_t aw, r, c0, c1;
    asm("v_mad_u64_u32 %0, %1, %2, %3, 0" : "=v"(aw), "=s"(c0) : "v"(a), "v"(w));
    const uint32_t q = __umulhi(a, ws);
    asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=v"(r), "=s"(c1) : "v"(q), "v"(0u - p), "v"(aw));
    return (uint32_t)r;
}

// H: Harvey (every prime < 2^30). p2 = 2p. Forward: a in [0, 2p) ([0, 4p) for H), b any word; outputs in [0, 2p)
// ([0, 4p)). Inverse: canonical in and out ([0, 2p) for H).
template <bool H>
__device__ __forceinline__ void ct(uint32_t& a, uint32_t& b, uint32_t w, uint32_t ws, uint32_t p, uint32_t p2) {
    uint32_t t = shoup3(b, w, ws, p);  // [0, 2p)
    if (H) {
        const uint32_t u = min(a, a - p2);  // [0, 4p) -> [0, 2p)
        a = u + t;
        b = sub_add(p2, t, u);  // u - t + 2p
    } else {
        const uint32_t u = min(a, a - p);  // [0, 2p) -> [0, p)
        t = min(t, t - p);
        a = u + t;
        b = sub_add(p, t, u);  // u - t + p
    }
}
template <bool H>
__device__ __forceinline__ void gs(uint32_t& a, uint32_t& b, uint32_t w, uint32_t ws, uint32_t p, uint32_t p2) {
    const uint32_t u = a, v = b;
    if (H) {  // [0, 2p) in and out
        const uint32_t s = u + v;
        a = min(s, s - p2);
        b = shoup3(sub_add(p2, v, u), w, ws, p);
    } else {  // canonical in and out
        const uint32_t s = u + v;
        a = min(s, s - p);
        const uint32_t d = shoup3(sub_add(p, v, u), w, ws, p);
        b = min(d, d - p);
    }
}
// a forward lazy word as its residue
template <bool H>
__device__ __forceinline__ uint32_t canon(uint32_t a, uint32_t p, uint32_t p2) {
    if (H) a = min(a, a - p2);
    return min(a, a - p);
}

// NG consecutive twiddles of one stage in one vector load: a stage's groups are NG = 8 / (h / T) (layout A) or 8 / h
// (layout B) consecutive table entries, and their first index is a multiple of NG.
template <int NG>
__device__ __forceinline__ void ldtw(const uint32_t* p, uint32_t (&v)[8]) {
    if constexpr (NG == 8) {
        const uint4 a = ((const uint4*)p)[0], b = ((const uint4*)p)[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else if constexpr (NG == 4) {
        const uint4 a = *(const uint4*)p;
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
    } else if constexpr (NG == 2) {
        const uint2 a = *(const uint2*)p;
        v[0] = a.x, v[1] = a.y;
    } else {
        v[0] = *p;
    }
}

// NG twiddles at a workgroup-uniform address, through the scalar cache into scalar registers (the tables are read-only
// for the whole launch)
typedef __attribute__((address_space(4))) const uint32_t* cptr;
template <int NG>
__device__ __forceinline__ void ldtw_uniform(const uint32_t* p, uint32_t (&v)[8]) {
    const cptr q = (cptr)p;
#pragma unroll
    for (int i = 0; i < NG; ++i) v[i] = q[i];
}

// Layout A (e = tau + T j), stage h = T 2^K: pairs (j, j + 2^K), group j / 2^(K+1), index base(h) + group. UNI: base()
// is the same for every thread of the workgroup (the column passes).
template <bool FWD, bool H, int T, int K, class Base, bool UNI = false>
__device__ __forceinline__ void stage_a(uint32_t (&x)[E], const uint32_t* w, const uint32_t* ws, uint32_t p,
                                        uint32_t p2, Base base) {
    constexpr int hh = 1 << K, NG = 8 >> K;
    const uint32_t b0 = base(T << K);
    uint32_t tw[8], tws[8];
    if constexpr (UNI) {
        ldtw_uniform<NG>(w + b0, tw);
        ldtw_uniform<NG>(ws + b0, tws);
    } else {
        ldtw<NG>(w + b0, tw);
        ldtw<NG>(ws + b0, tws);
    }
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (j & hh) continue;
        const int g = j >> (K + 1);
        if (FWD) ct<H>(x[j], x[j + hh], tw[g], tws[g], p, p2);
        else gs<H>(x[j], x[j + hh], tw[g], tws[g], p, p2);
    }
}
template <bool FWD, bool H, int T, class Base, bool UNI = false>
__device__ __forceinline__ void phase_a(uint32_t (&x)[E], const uint32_t* w, const uint32_t* ws, uint32_t p,
                                        uint32_t p2, Base base) {
    if (FWD) {
        stage_a<FWD, H, T, 3, Base, UNI>(x, w, ws, p, p2, base);
        stage_a<FWD, H, T, 2, Base, UNI>(x, w, ws, p, p2, base);
        stage_a<FWD, H, T, 1, Base, UNI>(x, w, ws, p, p2, base);
        stage_a<FWD, H, T, 0, Base, UNI>(x, w, ws, p, p2, base);
    } else {
        stage_a<FWD, H, T, 0, Base, UNI>(x, w, ws, p, p2, base);
        stage_a<FWD, H, T, 1, Base, UNI>(x, w, ws, p, p2, base);
        stage_a<FWD, H, T, 2, Base, UNI>(x, w, ws, p, p2, base);
        stage_a<FWD, H, T, 3, Base, UNI>(x, w, ws, p, p2, base);
    }
}
// Layout B (e = 16 tau + j), stage h = 2^K < T: pairs (j, j + h), group (16 tau + j) / (2h).
template <bool FWD, bool H, int K, class Base>
__device__ __forceinline__ void stage_b(uint32_t (&x)[E], int tau, const uint32_t* w, const uint32_t* ws, uint32_t p,
                                        uint32_t p2, Base base) {
    constexpr int h = 1 << K, NG = 8 >> K;
    const uint32_t b0 = base(h) + ((uint32_t)(E * tau) >> (K + 1));
    uint32_t tw[8], tws[8];
    ldtw<NG>(w + b0, tw);
    ldtw<NG>(ws + b0, tws);
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (j & h) continue;
        const int g = j >> (K + 1);
        if (FWD) ct<H>(x[j], x[j + h], tw[g], tws[g], p, p2);
        else gs<H>(x[j], x[j + h], tw[g], tws[g], p, p2);
    }
}
template <bool FWD, bool H, int T, class Base>
__device__ __forceinline__ void phase_b(uint32_t (&x)[E], int tau, const uint32_t* w, const uint32_t* ws, uint32_t p,
                                        uint32_t p2, Base base) {
    constexpr int LT = T == 16 ? 4 : T == 8 ? 3 : T == 4 ? 2 : 1;
    if (FWD) {
        if (LT > 3) stage_b<FWD, H, 3>(x, tau, w, ws, p, p2, base);
        if (LT > 2) stage_b<FWD, H, 2>(x, tau, w, ws, p, p2, base);
        if (LT > 1) stage_b<FWD, H, 1>(x, tau, w, ws, p, p2, base);
        stage_b<FWD, H, 0>(x, tau, w, ws, p, p2, base);
    } else {
        stage_b<FWD, H, 0>(x, tau, w, ws, p, p2, base);
        if (LT > 1) stage_b<FWD, H, 1>(x, tau, w, ws, p, p2, base);
        if (LT > 2) stage_b<FWD, H, 2>(x, tau, w, ws, p, p2, base);
        if (LT > 3) stage_b<FWD, H, 3>(x, tau, w, ws, p, p2, base);
    }
}

// A phase's twiddles preloaded into registers (15 values and 15 Shoup companions: the 1 + 2 + 4 + 8 group twiddles of
// its four stages, stage K's NG = 8 >> K at offset NG - 1), so that every load of a pass can be issued before its
// first LDS transpose.
struct Tw {
    uint32_t w[15], s[15];
};
template <int NG>
__device__ __forceinline__ void ldtw_at(const uint32_t* p, uint32_t* v) {
    uint32_t t[8];
    ldtw<NG>(p, t);
#pragma unroll
    for (int i = 0; i < NG; ++i) v[i] = t[i];
}
// layout A, stages h = T 2^K (K = 0..3)
template <int T, class Base>
__device__ __forceinline__ void load_tw_a(Tw& t, const uint32_t* w, const uint32_t* ws, Base base) {
#define PCH_LA(K)                                                    \
    {                                                                \
        const uint32_t b0 = base(T << K);                            \
        ldtw_at<(8 >> K)>(w + b0, t.w + ((8 >> K) - 1));             \
        ldtw_at<(8 >> K)>(ws + b0, t.s + ((8 >> K) - 1));            \
    }
    PCH_LA(3) PCH_LA(2) PCH_LA(1) PCH_LA(0)
#undef PCH_LA
}
// layout B, stages h = 2^K < T
template <int T, class Base>
__device__ __forceinline__ void load_tw_b(Tw& t, int tau, const uint32_t* w, const uint32_t* ws, Base base) {
    constexpr int LT = T == 16 ? 4 : T == 8 ? 3 : T == 4 ? 2 : 1;
#define PCH_LB(K)                                                                    \
    if (LT > K) {                                                                    \
        const uint32_t b0 = base(1 << K) + ((uint32_t)(E * tau) >> (K + 1));         \
        ldtw_at<(8 >> K)>(w + b0, t.w + ((8 >> K) - 1));                             \
        ldtw_at<(8 >> K)>(ws + b0, t.s + ((8 >> K) - 1));                            \
    }
    PCH_LB(3) PCH_LB(2) PCH_LB(1) PCH_LB(0)
#undef PCH_LB
}
// one stage of pairs (j, j + 2^K) over preloaded twiddles (both layouts: the group of j is j >> (K + 1))
template <bool FWD, bool H, int K>
__device__ __forceinline__ void stage_t(uint32_t (&x)[E], const Tw& t, uint32_t p, uint32_t p2) {
    constexpr int hh = 1 << K, o = (8 >> K) - 1;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (j & hh) continue;
        const int g = j >> (K + 1);
        if (FWD) ct<H>(x[j], x[j + hh], t.w[o + g], t.s[o + g], p, p2);
        else gs<H>(x[j], x[j + hh], t.w[o + g], t.s[o + g], p, p2);
    }
}
template <bool FWD, bool H>
__device__ __forceinline__ void phase_a_t(uint32_t (&x)[E], const Tw& t, uint32_t p, uint32_t p2) {
    if (FWD) {
        stage_t<FWD, H, 3>(x, t, p, p2);
        stage_t<FWD, H, 2>(x, t, p, p2);
        stage_t<FWD, H, 1>(x, t, p, p2);
        stage_t<FWD, H, 0>(x, t, p, p2);
    } else {
        stage_t<FWD, H, 0>(x, t, p, p2);
        stage_t<FWD, H, 1>(x, t, p, p2);
        stage_t<FWD, H, 2>(x, t, p, p2);
        stage_t<FWD, H, 3>(x, t, p, p2);
    }
}
template <bool FWD, bool H, int T>
__device__ __forceinline__ void phase_b_t(uint32_t (&x)[E], const Tw& t, uint32_t p, uint32_t p2) {
    constexpr int LT = T == 16 ? 4 : T == 8 ? 3 : T == 4 ? 2 : 1;
    if (FWD) {
        if (LT > 3) stage_t<FWD, H, 3>(x, t, p, p2);
        if (LT > 2) stage_t<FWD, H, 2>(x, t, p, p2);
        if (LT > 1) stage_t<FWD, H, 1>(x, t, p, p2);
        stage_t<FWD, H, 0>(x, t, p, p2);
    } else {
        stage_t<FWD, H, 0>(x, t, p, p2);
        if (LT > 1) stage_t<FWD, H, 1>(x, t, p, p2);
        if (LT > 2) stage_t<FWD, H, 2>(x, t, p, p2);
        if (LT > 3) stage_t<FWD, H, 3>(x, t, p, p2);
    }
}

// A row-pass block's 16 words of thread tau through the block's LDS (C + C/16 words, one padding word per 16):
// layout B (e = 16 tau + j) -> layout A (e = tau + T j) and back. The block lives in one wave.
template <int T>
__device__ __forceinline__ void b_to_a(uint32_t (&x)[E], uint32_t* l, int tau) {
#pragma unroll
    for (int j = 0; j < E; ++j) l[(E * tau + j) + tau] = x[j];
    wave_sync();
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int e = tau + T * j;
        x[j] = l[e + e / E];
    }
    wave_sync();
}
template <int T>
__device__ __forceinline__ void a_to_b(uint32_t (&x)[E], uint32_t* l, int tau) {
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int e = tau + T * j;
        l[e + e / E] = x[j];
    }
    wave_sync();
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = l[(E * tau + j) + tau];
    wave_sync();
}

// ------------------------------------------------------------------------------------------------ row pass, C = 256
// A 256-word block held by its 16 threads t in one of two layouts:
//  D: register 4 k + m holds word e = 64 k + 4 t + m (k, m < 4). For each k the block's 16 threads read or write 256
//     contiguous bytes with one 16-byte access each, so every global access of the pass moves whole cache lines (the
//     B layout's 64 contiguous bytes per thread put each 16-byte access of a wave on a different line: four times
//     the requests for the same bytes);
//  E: thread t = 4 k + m, register j holds word e = 64 k + 4 j + m.
// Stages h = 128, 64 (word bits 7, 6 = k) and h = 2, 1 (bits 1, 0 = m) run in D, h = 32 .. 4 (bits 5..2 = j) in E. The
// transposes D <-> E go through the block's LDS with one padding word per 16: both sides conflict-free.
__device__ __forceinline__ uint32_t dpos(uint32_t e) { return e + (e >> 4); }
__device__ __forceinline__ void ld_d(const uint32_t* q, uint32_t (&v)[E]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 a = *(const uint4*)(q + 64 * k);
        v[4 * k] = a.x, v[4 * k + 1] = a.y, v[4 * k + 2] = a.z, v[4 * k + 3] = a.w;
    }
}
// ld_d of words read once (streamed past the caches)
__device__ __forceinline__ void ld_d_nt(const uint32_t* q, uint32_t (&v)[E]) {
    typedef const __attribute__((address_space(1))) gu4* gq;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const gu4 a = __builtin_nontemporal_load((gq)(q + 64 * k));
        v[4 * k] = a.x, v[4 * k + 1] = a.y, v[4 * k + 2] = a.z, v[4 * k + 3] = a.w;
    }
}
__device__ __forceinline__ void st_d(uint32_t* q, const uint32_t (&v)[E]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) *(uint4*)(q + 64 * k) = make_uint4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
}
__device__ __forceinline__ void d_to_e(uint32_t (&x)[E], uint32_t* l, int t) {
#pragma unroll
    for (int r = 0; r < E; ++r) l[dpos(64 * (r >> 2) + 4 * t + (r & 3))] = x[r];
    wave_sync();
    const int k = t >> 2, m = t & 3;
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = l[dpos(64 * k + 4 * j + m)];
    wave_sync();
}
__device__ __forceinline__ void e_to_d(uint32_t (&x)[E], uint32_t* l, int t) {
    const int k = t >> 2, m = t & 3;
#pragma unroll
    for (int j = 0; j < E; ++j) l[dpos(64 * k + 4 * j + m)] = x[j];
    wave_sync();
#pragma unroll
    for (int r = 0; r < E; ++r) x[r] = l[dpos(64 * (r >> 2) + 4 * t + (r & 3))];
    wave_sync();
}
// the E layout's twiddles of stages h = 4 2^K (K = 3..0): NG = 8 >> K consecutive entries from base(h) + k NG, stage
// K's at offset NG - 1 (the phase_a_t order)
template <class Base>
__device__ __forceinline__ void load_tw_e(Tw& tw, const uint32_t* w, const uint32_t* ws, Base base, int k) {
#define PCH_LE(K)                                                                      \
    {                                                                                  \
        const uint32_t b0 = base(4 << K) + (uint32_t)k * (8 >> K);                     \
        ldtw_at<(8 >> K)>(w + b0, tw.w + ((8 >> K) - 1));                              \
        ldtw_at<(8 >> K)>(ws + b0, tw.s + ((8 >> K) - 1));                             \
    }
    PCH_LE(3) PCH_LE(2) PCH_LE(1) PCH_LE(0)
#undef PCH_LE
}
// stages h = 128 then 64 (FWD) or 64 then 128 in the D layout: h = 128 pairs registers (r, r + 8), r < 8, one twiddle
// base(128); h = 64 pairs (r, r + 4) for k in {0, 2}, twiddle base(64) + k / 2
template <bool FWD, bool H, class Base>
__device__ __forceinline__ void stages_hi_d(uint32_t (&x)[E], const uint32_t* w, const uint32_t* ws, Base base,
                                            uint32_t p, uint32_t p2) {
    const uint32_t a0 = w[base(128)], s0 = ws[base(128)];
    const uint2 a1 = *(const uint2*)(w + base(64)), s1 = *(const uint2*)(ws + base(64));
    auto h128 = [&] {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            if (FWD) ct<H>(x[r], x[r + 8], a0, s0, p, p2);
            else gs<H>(x[r], x[r + 8], a0, s0, p, p2);
        }
    };
    auto h64 = [&] {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (FWD) {
                ct<H>(x[r], x[r + 4], a1.x, s1.x, p, p2);
                ct<H>(x[r + 8], x[r + 12], a1.y, s1.y, p, p2);
            } else {
                gs<H>(x[r], x[r + 4], a1.x, s1.x, p, p2);
                gs<H>(x[r + 8], x[r + 12], a1.y, s1.y, p, p2);
            }
        }
    };
    if (FWD) {
        h128();
        h64();
    } else {
        h64();
        h128();
    }
}
// stages h = 2 then 1 (FWD) or 1 then 2 in the D layout: h = 2 pairs (4k + m, 4k + m + 2), m < 2, twiddle
// base(2) + 16 k + t; h = 1 pairs (4k + m, 4k + m + 1), m in {0, 2}, twiddle base(1) + 32 k + 2 t + m / 2
template <bool FWD, bool H, class Base>
__device__ __forceinline__ void stages_lo_d(uint32_t (&x)[E], const uint32_t* w, const uint32_t* ws, Base base, int t,
                                            uint32_t p, uint32_t p2) {
    uint32_t a2[4], s2[4];
    uint2 a1[4], s1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        a2[k] = w[base(2) + 16 * k + t];
        s2[k] = ws[base(2) + 16 * k + t];
        a1[k] = *(const uint2*)(w + base(1) + 32 * k + 2 * t);
        s1[k] = *(const uint2*)(ws + base(1) + 32 * k + 2 * t);
    }
    auto h2 = [&] {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (FWD) {
                ct<H>(x[4 * k], x[4 * k + 2], a2[k], s2[k], p, p2);
                ct<H>(x[4 * k + 1], x[4 * k + 3], a2[k], s2[k], p, p2);
            } else {
                gs<H>(x[4 * k], x[4 * k + 2], a2[k], s2[k], p, p2);
                gs<H>(x[4 * k + 1], x[4 * k + 3], a2[k], s2[k], p, p2);
            }
        }
    };
    auto h1 = [&] {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (FWD) {
                ct<H>(x[4 * k], x[4 * k + 1], a1[k].x, s1[k].x, p, p2);
                ct<H>(x[4 * k + 2], x[4 * k + 3], a1[k].y, s1[k].y, p, p2);
            } else {
                gs<H>(x[4 * k], x[4 * k + 1], a1[k].x, s1[k].x, p, p2);
                gs<H>(x[4 * k + 2], x[4 * k + 3], a1[k].y, s1[k].y, p, p2);
            }
        }
    };
    if (FWD) {
        h2();
        h1();
    } else {
        h1();
        h2();
    }
}

// Row i's prime id and offset (in rows of N words). Dense launches (roff and rprime both null; internal launchers
// only, the table entries reject them) take row i at i N with prime id i mod xnum.
__device__ __forceinline__ int row_prime(const NttArgs& A, int i) { return A.rprime ? A.rprime[i] : i % A.xnum; }
__device__ __forceinline__ size_t row_off(const NttArgs& A, int i) { return A.roff ? (size_t)A.roff[i] : (size_t)i; }

// The first pass's source words of row i: out of place (src + soff[i] N, the sum mod p of snum rows sstride apart)
// or in place (base + roff[i] N).
struct RowSrc {
    const uint32_t* p0;
    int n;
    uint64_t stride;
};
__device__ __forceinline__ RowSrc row_src(const NttArgs& A, int i, int logn) {
    if (A.soff) return RowSrc{(const uint32_t*)A.src + ((size_t)A.soff[i] << logn), A.snum, A.sstride};
    return RowSrc{(const uint32_t*)A.base + (row_off(A, i) << logn), 1, 0};
}
__device__ __forceinline__ uint32_t ld_src(const RowSrc& s, size_t off, uint32_t p) {
    uint32_t v = s.p0[off];
    for (int k = 1; k < s.n; ++k) v = addm(v, s.p0[off + k * s.stride], p);
    return v;
}
__device__ __forceinline__ void ld16_src(const RowSrc& s, size_t off, uint32_t p, uint32_t (&x)[E]) {
    ld16(s.p0 + off, x);
    for (int k = 1; k < s.n; ++k) {
        uint32_t y[E];
        ld16(s.p0 + off + k * s.stride, y);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = addm(x[j], y[j], p);
    }
}

// ld16_src in the D layout: the words of registers 4k + m at off + 64 k + m, summed over the source's rows
__device__ __forceinline__ void ld_d_src(const RowSrc& s, size_t off, uint32_t p, uint32_t (&x)[E]) {
    ld_d(s.p0 + off, x);
    for (int k = 1; k < s.n; ++k) {
        uint32_t y[E];
        ld_d(s.p0 + off + k * s.stride, y);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = addm(x[j], y[j], p);
    }
}

// the workgroup's logical (block in row, row) after the XCD renumbering of a (gx, rows) grid
struct Blk {
    int x, y;
};
__device__ __forceinline__ Blk blk_xy() {
    const uint32_t n = gridDim.x * gridDim.y;
    const uint32_t l = xcd_block(blockIdx.y * gridDim.x + blockIdx.x, n);
    return Blk{(int)(l % gridDim.x), (int)(l / gridDim.x)};
}

}  // namespace ntt
}  // namespace pch
