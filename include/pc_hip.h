/* pc-hip: the MI355X (gfx950) kernels of the CKKS key-switch / NTT path behind the reference's kernel ABI.
 *
 * Three layers, all plain C ABI (no HIP or torch types in a signature; a stream is a hipStream_t passed as void*):
 *
 *  1. The kernel table. Byte-identical mirrors of the reference's ABI-30 launch-argument structs
 *     (crates/pc-kernels/kernels/args.cuh) and its KernelTable of 52 launchers
 *     (args.cuh:1037-1097). pc_table_u32_barrett64() replaces the CUDA build's export of the same name
 *     (crates/pc-kernels/kernels/inst/instantiate.inc:32-91, looked up by crates/pc-kernels/src/table.rs:101-112).
 *     Every launcher reads *args, enqueues on the stream and returns 0, -1/-2/-3 for an argument outside the
 *     kernel's range (args.cuh:1036; crates/pc-cuda/src/error.rs:47-54) or a positive HIP error code. Launchers never
 *     allocate, free or synchronise, so they may be captured into a HIP graph.
 *  2. The runtime FFI (pc_hip_*), the HIP replacement of crates/pc-cuda's cudart bindings (ffi.rs:18-50, mem.rs:19-24):
 *     device, memory, streams, events, graphs.
 *  3. The key-switching driver (pcx_*), the launch sequences of crates/pc-gpu (ks.rs, rotate.rs, ntt.rs, keygen.rs)
 *     restated in C++ over the table: a context of one chain, setup-time plans per limb top, key groups, rotations.
 */
#ifndef PC_HIP_H
#define PC_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#define PC_STATIC_ASSERT(c, m) static_assert(c, m)
#else
#define PC_STATIC_ASSERT(c, m) _Static_assert(c, m)
#endif

#define PC_KERNELS_ABI 30u

typedef void* pc_stream_t; /* a hipStream_t */

/* ------------------------------------------------------------------------------------------ ABI-30 structs */
/* args.cuh:21-49 */
typedef struct PrimeConst {
    uint64_t p;
    uint64_t mu_lo;
    uint64_t mu_hi;
    uint64_t neal_mu;
    uint32_t bits;
    uint32_t word_bits;
    uint64_t mont_pinv;
    uint64_t mont_r2;
    uint64_t split;
} PrimeConst;
PC_STATIC_ASSERT(sizeof(PrimeConst) == 64, "PrimeConst layout");

/* args.cuh:52-57 */
typedef struct RowSet {
    int32_t nq, np, qmax, pad;
} RowSet;
PC_STATIC_ASSERT(sizeof(RowSet) == 16, "RowSet layout");

/* args.cuh:59-64 */
typedef struct PolyRef {
    void* base;
    uint64_t ct_stride, part_stride;
} PolyRef;
PC_STATIC_ASSERT(sizeof(PolyRef) == 24, "PolyRef layout");

/* args.cuh:67-107: in-place negacyclic NTT of nrows rows (row i at base + roff[i]*N, prime id rprime[i]), OpenFHE
 * order; soff: out-of-place first pass summing snum source rows; epi 1/2/3: forward epilogues; es/ess: the inverse's
 * per-row scale */
typedef struct NttArgs {
    void* base;
    const uint32_t* roff;
    const int32_t* rprime;
    const void* fw;
    const void* fws;
    const void* iw;
    const void* iws;
    const void* ninv;
    const void* ninvs;
    const PrimeConst* pr;
    int32_t nrows, chunk;
    const void* src;
    const uint32_t* soff;
    void* eout;
    const void* ex;
    const void* es;
    const void* ess;
    int32_t epi, snum;
    uint64_t sstride;
    int32_t xnum, lazy;
    uint64_t xstride;
    const void* ed;
} NttArgs;
PC_STATIC_ASSERT(sizeof(NttArgs) == 176, "NttArgs layout");

/* args.cuh:110-128: one fast base-conversion job; pool at pool_off: src_row[ns], src_prime[ns], pre[ns],
 * tgt_row[nt], tgt_prime[nt], M[ns][nt] (u32 words) */
typedef struct BconvJob {
    uint32_t src_off, dst_off;
    uint32_t nsrc, ntgt;
    uint32_t pool_off;
    uint32_t exact;
    uint32_t prescaled;
    uint32_t split;
} BconvJob;
PC_STATIC_ASSERT(sizeof(BconvJob) == 32, "BconvJob layout");

typedef struct BconvArgs {
    const void* src;
    void* dst;
    const BconvJob* jobs;
    const void* pool;
    const PrimeConst* pr;
    int32_t njobs, max_tgt;
    int32_t kind, pad;
} BconvArgs;
PC_STATIC_ASSERT(sizeof(BconvArgs) == 56, "BconvArgs layout");

/* args.cuh:144-157: element-wise row-set kernels */
typedef struct EwArgs {
    PolyRef out, a, b;
    RowSet rs;
    const void* sc;
    const void* scs;
    const PrimeConst* pr;
    int32_t K, nparts, sub, zero_p;
} EwArgs;
PC_STATIC_ASSERT(sizeof(EwArgs) == 128, "EwArgs layout");

/* args.cuh:211-228: hybrid key-switch inner product */
#define PC_KS_ACC 4
#define PC_KS_SUM 8
typedef struct KsArgs {
    const void* c1;
    const void* modup;
    const void* c0;
    void* out0;
    void* out1;
    const void* const* kb;
    const void* const* ka;
    const uint32_t* autok;
    const uint32_t* rows;
    const int32_t* digit_of;
    const void* pmod;
    const void* pmods;
    const PrimeConst* pr;
    uint64_t ct_stride, mu_ct_stride, mu_digit_stride, out_ct_stride, out_rot_stride, key_digit_stride;
    int32_t K, R, ndig, c0_mode, nq, nrows;
} KsArgs;
PC_STATIC_ASSERT(sizeof(KsArgs) == 176, "KsArgs layout");

/* args.cuh:263-277 */
typedef struct EpiArgs {
    void* dst;
    const void* conv;
    const void* binv;
    const void* binvs;
    const void* k;
    uint64_t part_stride;
    int32_t dbl, pad;
    const void* alpha;
    const void* alphas;
} EpiArgs;
PC_STATIC_ASSERT(sizeof(EpiArgs) == 72, "EpiArgs layout");

/* args.cuh:279-290: switching keys read in their stored form, `a` regenerated from each key's KSKA seed */
typedef struct KeyTab {
    const void* const* kb;
    const uint32_t* const* seed;
    uint64_t row_words;
    int32_t bits;
    int32_t q_top;
    int32_t srows;
    int32_t nregen;
} KeyTab;
PC_STATIC_ASSERT(sizeof(KeyTab) == 40, "KeyTab layout");

/* args.cuh:292-304 */
typedef struct KsRegenArgs {
    KsArgs ks;
    const uint32_t* seed;
    EpiArgs epi;
    int32_t use_epi, pad;
    KeyTab key;
    const void* add;
} KsRegenArgs;
PC_STATIC_ASSERT(sizeof(KsRegenArgs) == 312, "KsRegenArgs layout");

/* args.cuh:306-323: KSKA rows out[d - d0][m][N] */
typedef struct KskExpandArgs {
    void* out;
    const uint32_t* seed;
    const int32_t* prime_ids;
    const PrimeConst* pr;
    int32_t nmod, dnum;
    int32_t d0, pad;
} KskExpandArgs;
PC_STATIC_ASSERT(sizeof(KskExpandArgs) == 48, "KskExpandArgs layout");

/* args.cuh:582-592: sigma_k gather in the bit-reversed evaluation order */
typedef struct AutomorphArgs {
    PolyRef out, in, add;
    RowSet rs;
    const PrimeConst* pr;
    uint32_t k;
    int32_t K, nparts, has_add;
} AutomorphArgs;
PC_STATIC_ASSERT(sizeof(AutomorphArgs) == 112, "AutomorphArgs layout");

/* args.cuh:614-628: secret-key encryption, a from the "ENCA" expander lane */
typedef struct EncryptArgs {
    void* c0;
    void* c1;
    const void* s;
    const void* e;
    const void* m;
    const uint32_t* seed;
    const PrimeConst* pr;
    uint32_t nonce;
    int32_t nl;
} EncryptArgs;
PC_STATIC_ASSERT(sizeof(EncryptArgs) == 64, "EncryptArgs layout");

/* args.cuh:631-654: one hybrid switching key (OpenFHE KeySwitchGenInternal relation), dense or bit-packed b */
typedef struct KskGenArgs {
    void* b;
    void* a;
    const void* e;
    const void* s_new;
    const void* s_old;
    const uint32_t* seed;
    const int32_t* ids;
    const int32_t* digit_of;
    const void* pmod;
    const void* pmods;
    const PrimeConst* pr;
    uint64_t row_words;
    int32_t nrows, ndig, nq, bits, sq, pad;
} KskGenArgs;
PC_STATIC_ASSERT(sizeof(KskGenArgs) == 120, "KskGenArgs layout");

/* args.cuh:656-663 */
typedef struct KskUnpackArgs {
    void* out;
    const uint32_t* in;
    uint64_t row_words;
    int32_t nrows, bits;
} KskUnpackArgs;
PC_STATIC_ASSERT(sizeof(KskUnpackArgs) == 32, "KskUnpackArgs layout");

/* args.cuh:760-768 */
typedef struct KsKeyArgs {
    KsArgs ks;
    KeyTab key;
} KsKeyArgs;
PC_STATIC_ASSERT(sizeof(KsKeyArgs) == 216, "KsKeyArgs layout");

/* args.cuh:325-355: the fused CtS / StC stage core (hoisted baby-step rotations times the BSGS plaintext diagonals
 * in the extended basis, gather form). For output slot o of row t = rows[y]:
 *   rot_0[o] = (P c0[o], P c1[o]) on Q rows, 0 on special rows (P = pmod[t], Shoup companion pmods[t]); with x0
 *              non-null, x0's words as stored (every row);
 *   rot_i[o] = (P c0[s] + sum_d D_d[s] b_{i,d}[s], sum_d D_d[s] a_{i,d}[s]), s = automorph_slot(kinv[i-1], o),
 *              D_d = c1 on the rows of digit d (digit_of), else modup's digit d;
 *   res_j[o] = sum_i rot_i[o] pt_{B j + i}[prow][ptidx(o, enc)], j < G, diagonals >= npts skipped; prow = t on Q rows,
 *              pt_prow + (t - nq) on special rows; ptidx = o >> (enc & 0xFF) when enc >> 24 == 0x7F, else o & enc.
 * Ciphertext c at x + c ct_stride (c1 at + part_stride), ModUp at modup + c mu_ct_stride + d mu_digit_stride, baby keys
 * kb / ka [i-1] + d key_digit_stride + t N; results (c, j) at res + (c G + j) ct_stride, or with pair_cts > 0 (K = 1
 * regen launches of up to 4 giant steps) at res + ((j >> 1) pair_cts + (j & 1)) ct_stride. Strides in words; rows of
 * N words, 16-byte aligned. */
typedef struct CtsArgs {
    const void* x;
    const void* modup;
    void* res;
    const void* const* kb;
    const void* const* ka;
    const uint32_t* kinv;
    const void* const* pts;
    const uint32_t* rows;
    const int32_t* digit_of;
    const void* pmod;
    const void* pmods;
    const PrimeConst* pr;
    uint64_t ct_stride, part_stride, mu_ct_stride, mu_digit_stride, key_digit_stride;
    int32_t K, B, G, npts, ndig, nq, nlive, ptw, pt_prow;
    uint32_t enc;
    int32_t ngrp;
    int32_t nrows, kmax;
    int32_t pair_cts;
    const void* x0;
} CtsArgs;
PC_STATIC_ASSERT(sizeof(CtsArgs) == 200, "CtsArgs layout");

/* args.cuh:753-758: cts_fused with the baby keys through a KeyTab: `b` read in its stored form (dense or packed),
 * `a` regenerated for digits < key.nregen, else read from cts.ka */
typedef struct CtsRegenArgs {
    CtsArgs cts;
    KeyTab key;
} CtsRegenArgs;
PC_STATIC_ASSERT(sizeof(CtsRegenArgs) == 240, "CtsRegenArgs layout");

/* ---- EvalMod / plaintext-product element-wise kernels (em.cuh). Q rows [0, n) of K ciphertexts, row index = prime
 * id; grid (N/1024, n, K or 2K); every output word a canonical residue. */

/* args.cuh:356-367: (c0, c1, d2) (= | +=) sum_{j < min(npairs, 2)} (a_j0 b_j0, a_j0 b_j1 + a_j1 b_j0, a_j1 b_j1); d2
 * written to part 1 of `d2` (and to coef + c coef_ct_stride + row N when coef is set); acc: (c0, c1) += the old
 * words, acc_d2: d2 += its old words; dbl: all three doubled after the adds */
typedef struct TensorArgs {
    PolyRef out, d2, a0, b0, a1, b1;
    void* coef;
    uint64_t coef_ct_stride;
    const PrimeConst* pr;
    int32_t npairs, acc, n, K;
    int32_t dbl, acc_d2;
} TensorArgs;
PC_STATIC_ASSERT(sizeof(TensorArgs) == 192, "TensorArgs layout");

/* args.cuh:369-378: tensor, then (c0, c1) +-= y c[row] (Shoup companion cs) after the doubling; d2 unchanged */
typedef struct TensorYArgs {
    TensorArgs t;
    PolyRef y;
    const void* c;
    const void* cs;
    int32_t sub, pad;
} TensorYArgs;
PC_STATIC_ASSERT(sizeof(TensorYArgs) == 240, "TensorYArgs layout");

/* args.cuh:379-389: tensor over up to PC_TSUM_MAX pairs passed by value; acc nonzero: (c0, c1) +=, acc & 2: d2 += */
#define PC_TSUM_MAX 16
typedef struct TensorSumArgs {
    PolyRef out, d2;
    PolyRef a[PC_TSUM_MAX], b[PC_TSUM_MAX];
    const PrimeConst* pr;
    int32_t npairs, acc, n, K;
} TensorSumArgs;
PC_STATIC_ASSERT(sizeof(TensorSumArgs) == 2 * 24 + 2 * PC_TSUM_MAX * 24 + 8 + 16, "TensorSumArgs layout");

/* args.cuh:391-406: nout <= 4 tensor sums in one call, output o = sum_{j < npairs <= 32} a[o][j] b[o][j] (c0, c1 into
 * out[o], d2 into part 1 of d2[o]; acc as tensor_sum's). Here each output's pairs run as launches of 16, so no
 * output may alias an operand of the call. */
#define PC_TMULTI_OUT 4
#define PC_TMULTI_PAIRS 32
typedef struct TensorMultiArgs {
    PolyRef out[PC_TMULTI_OUT], d2[PC_TMULTI_OUT];
    PolyRef a[PC_TMULTI_OUT][PC_TMULTI_PAIRS], b[PC_TMULTI_OUT][PC_TMULTI_PAIRS];
    const PrimeConst* pr;
    int32_t nout, npairs, acc, n, K, pad;
} TensorMultiArgs;
PC_STATIC_ASSERT(sizeof(TensorMultiArgs) == (2 * PC_TMULTI_OUT + 2 * PC_TMULTI_OUT * PC_TMULTI_PAIRS) * 24 + 8 + 24,
                 "TensorMultiArgs layout");

/* args.cuh:438-447: for parts 0, 1: dst = f (dst + (x - t) binv) [+ k[row] on part 0, reduced once], f = 2 when dbl */
typedef struct MdEpiArgs {
    PolyRef dst, x, t;
    const void* binv;
    const void* binvs;
    const void* k;
    const PrimeConst* pr;
    int32_t dbl, n, K, pad;
} MdEpiArgs;
PC_STATIC_ASSERT(sizeof(MdEpiArgs) == 120, "MdEpiArgs layout");

/* args.cuh:449-456: dst = a +- (x - t) binv, both parts (sub: minus) */
typedef struct MdEpiToArgs {
    MdEpiArgs m;
    PolyRef a;
    int32_t sub, pad;
} MdEpiToArgs;
PC_STATIC_ASSERT(sizeof(MdEpiToArgs) == 152, "MdEpiToArgs layout");

/* args.cuh:458-467: out = sum_{j < nsrc <= 8} w[j rowstride + row] src_j (both parts), Shoup companions ws */
typedef struct WsumArgs {
    PolyRef out;
    PolyRef src[8];
    const void* w;
    const void* ws;
    const PrimeConst* pr;
    int32_t nsrc, rowstride, n, K;
} WsumArgs;
PC_STATIC_ASSERT(sizeof(WsumArgs) == 256, "WsumArgs layout");

/* args.cuh:469-474: wsum, then part 0 += k[row] (reduced once) */
typedef struct WsumKArgs {
    WsumArgs w;
    const void* k;
} WsumKArgs;
PC_STATIC_ASSERT(sizeof(WsumKArgs) == 264, "WsumKArgs layout");

/* args.cuh:476-489: nout <= 3 weighted sums of one source list: out[m] = sum_j w[m][j rowstride + row] src_j
 * [+ k[m][row] on part 0] on rows [0, n[m]); blocks over rows [0, nmax) */
typedef struct WsumMultiArgs {
    PolyRef out[3];
    PolyRef src[8];
    const void* w[3];
    const void* ws[3];
    const void* k[3];
    const PrimeConst* pr;
    int32_t nout, nsrc, rowstride, K;
    int32_t n[3], nmax;
} WsumMultiArgs;
PC_STATIC_ASSERT(sizeof(WsumMultiArgs) == 376, "WsumMultiArgs layout");

/* args.cuh:491-498: part 0 += k[row] (reduced once) */
typedef struct AddConstArgs {
    PolyRef x;
    const void* k;
    const PrimeConst* pr;
    int32_t n, K;
} AddConstArgs;
PC_STATIC_ASSERT(sizeof(AddConstArgs) == 48, "AddConstArgs layout");

/* args.cuh:500-506: out = in t[row][i] (both parts; t one table of rows of N words) */
typedef struct MulTableArgs {
    PolyRef out, in;
    const void* t;
    const PrimeConst* pr;
    int32_t n, K;
} MulTableArgs;
PC_STATIC_ASSERT(sizeof(MulTableArgs) == 72, "MulTableArgs layout");

/* args.cuh:508-515: out = y + m (sub 0), y - m (1), m - y (2), m = in t as mul_table's; out may alias y or in */
typedef struct MulAddArgs {
    MulTableArgs m;
    PolyRef y;
    int32_t sub, pad;
} MulAddArgs;
PC_STATIC_ASSERT(sizeof(MulAddArgs) == 104, "MulAddArgs layout");

/* args.cuh:517-528: out = y + sum_{j < nterm <= 8} x_j t_j (y.base null: no y), rows [0, n) of K cts, both parts; lazy
 * only chooses the reference's accumulation (the same canonical words either way) */
typedef struct MulAddNArgs {
    PolyRef out, y;
    PolyRef x[8];
    const void* t[8];
    const PrimeConst* pr;
    int32_t n, K, nterm, lazy;
} MulAddNArgs;
PC_STATIC_ASSERT(sizeof(MulAddNArgs) == 328, "MulAddNArgs layout");

/* args.cuh:531-552: the composite one-pass rescale by the top ndrop (1 or 2) primes, a = top, b = top - 1,
 * lift(y, q) = y - q when y > q/2, reduced mod q_i:
 *   ndrop 2: y' = qinv_ab y_b + C_ab lift(y_a) mod q_b;  tmp_i = A_i lift(y_a) + B_i lift(y')
 *   ndrop 1: tmp_i = A_i lift(y_a)
 * on rows i < nrows, coefficient form; ca (cb): the tops scaled first when ca != 1. qam / qbm: q_a, q_b mod q_i. */
typedef struct RescaleArgs {
    PolyRef x, tmp;
    const void* A;
    const void* B;
    const void* As;
    const void* Bs;
    const void* qam;
    const void* qbm;
    const PrimeConst* pr;
    uint64_t qinv_ab, C_ab, ca, cb;
    int32_t top, nrows, K, ndrop;
} RescaleArgs;
PC_STATIC_ASSERT(sizeof(RescaleArgs) == 152, "RescaleArgs layout");

/* args.cuh:554-563: rescale_coef (ndrop 2) and the forward NTT of its rows in one pipeline, the correction never
 * stored: the tops' two sources go to tmp rows top, top - 1, the column pass generates tmp_i from them (the sources
 * sit top - r and top - 1 - r rows above row r of the same polynomial); ntt's epilogue applies (3: the combine) */
typedef struct RescaleNttArgs {
    RescaleArgs rs;
    NttArgs ntt;
} RescaleNttArgs;
PC_STATIC_ASSERT(sizeof(RescaleNttArgs) == 328, "RescaleNttArgs layout");

/* args.cuh:565-572: x_i = alpha_i x_i + tmp_i (NTT domain), both parts */
typedef struct RescaleCombineArgs {
    PolyRef x, tmp;
    const void* alpha;
    const void* alphas;
    const PrimeConst* pr;
    int32_t n, K;
} RescaleCombineArgs;
PC_STATIC_ASSERT(sizeof(RescaleCombineArgs) == 80, "RescaleCombineArgs layout");

/* args.cuh:574-579: out_i = alpha_i x_i + tmp_i, x read only */
typedef struct RescaleCombineToArgs {
    RescaleCombineArgs a;
    PolyRef out;
} RescaleCombineToArgs;
PC_STATIC_ASSERT(sizeof(RescaleCombineToArgs) == 104, "RescaleCombineToArgs layout");

/* args.cuh:162-170: out[i] = a[i] (+ b[i]) (+ c[i]) for n <= 48 polynomials by pointer (rows [0, nrows), row r at
 * + r N); a null b / c is skipped */
#define PC_EWM_MAX 48
typedef struct EwManyArgs {
    void* out[PC_EWM_MAX];
    const void* a[PC_EWM_MAX];
    const void* b[PC_EWM_MAX];
    const void* c[PC_EWM_MAX];
    const PrimeConst* pr;
    int32_t n, nrows;
} EwManyArgs;
PC_STATIC_ASSERT(sizeof(EwManyArgs) == 4 * PC_EWM_MAX * 8 + 16, "EwManyArgs layout");

/* args.cuh:172-182: out[i] = (a[i] - b[i]) t[row] for n <= 48 polynomials by pointer */
typedef struct SubMulManyArgs {
    void* out[PC_EWM_MAX];
    const void* a[PC_EWM_MAX];
    const void* b[PC_EWM_MAX];
    const void* t;
    const PrimeConst* pr;
    int32_t n, nrows;
} SubMulManyArgs;
PC_STATIC_ASSERT(sizeof(SubMulManyArgs) == 3 * PC_EWM_MAX * 8 + 24, "SubMulManyArgs layout");

/* args.cuh:665-676: composite ModRaise, coefficient form: for rows t in [r0, r1) of K ciphertexts (nparts polynomials
 * from part 0), x[t] = sum_{k < d} centred([x_k qhatinv_k]_{q_k}) qhat[k][t] mod q_t, the sources x_k = rows 0..d-1
 * of the same polynomial (each term centred on its own prime; not written) */
typedef struct ModRaiseArgs {
    void* x;
    const PrimeConst* pr;
    uint64_t ct_stride, part_stride;
    uint64_t qhatinv[4];
    uint64_t qhat[4][64];
    int32_t K, d, r0, r1, nparts, pad;
} ModRaiseArgs;
PC_STATIC_ASSERT(sizeof(ModRaiseArgs) == 2136, "ModRaiseArgs layout");

/* args.cuh:678-697: exact small-integer scaling: per coefficient, Garner from the k source rows, centre against Q_k / 2,
 * optionally q = floor((|x| R + 2^191) / 2^192) (R = round(2^192 / D)), reduce modulo every output row orow[o] (prime
 * ids; pow32[o][w] = (2^32)^w mod p), restore the sign. Source primes below 2^31. */
#define PC_SI_MAXK 4
#define PC_SI_MAXW 8
#define PC_SI_MAXR 8
#define PC_SI_SHIFT 192
#define PC_SI_MAXOUT 64
typedef struct SmallIntTab {
    int32_t k, nout, nw, nr, divide, pad;
    uint32_t q[PC_SI_MAXK];
    uint32_t qinv[PC_SI_MAXK][PC_SI_MAXK]; /* qinv[i][j] = q_j^-1 mod q_i, j < i */
    uint32_t Qk[PC_SI_MAXW], Qkh[PC_SI_MAXW];
    uint32_t R[PC_SI_MAXR];
    int32_t orow[PC_SI_MAXOUT];
    uint32_t pow32[PC_SI_MAXOUT][PC_SI_MAXW + PC_SI_MAXR];
} SmallIntTab;
PC_STATIC_ASSERT(sizeof(SmallIntTab) == 4552, "SmallIntTab layout");

/* args.cuh:698-709: source row i of (c, part) at src + c src_ct_stride + part src_part_stride + i N; output row
 * orow[o] at out + c ct_stride + part part_stride + orow[o] N; tab in device memory */
typedef struct SmallIntArgs {
    const void* src;
    void* out;
    const SmallIntTab* tab;
    const PrimeConst* pr;
    uint64_t src_ct_stride, src_part_stride, ct_stride, part_stride;
    int32_t K, nparts;
} SmallIntArgs;
PC_STATIC_ASSERT(sizeof(SmallIntArgs) == 72, "SmallIntArgs layout");

/* args.cuh:890-907: the scaling from one source prime: x = row 0 centred against q0, q = floor((|x| mc + 2^(sh-1)) /
 * 2^sh), row t := sign(x) q mod q_t for t < nrows, in place (row 0 read first); 1 <= sh <= 127, q < 2^64 */
typedef struct SmallInt1Args {
    void* x;
    const PrimeConst* pr;
    uint64_t ct_stride, part_stride;
    uint64_t mc;
    int32_t sh, nrows, K, nparts;
} SmallInt1Args;
PC_STATIC_ASSERT(sizeof(SmallInt1Args) == 56, "SmallInt1Args layout");

/* args.cuh:184-198: the BSGS plaintext dot of a stage in the extended basis, K <= 8 ciphertexts sharing the diagonals:
 * res[c][j][part] = sum_{i < bstep} rot[c][i][part] pt[bstep j + i] (j < gstep, diagonals >= npts skipped); rot (c, i)
 * at rot.base + c rot.ct_stride + i rot_stride, res (c, j) at res.base + c res.ct_stride + j res_stride; pts[d]: the
 * diagonal's rows (ptw words each; Q rows, then the special rows from pt_prow), read at the compact index (enc as
 * CtsArgs.enc). res must not overlap rot: past 8 baby steps the sums of later groups of rotations are added onto the
 * results stored by the earlier groups, so a result row written over a rotation not yet read would feed it back. */
typedef struct PtDotArgs {
    PolyRef rot, res;
    uint64_t rot_stride, res_stride;
    const void* const* pts;
    const PrimeConst* pr;
    RowSet rs;
    int32_t npts, bstep, gstep, K;
    int32_t ptw, pt_prow;
    uint32_t enc;
    int32_t pad;
} PtDotArgs;
PC_STATIC_ASSERT(sizeof(PtDotArgs) == 128, "PtDotArgs layout");

/* args.cuh:230-241: the subring switch's split, coefficient form: row y of polynomial c (q + c q_stride + y N for
 * y < nq, else p + c p_stride + (y - nq) N) into sub digits, digit j = the coefficients at the exponents = j mod sub
 * (the rest 0), written at out + c out_stride + (j nrows + y) N */
typedef struct PackSplitArgs {
    const void* q;
    const void* p;
    void* out;
    uint64_t q_stride, p_stride, out_stride;
    int32_t K, sub, nq, nrows;
} PackSplitArgs;
PC_STATIC_ASSERT(sizeof(PackSplitArgs) == 64, "PackSplitArgs layout");

/* args.cuh:243-259: the subring switch's dot, evaluation form: s1 = sum_j D_j a_j, s0 = sum_j D_j b_j (+ pmod c0 on
 * the Q rows y < nq), row y at prime id rows[y]; D as pack_split's out (dig, dig_stride), kb / ka [digit][row y][N];
 * c0 and the outputs in prime-id rows, polynomial c at + c ct_stride / + c out_ct_stride */
typedef struct PackDotArgs {
    const void* dig;
    const void* kb;
    const void* ka;
    const void* c0;
    void* out0;
    void* out1;
    const uint32_t* rows;
    const void* pmod;
    const void* pmods;
    const PrimeConst* pr;
    uint64_t dig_stride, ct_stride, out_ct_stride;
    int32_t K, sub, nq, nrows;
} PackDotArgs;
PC_STATIC_ASSERT(sizeof(PackDotArgs) == 120, "PackDotArgs layout");

/* args.cuh:906-927 (coeff_sum, ABI 9): streamed-weight inner sum out (+)= sum_{r < n} ct[r] pt_r over Q limbs
 * 0..L-1 (prime id = limb), pt_r = NTT(round(rows[r] scale) mod p): round half to even, a product of magnitude
 * 9.2e18 or more clamped to +-2^62 and counted in *overflow (when non-null) once per limb and coefficient. ct[r], out:
 * part 0 row 0 of a ciphertext (part 1 at + part_stride words, row l at + l N); rows[r]: N float32 coefficients in
 * device memory; scratch: n L N words (left holding the NTT'd plaintexts). n in [1, MAXT], L in [1, MAXL]. */
#define PC_COEFF_MAXT 32
#define PC_COEFF_MAXL 64
typedef struct CoeffArgs {
    void* scratch;
    void* out;
    const void* fw;
    const void* fws;
    const PrimeConst* pr;
    unsigned long long* overflow;
    uint64_t part_stride;
    double scale;
    int32_t n, L, accumulate, pad;
    const float* rows[PC_COEFF_MAXT];
    const void* ct[PC_COEFF_MAXT];
} CoeffArgs;
PC_STATIC_ASSERT(sizeof(CoeffArgs) == 80 + 16 * PC_COEFF_MAXT, "CoeffArgs layout");

/* args.cuh:407-436 (tensor_seeded, ABI 27-28): tensor_multi over seeded first operands that share their second ones,
 * single ciphertexts, rows [0, n): output q nout + o = sum_{j < npairs} a[o][j] * set q's j-th second operand (set 0:
 * b[j]; set q > 0: bq[q - 1][j] with b[j]'s strides); c0, c1 into out[], d2 into part 1 of d2[]; acc as
 * tensor_sum's (nonzero: onto out's c0, c1; bit 1: onto d2). a[o][j] is a seeded ciphertext's c0, row r at r N words
 * (packed: r PC_PACK_ROW_WORDS words, 28 bits per coefficient, one little-endian bit stream per row); its rows' 8-word
 * seeds at a[o][j] + seed_off + 8 r; its c1 word (row, slot) is drawn in the kernel by the "CTSA" expander
 * (crates/pc-core/src/keys.rs:580-630). cout and swords only schedule the reference's blocks; here they are ignored.
 * Every sum is reduced exactly (no lazy bound on the pairs). u32 words only. */
#define PC_PACK_BITS 28
#define PC_TSEED_OUT 16
#define PC_TSEED_PAIRS 128
#define PC_TSEED_Q 4
#define PC_TSEED_QOUT 64
typedef struct TensorSeededArgs {
    PolyRef out[PC_TSEED_QOUT], d2[PC_TSEED_QOUT];
    PolyRef b[PC_TSEED_PAIRS];
    const void* a[PC_TSEED_OUT][PC_TSEED_PAIRS];
    const PrimeConst* pr;
    uint64_t seed_off;
    int32_t nout, npairs, acc, n, packed, pad;
    const void* bq[PC_TSEED_Q - 1][PC_TSEED_PAIRS];
    int32_t nq, cout, swords, qpad;
} TensorSeededArgs;
PC_STATIC_ASSERT(sizeof(TensorSeededArgs) == (2 * PC_TSEED_QOUT + PC_TSEED_PAIRS) * 24 + PC_TSEED_OUT * PC_TSEED_PAIRS * 8 +
                                                 16 + 24 + (PC_TSEED_Q - 1) * PC_TSEED_PAIRS * 8 + 16,
                 "TensorSeededArgs layout");

/* args.cuh:726-734 (spru_fft_pass, ABI 3): one forward Stockham pass of half-size ns over batch size-N complex
 * transforms (transform e at in/out + e N double2; in and out distinct), twiddle table tw of N/2 double2 with
 * tw[m] = exp(-i pi m / (N/2)). Output pair (idx, idx + ns), idx = (j / ns) 2 ns + j % ns, for j < N/2:
 * v0 +- t with t = v1 w, w = tw[(j % ns) (N/2) / ns], as the reference compiles it:
 * t.x = fma(v1.x, w.x, -(v1.y w.y)), t.y = fma(v1.y, w.x, v1.x w.y), every other product and sum rounded alone.
 * Replaces crates/pc-host/src/spru.rs:83-107 spru_fft_pass. ns a power of two in [1, N/2] (the reference checks
 * only the range), batch >= 1. */
typedef struct SpruFftArgs {
    const void* in;
    void* out;
    const void* tw;
    int32_t ns, batch;
} SpruFftArgs;
PC_STATIC_ASSERT(sizeof(SpruFftArgs) == 32, "SpruFftArgs layout");

/* args.cuh:735-746 (spru_scatter, ABI 3): coefficients of batch FFT outputs y (transform e at y + e N double2):
 * m_k = rint(fma(y.x, zt.x, -(y.y zt.y)) 2^-logN scale) (round half to even), zt[k] = exp(-i pi k / N), reduced into
 * limbs l < nl (prime ids 0..nl-1) at out + e out_stride + l N words, coefficient form. Replaces
 * crates/pc-host/src/spru.rs:110-140 spru_scatter. |m_k| < 2^63 is the caller's guarantee, as in the reference. */
typedef struct SpruScatterArgs {
    const void* y;
    void* out;
    const void* zt;
    const PrimeConst* pr;
    double scale;
    int32_t nl, batch;
    uint64_t out_stride;
} SpruScatterArgs;
PC_STATIC_ASSERT(sizeof(SpruScatterArgs) == 56, "SpruScatterArgs layout");

/* Argument structs of the table entries this library does not implement (their launchers return -1): declared
 * only. */
/* args.cuh:595-611 (encode): N/2 complex slots v (re, im doubles) -> coefficient-form rows out[l][N], l < nl
 * (prime id l): slot j at zeta^(5^j) and its conjugate, an N-point DFT in double, c_k = scale Re(Y_k zeta^-k) / N and
 * max |c_k|, OpenFHE's 2^61 split, residues times deg_factor[l] (round(scale)^(deg - 1) mod p_l) and 2^split.
 * Workspaces: a, b N double2 each, c N doubles, cmax one u64. */
typedef struct EncodeArgs {
    const void* v;
    void* a;
    void* b;
    void* c;
    unsigned long long* cmax;
    void* out;
    const void* deg_factor;
    const PrimeConst* pr;
    double scale;
    int32_t nl, pad;
} EncodeArgs;
PC_STATIC_ASSERT(sizeof(EncodeArgs) == 80, "EncodeArgs layout");
struct SpruExtractArgs;
struct PcmmArgs;
struct CcmmArgs;
struct TfheArgs;

/* args.cuh:1035-1097 */
typedef struct KernelTable {
    uint32_t abi;
    uint32_t word_bytes;
    uint32_t mm;
    uint32_t log_n;
    int (*ntt_fwd)(const NttArgs*, pc_stream_t);
    int (*ntt_inv)(const NttArgs*, pc_stream_t);
    int (*bconv)(const BconvArgs*, pc_stream_t);
    int (*ew_add)(const EwArgs*, pc_stream_t);
    int (*ew_scale)(const EwArgs*, pc_stream_t);
    int (*ew_sub_mul)(const EwArgs*, pc_stream_t);
    int (*ew_copy)(const EwArgs*, pc_stream_t);
    int (*pt_dot)(const struct PtDotArgs*, pc_stream_t);
    int (*ks_dot)(const KsArgs*, pc_stream_t);
    int (*ks_dot_regen)(const KsRegenArgs*, pc_stream_t);
    int (*ksk_expand)(const KskExpandArgs*, pc_stream_t);
    int (*cts_fused)(const CtsArgs*, pc_stream_t);
    int (*tensor)(const struct TensorArgs*, pc_stream_t);
    int (*md_epilogue)(const struct MdEpiArgs*, pc_stream_t);
    int (*wsum)(const struct WsumArgs*, pc_stream_t);
    int (*add_const)(const struct AddConstArgs*, pc_stream_t);
    int (*mul_table)(const struct MulTableArgs*, pc_stream_t);
    int (*rescale_coef)(const struct RescaleArgs*, pc_stream_t);
    int (*rescale_combine)(const struct RescaleCombineArgs*, pc_stream_t);
    int (*automorph)(const AutomorphArgs*, pc_stream_t);
    int (*encode)(const struct EncodeArgs*, pc_stream_t);
    int (*encrypt)(const EncryptArgs*, pc_stream_t);
    int (*ksk_gen)(const KskGenArgs*, pc_stream_t);
    int (*ksk_unpack)(const KskUnpackArgs*, pc_stream_t);
    int (*mod_raise)(const struct ModRaiseArgs*, pc_stream_t);
    int (*small_int)(const struct SmallIntArgs*, pc_stream_t);
    int (*spru_extract)(const struct SpruExtractArgs*, pc_stream_t);
    int (*spru_fft_pass)(const struct SpruFftArgs*, pc_stream_t);
    int (*spru_scatter)(const struct SpruScatterArgs*, pc_stream_t);
    int (*cts_fused_regen)(const CtsRegenArgs*, pc_stream_t);
    int (*ks_dot_key)(const KsKeyArgs*, pc_stream_t);
    int (*pcmm)(const struct PcmmArgs*, pc_stream_t);
    int (*ccmm)(const struct CcmmArgs*, pc_stream_t);
    int (*wsum_k)(const struct WsumKArgs*, pc_stream_t);
    int (*rescale_combine_to)(const struct RescaleCombineToArgs*, pc_stream_t);
    int (*md_epilogue_to)(const struct MdEpiToArgs*, pc_stream_t);
    int (*small_int1)(const struct SmallInt1Args*, pc_stream_t);
    int (*coeff_sum)(const struct CoeffArgs*, pc_stream_t);
    int (*mul_add)(const struct MulAddArgs*, pc_stream_t);
    int (*rescale_fwd)(const struct RescaleNttArgs*, pc_stream_t);
    int (*mul_add_n)(const struct MulAddNArgs*, pc_stream_t);
    int (*tensor_y)(const struct TensorYArgs*, pc_stream_t);
    int (*wsum_multi)(const struct WsumMultiArgs*, pc_stream_t);
    int (*bconv_wide)(const BconvArgs*, pc_stream_t);
    int (*tfhe)(const struct TfheArgs*, pc_stream_t);
    int (*tensor_sum)(const struct TensorSumArgs*, pc_stream_t);
    int (*tensor_multi)(const struct TensorMultiArgs*, pc_stream_t);
    int (*tensor_seeded)(const struct TensorSeededArgs*, pc_stream_t);
    int (*ew_many)(const struct EwManyArgs*, pc_stream_t);
    int (*submul_many)(const struct SubMulManyArgs*, pc_stream_t);
    int (*pack_split)(const struct PackSplitArgs*, pc_stream_t);
    int (*pack_dot)(const struct PackDotArgs*, pc_stream_t);
} KernelTable;
PC_STATIC_ASSERT(sizeof(KernelTable) == 16 + 52 * 8, "KernelTable layout");

/* The u32 x Barrett64 table at N = 2^16 (instantiate.inc:32-91; header {abi 30, word_bytes 4, mm 0, log_n 16}). */
const KernelTable* pc_table_u32_barrett64(void);
/* The same kernels at N = 2^log_n, log_n in [12, 16] (the header's log_n field says which). No counterpart in the
 * reference, whose table is fixed at 2^16 (args.cuh:14-18): it exists for ring degrees such as 2^14. NULL outside
 * the range. */
const KernelTable* pc_table_u32_logn(uint32_t log_n);

/* ------------------------------------------------------------------------------------------ runtime FFI */
/* crates/pc-cuda/src/ffi.rs:18-50 and mem.rs:19-24: each returns 0 or a positive HIP error code */
int pc_hip_device_count(int* n);
int pc_hip_set_device(int dev);
int pc_hip_device_name(int dev, char* out, int len);
/* cudaRuntimeGetVersion / cudaDriverGetVersion (crates/pc-cuda/src/device.rs:83-84, Device::open): HIP's numbers */
int pc_hip_runtime_version(int* v);
int pc_hip_driver_version(int* v);
/* cudaDeviceGetAttribute (device.rs:115 sm_count, :126 clusters). attr takes the cudaDeviceAttr numbers the reference
 * passes (16: compute units; 75 / 76: the gfx major / minor HIP reports, 9 / 5 on gfx950), PC_HIP_ATTR_CLUSTERS (0:
 * CDNA has no thread-block clusters, the value Device::clusters should read) and PC_HIP_ATTR_GFX_ARCH (the gfx code as
 * hexadecimal digits, 0x950); also 13, the peak shader clock in kHz (cudaDevAttrClockRate's number; the reference
 * does not read it). Any other attr: hipErrorInvalidValue. */
#define PC_HIP_ATTR_CLOCK_KHZ 13
#define PC_HIP_ATTR_CU_COUNT 16
#define PC_HIP_ATTR_CC_MAJOR 75
#define PC_HIP_ATTR_CC_MINOR 76
#define PC_HIP_ATTR_CLUSTERS 0x10000
#define PC_HIP_ATTR_GFX_ARCH 0x10001
int pc_hip_device_attribute(int* v, int attr, int dev);
/* cudaMemGetInfo (device.rs:137 mem_info, :188 mem_info_current): free and total bytes of the current device */
int pc_hip_mem_get_info(size_t* free_bytes, size_t* total_bytes);
/* cudaProfilerStart / cudaProfilerStop (device.rs:151-158 profiler): synchronise the device, then ask a running
 * rocprofv3 to resume / pause collection (roctx, its --selected-regions mode); a no-op without a profiler */
int pc_hip_profiler_start(void);
int pc_hip_profiler_stop(void);
int pc_hip_malloc(void** p, size_t bytes);
int pc_hip_free(void* p);
int pc_hip_malloc_host(void** p, size_t bytes);
int pc_hip_free_host(void* p);
int pc_hip_memcpy_htod(void* dst, const void* src, size_t bytes, pc_stream_t s);
int pc_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes, pc_stream_t s);
int pc_hip_memcpy_dtod(void* dst, const void* src, size_t bytes, pc_stream_t s);
/* cudaMemsetAsync (crates/pc-cuda/src/mem.rs:305-331): the low byte of value into bytes bytes from dst, any alignment,
 * enqueued on s as a fill kernel (so a captured replay holds no memset node) */
int pc_hip_memset(void* dst, int value, size_t bytes, pc_stream_t s);
int pc_hip_stream_create(pc_stream_t* s);
/* cudaDeviceGetStreamPriorityRange / cudaStreamCreateWithPriority (stream.rs:33-44, Stream::high_priority): every
 * stream of this library runs at the default priority (mixed-priority streams have been seen to stall on MI355X), so
 * the range reads (0, 0) and the priority argument is accepted and not applied */
int pc_hip_stream_priority_range(int* least, int* greatest);
int pc_hip_stream_create_with_priority(pc_stream_t* s, int priority);
int pc_hip_stream_destroy(pc_stream_t s);
int pc_hip_stream_sync(pc_stream_t s);
int pc_hip_stream_wait_event(pc_stream_t s, void* ev);
int pc_hip_device_sync(void);
int pc_hip_event_create(void** ev);
/* cudaEventCreateWithFlags (stream.rs:146): flags 0 (a timing event, Event::timing) or PC_HIP_EVENT_DISABLE_TIMING
 * (ordering only, Event::new); other bits: hipErrorInvalidValue */
#define PC_HIP_EVENT_DISABLE_TIMING 2
int pc_hip_event_create_flags(void** ev, unsigned flags);
int pc_hip_event_destroy(void* ev);
int pc_hip_event_record(void* ev, pc_stream_t s);
int pc_hip_event_sync(void* ev);
int pc_hip_event_elapsed_ms(float* ms, void* start, void* stop);
int pc_hip_graph_begin_capture(pc_stream_t s);
int pc_hip_graph_end_capture(pc_stream_t s, void** graph);
int pc_hip_graph_instantiate(void** exec, void* graph);
int pc_hip_graph_launch(void* exec, pc_stream_t s);
int pc_hip_graph_destroy(void* graph);
int pc_hip_graph_exec_destroy(void* exec);
const char* pc_hip_error_string(int code);
/* cudaGetErrorName (crates/pc-cuda/src/error.rs:29-32): the code's symbolic name */
const char* pc_hip_error_name(int code);
/* the last launch error of the calling thread (hipGetLastError), 0 if none */
int pc_hip_last_error(void);

/* ------------------------------------------------------------------------------------------ driver (pc-gpu) */
/* A context: one chain (nq Q primes then kp special primes, all < 2^31 and = 1 mod 2N), N = 2^log_n, dnum hybrid
 * digits of ceil(nq / dnum) limbs (crates/pc-core/src/params.rs:500-510), and device tables: prime constants, twiddles
 * (crates/pc-gpu/src/context.rs:169-261), key-switching plans of every limb top (crates/pc-gpu/src/ks.rs:521-828) and
 * a workspace for up to k_rot extended ciphertexts per hoisted chunk. Errors: NULL, with *err set. */
typedef struct pcx_ctx pcx_ctx;
pcx_ctx* pcx_ctx_new(uint32_t log_n, const uint64_t* primes, int nq, int kp, int dnum, int k_rot, int* err);
/* pcx_ctx_new with plans and workspace for K-ciphertext ModUps, products and rescales, K <= k_max <= 8 (the
 * reference's k_max, crates/pc-gpu/src/ops.rs:1554-1595: K ciphertexts per launch; a product's key dot takes at most
 * 4); pcx_ctx_new is k_max 1. */
pcx_ctx* pcx_ctx_new_k(uint32_t log_n, const uint64_t* primes, int nq, int kp, int dnum, int k_rot, int k_max,
                       int* err);
void pcx_ctx_free(pcx_ctx* c);
const KernelTable* pcx_ctx_table(const pcx_ctx* c);
const PrimeConst* pcx_ctx_primes(const pcx_ctx* c); /* device table by prime id */
/* device twiddle tables [prime id][N]: fw, fws, iw, iws, then ninv, ninvs [prime id] */
const void* pcx_ctx_twiddle(const pcx_ctx* c, int which);
uint64_t pcx_ctx_root(const pcx_ctx* c, int prime_id);
size_t pcx_ctx_workspace_bytes(const pcx_ctx* c);
/* Every launch of the context's operations through the kernel table alone, as crates/pc-gpu issues them (on != 0):
 * the ModDown conversion as the table's bconv then ntt_fwd with its epilogue, the key dots as ks_dot_key (a key
 * group's retry-value table unused); off: the driver's fused forms. Returns the previous setting, -1 on NULL. */
int pcx_ctx_table_only(pcx_ctx* c, int on);
/* No counterpart in the reference: a tuning switch. Which conversions the driver streams into the forward NTT's
 * column pass instead of the table's bconv then ntt_fwd: bit 0 the ModUp, bit 1 the ModDown the register-held fused
 * form does not take (more than 6 special primes), bit 2 the ModDown-rescale (default 3, or PCX_CC_FUSED at context
 * creation; the table-only mode uses none). mask < 0 reads the setting. Returns the previous mask, -1 on NULL. The
 * words are the same either way. */
int pcx_ctx_conv_fusion(pcx_ctx* c, int mask);

/* No counterpart in the reference: a tuning switch. Launches of N = 2^16 with at least `rows` rows take the one-pass
 * transform (one workgroup per row) instead of the two-pass one; 0 (the default, or PCX_NTT1_MIN) never. Returns the
 * previous threshold. The words are the same either way. */
int pcx_ntt_one_pass_min(int rows);
/* Batched NTT of nrows rows of one buffer: row i at base + roff[i]*N (prime id ids[i]); host row tables are uploaded
 * into a device row list made once (crates/pc-gpu/src/ntt.rs:293-326 transform_rows over a RowList). dir: 1 forward,
 * -1 inverse (scaled by N^-1). */
typedef struct pcx_rows pcx_rows;
pcx_rows* pcx_rows_new(pcx_ctx* c, const uint32_t* roff, const int32_t* ids, int nrows);
void pcx_rows_free(pcx_rows* r);
int pcx_ntt(pcx_ctx* c, int dir, void* base, const pcx_rows* rows, pc_stream_t s);

/* A key group: R rotation keys (galois elements g_r), each a 256-bit KSKA seed of `a` plus its stored `b`
 * [dnum][nq + kp][N] (full layout: slot = prime id), dense (bits = 0) or bit-packed at `bits` per value
 * (crates/pc-gpu/src/keys.rs:24-70). The host b arrays are uploaded (and packed) once. */
typedef struct pcx_keys pcx_keys;
pcx_keys* pcx_keys_new(pcx_ctx* c, int nkeys, const uint64_t* galois, const uint32_t* seeds,
                       const uint32_t* const* b_host, int bits, int* err);
/* A banded key group (crates/pc-gpu/src/keys.rs:81-103 KskShape::banded, :351-376 KeySetSpec::with_band): every key
 * stores digits 0..ndig (each digit whose first prime id is <= q_top, ndig = q_top / ceil(nq / dnum) + 1), each the Q
 * rows 0..=q_top then the kp special rows: host b [ndig][q_top + 1 + kp][N] per key. Its `a` is the full key's (the
 * KSKA words depend on the seed, digit and prime only), so the band is the full key's rows restricted. The group
 * serves ciphertexts at top <= q_top; an operation at a higher top returns -1. Its dots go through the kernel
 * table's in-place reads of the stored slots (KeyTab.q_top, srows); no retry-value table is built. q_top = nq - 1 is
 * pcx_keys_new. Special primes: all kp of the chain (chains with fewer special primes at low tops are not built). */
pcx_keys* pcx_keys_new_banded(pcx_ctx* c, int nkeys, const uint64_t* galois, const uint32_t* seeds,
                              const uint32_t* const* b_host, int bits, int q_top, int* err);
/* the highest ciphertext top the group serves (nq - 1 for full keys), -1 on NULL */
int pcx_keys_q_top(const pcx_keys* k);
/* The host sampler of key generation (perseus_amd/csrc/drbg.cpp): the DRBG of crates/pc-core/src/keys.rs:113-232
 * (Prng: ChaCha20, a 64-bit block counter in state words 12..13, word 14 the stream id, word 15 "DRBG"; from_seed,
 * next_u32, ksk_seed), the sparse ternary secret (keys.rs:245-262 sample_sparse_ternary: -1 when h > n) and the
 * discrete Gaussian (keys.rs DiscreteGaussian: inversion of the CDF on |x| <= ceil(14 sigma), one uniform double then
 * a sign word when x != 0; -1 for sigma outside (0, 1e6)). A host object, not thread-safe. */
typedef struct pcx_drbg pcx_drbg;
pcx_drbg* pcx_drbg_new(const uint32_t key[8], uint32_t stream);
void pcx_drbg_free(pcx_drbg* g);
uint32_t pcx_drbg_u32(pcx_drbg* g);
int pcx_drbg_ksk_seed(pcx_drbg* g, uint32_t out[8]);
int pcx_drbg_sparse_ternary(pcx_drbg* g, uint32_t n, uint32_t h, int8_t* out);
int pcx_drbg_gaussian(pcx_drbg* g, double sigma, uint32_t n, int64_t* out);
/* The host draws of nkeys switching keys in crates/pc-gpu/src/keygen.rs:193-210 (generate_with) order: per key its seed
 * (8 words of g), the key of its per-digit error streams (8 more), then digit d's n errors from the stream (that key,
 * d). seeds[nkeys][8], errors[nkeys][ndig][n]: pcx_keys_generate's inputs. */
int pcx_keygen_draw(pcx_drbg* g, int nkeys, int ndig, uint32_t n, double sigma, uint32_t* seeds, int64_t* errors);
/* Keys generated on the device (crates/pc-gpu/src/keygen.rs:172-262): secret s (ternary coefficients), per key the
 * seed of a and the Gaussian errors e[dnum][N] (signed coefficients, the same error on every limb of a digit). */
pcx_keys* pcx_keys_generate(pcx_ctx* c, int nkeys, const uint64_t* galois, const int8_t* secret,
                            const uint32_t* seeds, const int64_t* errors, int bits, int* err);
void pcx_keys_free(pcx_keys* k);
/* bytes of the group's KSKA retry-value table (dense keys: the accepted redraws of the rejected ChaCha words, built
 * when the keys are made and read by the dot instead of redrawing them; about 1-2% of b at 31-bit primes); 0 if none.
 * No counterpart in the reference, whose dot redraws in the kernel (as the table entry ks_dot_key does here). */
size_t pcx_keys_patch_bytes(const pcx_keys* k);
/* Keys with a resident dense `a` (crates/pc-gpu/src/ks.rs:346-347, 408-411, 1259-1262 set_regen_digits: a group that stores `a` regenerates its
 * digits below regen_digits and reads the rest, KeyTab.nregen): the first call expands every key's `a` on the device
 * into [dnum][nq + kp][N] words per key (pcx_keys_resident_bytes); later calls only change regen_digits (>= dnum:
 * every digit regenerated again). Memory for VALU work: each resident digit trades one ChaCha12 block per 16 slots for
 * 64 bytes of HBM reads. Full-layout groups only (-1 for a band or a negative count); s: the expansion's stream
 * (synchronised before returning). */
int pcx_keys_resident_a(pcx_keys* k, int regen_digits, pc_stream_t s);
size_t pcx_keys_resident_bytes(const pcx_keys* k);
/* download key r's stored b as dense words [ndig][srows][N] (full keys: [dnum][nq + kp][N]) */
int pcx_keys_download_b(pcx_keys* k, int r, uint32_t* b_host);

/* Ciphertexts are device buffers in the context layout [part][row = prime id over Q u P][N] words (2 (nq+kp) N words;
 * crates/pc-gpu/src/poly.rs:1-53), Q rows 0..top live. */
size_t pcx_ct_words(const pcx_ctx* c);
/* out = rot(ct) by key r of the group (g = 1: a copy): ModUp, key dot, ModDown (crates/pc-gpu/src/rotate.rs:179-204) */
int pcx_rotate(pcx_ctx* c, pcx_keys* k, int r, const void* ct, int top, void* out, pc_stream_t s);
/* hoisted rotations (crates/pc-gpu/src/rotate.rs:456-507): one ModUp, then the keys idx[0..n) in chunks of at most
 * k_rot, output j at out + j * ct_words (words) */
int pcx_rotate_hoisted(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* ct, int top, void* out,
                       pc_stream_t s);
/* out = onto + sum_j rot(ct, key idx[j]) (crates/pc-gpu/src/rotate.rs:692-776 rotate_sum_core, InModDown form): ModUp
 * once, the key dots summed in the extended basis (runs of consecutive keys through the table's ks_dot_key with
 * KS_SUM, later runs added with KS_ACC), then ONE ModDown whose epilogue adds onto `onto` (onto == out: in place;
 * NULL: out = the sum alone). No key of the sum may be the identity (-1). */
int pcx_rotate_sum(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* ct, int top, void* out,
                   const void* onto, pc_stream_t s);
/* out = onto + sum_j rot(cts[j], key idx[j]): the giant-step sum of a BSGS linear transform over n distinct ciphertexts
 * (crates/pc-gpu/src/bts/cts.rs:958-971, the Horner sums kept in the extended basis; rotate.rs:692-776 for the sum's
 * ModDown): a ModUp of each input, its key dot added onto one extended sum (KS_ACC after the first), then ONE ModDown
 * whose epilogue adds onto `onto` (onto == out: in place; NULL: the sum alone). cts: a HOST array of n device
 * ciphertexts. No key may be the identity (-1). */
int pcx_rotate_many(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* const* cts, int top, void* out,
                    const void* onto, pc_stream_t s);
/* pcx_rotate_many then the two-prime rescale, fused into its ModDown (B = P q_top q_{top-1}, the exact conversion of
 * crates/pc-gpu/src/bts/cts.rs:740-751, LtEnd::FusedRescale, applied to the extended sum + P onto): out's Q rows
 * 0..top - 2 = round((P onto + sum) / B). top >= 2; onto NULL or a ciphertext at top (may alias out). */
int pcx_rotate_many_rescale(pcx_ctx* c, pcx_keys* k, const int* idx, int n, const void* const* cts, int top,
                            void* out, const void* onto, pc_stream_t s);
/* The rotate-and-sum ladder (crates/pc-gpu/src/rotate.rs:924-992): out = the sum of x over its rotations by every
 * multiple of start below stop (start < 0: the negative steps), rung by rung (out += rot(out, gap), gap doubling), or
 * radix_bits >= 2 rungs at a time through pcx_rotate_sum when the group holds every step of the rung. tmp: a scratch
 * ciphertext. The group must hold the key of every step the ladder takes (-1 otherwise). */
int pcx_rotate_and_sum(pcx_ctx* c, pcx_keys* k, const void* x, int top, int64_t start, int64_t stop, int radix_bits,
                       void* out, void* tmp, pc_stream_t s);
/* pcx_rotate_and_sum of K consecutive ciphertexts (x, out and tmp each K ciphertexts, ct_words apart; K <= the
 * context's k_max and k_rot): when every rung is a radix rung (2 to 8 bits) whose steps the group holds, the K go
 * rung by rung together, each rung one ModUp launch sequence and one ModDown for the K (the reference's K-ciphertext
 * launches, crates/pc-gpu/src/ops.rs:1554-1595); otherwise each takes pcx_rotate_and_sum. Each output's words are
 * those of the one-ciphertext ladder. */
int pcx_rotate_and_sum_k(pcx_ctx* c, pcx_keys* k, const void* x, int top, int64_t start, int64_t stop,
                         int radix_bits, void* out, void* tmp, int K, pc_stream_t s);
/* No counterpart in the reference: pcx_rotate_and_sum for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation). The scratch ciphertext is a file-scope device
 * array of PCX_NOALLOC_SCRATCH_WORDS u32 words (32 MiB per device, held until the process ends) instead of tmp; the
 * call allocates nothing. -2 when the context's ciphertext (pcx_ct_words) exceeds the array or radix_bits > 8; other
 * arguments and errors as pcx_rotate_and_sum. Calls that overlap on one device (another stream, another thread) race
 * on the shared array. */
#define PCX_NOALLOC_SCRATCH_WORDS (2u * 64u * 65536u)
int pcx_rotate_and_sum_noalloc(pcx_ctx* c, pcx_keys* k, const void* x, int top, int64_t start, int64_t stop,
                               int radix_bits, void* out, pc_stream_t s);
/* One CtS / StC stage's hoisted baby steps and plaintext products (crates/pc-gpu/src/bts/cts.rs:840-960, LtStage::run
 * steps 1 and 2): ModUp of ct's c1 once, then through the table's cts_fused_regen
 *   res_j = sum_{i < B} rot_i(ct) pt_{B j + i},  j < G,
 * in the extended basis (Q rows 0..top and the special rows), rot_0 = P ct and rot_i (i >= 1) the key switch before
 * ModDown by key r0 + i - 1 of the group, its `a` regenerated in the kernel. pts: a DEVICE array of npts device
 * pointers to diagonals of top + 1 + kp rows (Q rows 0..top, then the special rows) of ptw words; enc the compact index
 * map (0xFFFFFFFF: full rows; 0x7F000000 | s: o >> s; else o & enc). res: G extended ciphertexts, res_j at
 * res + j ct_words. */
int pcx_cts_stage(pcx_ctx* c, pcx_keys* k, int r0, int B, int G, const void* const* pts, int npts, int ptw,
                  uint32_t enc, const void* ct, int top, void* res, pc_stream_t s);
/* pcx_cts_stage's words by the hoisted route (no counterpart in the reference, whose stage fuses the babies' key
 * products with the diagonal products): rot_0 = P ct (the table's ew_scale, special rows zeroed), one ModUp and one
 * key-dot launch for the B - 1 babies (each key regenerated once) into rot's extended ciphertexts 1..B-1, then the
 * table's pt_dot over Q rows 0..top and the special rows. rot: B extended ciphertexts of workspace (ct_words apart). */
int pcx_cts_stage_hoisted(pcx_ctx* c, pcx_keys* k, int r0, int B, int G, const void* const* pts, int npts, int ptw,
                          uint32_t enc, const void* ct, int top, void* rot, void* res, pc_stream_t s);
/* pcx_moddown of m <= k_rot extended ciphertexts (ct_words apart) into m ciphertexts in one launch sequence (no
 * counterpart in the reference beyond its k_max batching of ModDown). */
int pcx_moddown_k(pcx_ctx* c, void* ext, int top, void* out, int m, pc_stream_t s);
/* The relinearization key s^2 -> s (crates/pc-gpu/src/keygen.rs:225-226): one key of galois 1 generated as
 * pcx_keys_generate's, its old secret squared in the kernel (KskGenArgs.sq). */
pcx_keys* pcx_keys_relin(pcx_ctx* c, const int8_t* secret, const uint32_t* seed, const int64_t* errors, int bits,
                         int* err);
/* Rescale by the top ndrop (1 or 2) primes (crates/pc-gpu/src/rescale.rs:318-440 Rescaler::rescale): out's Q rows
 * 0..top - ndrop = the rescale of ct's rows 0..top, both parts in the evaluation domain, the same words as dropping
 * the primes one at a time; out's rows above are scratch. Two primes run the table's rescale_fwd (the corrections
 * generated in the forward NTT), one prime rescale_coef and the NTT. out may be ct. */
int pcx_rescale(pcx_ctx* c, const void* ct, int top, int ndrop, void* out, pc_stream_t s);
/* pcx_rescale of K <= k_max consecutive ciphertexts (ct_words apart) in the same launches; each ciphertext's words
 * are those of pcx_rescale on it alone. */
int pcx_rescale_k(pcx_ctx* c, const void* ct, int top, int ndrop, void* out, int K, pc_stream_t s);
/* The relinearized product (crates/pc-gpu/src/relin.rs:213-235 mult): the tensor (c0, c1, d2), then d2 key-switched
 * by key 0 of k (the relinearization key: galois 1) and added: out = (c0, c1) + ModDown(dot(ModUp(d2))) on Q rows
 * 0..top (degree 2, rescale pending). out may be a or b. */
int pcx_mul_relin(pcx_ctx* c, pcx_keys* k, const void* a, const void* b, int top, void* out, pc_stream_t s);
/* pcx_mul_relin then the two-prime rescale, fused into one ModDown by B = P q_top q_{top-1} (the exact conversion of
 * crates/pc-gpu/src/bts/cts.rs:740-751, LtEnd::FusedRescale, applied to x + P (d0, d1)): out's Q rows 0..top - 2 =
 * round((P (d0, d1) + KS(d2)) / B). top >= 2. out may alias a or b. */
int pcx_mul_relin_rescale(pcx_ctx* c, pcx_keys* k, const void* a, const void* b, int top, void* out, pc_stream_t s);
/* pcx_mul_relin_rescale of K <= k_max pairs: a, b and out each K consecutive ciphertexts (ct_words apart), product k
 * = a_k b_k, every stage one launch for the K (the tensor, ModUp, key dot and fused ModDown-rescale of
 * crates/pc-gpu/src/relin.rs:213-235 at K ciphertexts); each product's words are those of the K = 1 call. twice
 * nonzero: the tensor's outputs doubled (its dbl, args.cuh TensorArgs), the words of the product of 2a and b. */
int pcx_mul_relin_rescale_k(pcx_ctx* c, pcx_keys* k, const void* a, const void* b, int top, void* out, int K,
                            int twice, pc_stream_t s);
/* pcx_mul_relin_rescale_k over K <= min(k_max, 8) pairs at their own addresses: product j = a[j] b[j] (each a
 * ciphertext at top), out K consecutive ciphertexts; one tensor launch for the K pairs, then the ModUp, key dots (four
 * ciphertexts per launch) and ModDown-rescale of pcx_mul_relin_rescale_k. No counterpart in the reference: independent
 * products of one level (a Chebyshev basis's T_{a+b} = 2 T_a T_b) batched without gathering their operands first.
 * Aliasing: out's slot j may be a[j] or b[j] exactly (in place); a slot overlapping any other pair's operand, or
 * overlapping its own partly, is refused with -1 (the one tensor launch stores every slot while it reads every pair). */
int pcx_mul_relin_rescale_list(pcx_ctx* c, pcx_keys* k, const void* const* a, const void* const* b, int K, int top,
                               void* out, int twice, pc_stream_t s);
/* pcx_mul_relin_rescale_list with each product a sum of pairs: product j = sum of a[i] b[i] over i in off[j] ..
 * off[j + 1] - 1 (off[0] = 0, each range non-empty, off[K] <= 8 pairs in all), relinearized and rescaled once: the
 * words of relinearizing and rescaling the summed tensor (d0, d1, d2); twice: the tensor doubled. y (NULL, or K
 * pointers, each NULL or a ciphertext at top or above): y[j] times its multiplier is added to product j's (d0, d1)
 * before the key switch (subtracted where bit j of ysub is set), so it is rescaled with the product: a term at the
 * product's scale and top rides along for free. yk (NULL, or K pointers, each NULL for 1): y[j]'s multiplier, device
 * rows of the context's row count of words, k mod q by prime id, then their Shoup companions floor(k 2^32 / q).
 * K <= k_max. No out slot may overlap any operand or addend (-1). No counterpart in the reference: a Chebyshev split's
 * product, its remainder's own products and the last remainder, which land on one (top, scale), share one
 * relinearization and one rescale. */
int pcx_mul_sum_relin_rescale_list(pcx_ctx* c, pcx_keys* k, const void* const* a, const void* const* b,
                                   const int* off, int K, int top, const void* const* y, const void* const* yk,
                                   unsigned ysub, int twice, void* out, pc_stream_t s);
/* The plaintext product (mult_pt; the table's mul_table): out = ct pt on Q rows 0..top of both parts, pt evaluation-
 * form rows by prime id (rows 0..top read). out may be ct. */
int pcx_mul_plain(pcx_ctx* c, const void* ct, const void* pt, int top, void* out, pc_stream_t s);
/* pcx_mul_plain of K <= 8 ciphertexts (ct and out each K consecutive ciphertexts), ciphertext j by its own plaintext
 * pts[j], in one launch. No counterpart in the reference, whose mul_table multiplies its K ciphertexts by one table:
 * for a batch of independent scorings (one plaintext query per ciphertext). */
int pcx_mul_plain_k(pcx_ctx* c, const void* ct, const void* const* pts, int K, int top, void* out, pc_stream_t s);
/* the stages alone, for tests and profiles: ModUp of ct's c1 into the context's digit workspace; the dot of key r
 * into ext (one extended ciphertext); ModDown of ext into out */
int pcx_modup(pcx_ctx* c, const void* ct, int top, pc_stream_t s);
const void* pcx_modup_digits(const pcx_ctx* c); /* [dnum][nq + kp][N] */
int pcx_dot(pcx_ctx* c, pcx_keys* k, int r, const void* ct, int top, void* ext, pc_stream_t s);
int pcx_moddown(pcx_ctx* c, void* ext, int top, void* out, pc_stream_t s);

/* Decryption on the device (crates/pc-gpu/src/decrypt.rs:27-117, Decryptor): c0 + c1 s over the bottom d rows through
 * the tensor kernel with the key pair (s, 1), then the inverse NTT. pcx_decryptor_new carves its buffers (the key
 * pairs and k_max outputs of 2 d rows); load_secret takes the secret's evaluation-form rows 0..d-1 from the host
 * ([nwhich][d][N]: dense, then sparse when nwhich is 2; each word below its prime) and synchronises s;
 * pcx_decrypt_rows writes the coefficient rows [K][d][N] of K consecutive ciphertexts at top >= d - 1 into out
 * (device), enqueued on s (the reference's decrypt_rows also downloads them). which: 0 dense, 1 sparse. Returns -1 on
 * arguments out of range (K > k_max, top < d - 1, a secret not loaded). */
typedef struct pcx_decryptor pcx_decryptor;
pcx_decryptor* pcx_decryptor_new(pcx_ctx* c, int d, int k_max, int* err);
void pcx_decryptor_free(pcx_decryptor* x);
int pcx_decryptor_load_secret(pcx_decryptor* x, const uint32_t* s_rows, int nwhich, pc_stream_t s);
int pcx_decrypt_rows(pcx_decryptor* x, const void* ct, int K, int top, int which, void* out, pc_stream_t s);

/* Stage timing, for measurement: while on, the driver records a HIP event pair on the launch stream around each
 * stage it enqueues (0 ModUp INTT, 1 ModUp conversion, 2 ModUp NTT, 3 key dot, 4 ModDown INTT, 5 ModDown conversion,
 * 6 ModDown NTT + epilogue, 7 CtS baby steps and plaintext products, 8 tensor, 9 rescale). pcx_timing(c, n) turns it
 * on for up to n stages
 * (resetting the record); 0 turns it off. pcx_timing_read sums the device time of one stage after the stream has
 * synchronised. No counterpart in the reference (its benches time with CUDA events around whole ops,
 * crates/pc-gpu/benches/ks.rs:80-98). */
int pcx_timing(pcx_ctx* c, int max_stages);
int pcx_timing_read(pcx_ctx* c, int stage, double* total_ms, int* count);

/* HBM stream-copy probe: copies `bytes` (a multiple of 16 KiB) from src to dst with a plain 16-byte-access kernel, to
 * state the achievable bandwidth next to the spec figure and to calibrate the FETCH_SIZE / WRITE_SIZE counters. No
 * counterpart in the reference. */
int pcx_copy_probe(void* dst, const void* src, size_t bytes, pc_stream_t s);
/* VALU throughput probe: `blocks` workgroups of 256 threads, each thread `iters` rounds of 8 independent chains of one
 * instruction form (kind 0 v_add_u32, 1 v_xor_b32, 2 v_alignbit_b32, 3 v_min_u32, 4 v_mul_lo_u32, 5 v_mul_hi_u32,
 * 6 v_mad_u64_u32): 8 iters wave-instructions per wave. `out` holds 1024 words (written only on a value the chains
 * never reach). States the integer rates the kernels can reach beside the spec figures. No counterpart in the
 * reference. -1 on a bad kind or size. */
int pcx_valu_probe(int kind, int blocks, int iters, uint32_t* out, pc_stream_t s);

#ifdef __cplusplus
}
#endif
#endif
