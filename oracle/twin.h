/* CPU twin of the CKKS key-switch / NTT path: the ORACLE of this repository's tests.
 *
 * Test infrastructure only. Nothing in the product library (perseus_amd/) links, loads or calls this code; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, to check the GPU's results against and as the
 * host-CPU baseline.
 *
 * It restates the reference's CPU twin (crates/pc-host) and the math it rests on (crates/pc-core), and the launch
 * sequences of crates/pc-gpu (ks.rs, rotate.rs, keygen.rs) as whole functions, in plain loops over canonical
 * residues. Layouts follow the reference: a ciphertext is [part][row = prime id over Q u P][N] words, a switching
 * key's b is [digit][slot = prime id][N] (full layout), a ModUp output is [digit][row][N].
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number theory (crates/pc-core/src/params/nbtheory.rs) ---- */
int or_is_prime(uint64_t n);
uint64_t or_first_prime(uint32_t bits, uint64_t m);
uint64_t or_last_prime(uint32_t bits, uint64_t m);
uint64_t or_previous_prime(uint64_t q, uint64_t m);
uint64_t or_root_of_unity(uint64_t m, uint64_t p);
uint64_t or_invmod(uint64_t a, uint64_t p);
uint64_t or_powmod(uint64_t b, uint64_t e, uint64_t m);
/* n primes q = 1 mod m with exactly `bits` bits, descending from the largest (OpenFHE LastPrime / PreviousPrime) */
int or_descending_primes(uint32_t bits, uint64_t m, int n, uint64_t* out);

/* ---- device prime constants (args.cuh PrimeConst, 64 bytes; crates/pc-core/src/modmul.rs:364-413) ---- */
void or_prime_const(uint64_t p, uint32_t word_bits, void* out64);

/* ---- ChaCha and the frozen expanders (crates/pc-core/src/keys.rs:29-49, :454-560) ---- */
void or_chacha_block(const uint32_t key[8], uint32_t w12, uint32_t w13, uint32_t w14, uint32_t w15, uint32_t rounds,
                     uint32_t out[16]);
void or_kska_expand_row(const uint32_t seed[8], uint32_t digit, uint32_t p, uint32_t n, uint32_t* out);
uint32_t or_kska_expand(const uint32_t seed[8], uint32_t digit, uint32_t p, uint32_t slot, uint32_t n);
/* the expander rule of or_kska_expand_row under any tag (w15) and w13: "ENCA" with w13 = the nonce gives secret-key
 * encryption's a (crates/pc-kernels/kernels/args.cuh:614-617) */
void or_expand_row(const uint32_t seed[8], uint32_t w13, uint32_t p, uint32_t n, uint32_t tag, uint32_t* out);
void or_cts_expand_row(const uint32_t seed[8], uint32_t p, uint32_t n, uint32_t* out);
void or_kskb_expand_row(const uint32_t seed[8], uint32_t digit, uint64_t p, uint32_t n, uint64_t* out);

/* ---- sampler DRBG and samplers (crates/pc-core/src/keys.rs:122-325) ---- */
typedef struct or_prng or_prng;
or_prng* or_prng_new(const uint32_t key[8], uint32_t stream);
void or_prng_free(or_prng* g);
uint32_t or_prng_next_u32(or_prng* g);
uint64_t or_prng_next_u64(or_prng* g);
uint64_t or_prng_uniform_below(or_prng* g, uint64_t q);
double or_prng_uniform_f64(or_prng* g);
void or_prng_ksk_seed(or_prng* g, uint32_t out[8]);
int or_sample_sparse_ternary(or_prng* g, uint32_t n, uint32_t h, int8_t* out);
void or_sample_gaussian(or_prng* g, double sigma, uint32_t n, int64_t* out);
// the sampler's parts, callable alone: uniform_below's accept rule on one word, the Gaussian's CDF table and inversion
int or_below_accept(uint64_t v, uint64_t q, uint64_t* out);
int or_gauss_cdf(double sigma, double* out, int cap);
int or_gauss_index(double sigma, double u);

/* ---- galois (crates/pc-core/src/galois.rs) ---- */
uint32_t or_automorph_slot(uint32_t k, uint32_t slot, uint32_t logn);
uint64_t or_rotation_galois(int64_t r, uint32_t n);
uint64_t or_galois_inverse(uint64_t g, uint32_t n);

/* ---- context: a chain of nq Q primes then kp special primes, N = 2^logn, dnum hybrid digits ---- */
typedef struct or_ctx or_ctx;
or_ctx* or_ctx_new(uint32_t logn, const uint64_t* primes, int nq, int kp, int dnum);
void or_ctx_free(or_ctx* c);
void or_set_threads(int n);
// pin the pool's threads one per logical CPU of the list (empty: unpinned); the expanded-key (KSKA row) cache's byte
// budget (0: off, cleared)
void or_set_cpus(const int* cpus, int n);
void or_set_kska_cache(size_t bytes);
int or_get_threads(void);
/* twiddle tables of prime id (crates/pc-gpu/src/context.rs:190-230): fw[i] = psi^brev(i), iw = psi^-brev(i) and the
 * Shoup companions floor(w 2^32 / p) */
void or_ctx_twiddles(const or_ctx* c, int id, uint32_t* fw, uint32_t* fws, uint32_t* iw, uint32_t* iws);
uint64_t or_ctx_root(const or_ctx* c, int id);
/* in-place NTT / INTT of nrows rows of N words (row i at rows + i*N, prime id ids[i]); the inverse scales by N^-1 */
void or_ntt_fwd_rows(const or_ctx* c, uint32_t* rows, const int32_t* ids, int nrows);
void or_ntt_inv_rows(const or_ctx* c, uint32_t* rows, const int32_t* ids, int nrows);
/* fast base conversion, one job (crates/pc-host/src/bconv.rs): out_t = sum_i [x_i pre_i]_{s_i} [S/s_i]_t mod t;
 * prescaled = 1: the rows already hold x_i pre_i */
void or_bconv(const or_ctx* c, const uint32_t* const* src, const int32_t* src_ids, int ns, uint32_t* const* dst,
              const int32_t* tgt_ids, int nt, int prescaled);

/* key-switching geometry of the context at limb top `top` */
int or_live_digits(const or_ctx* c, int top);
int or_digit_of(const or_ctx* c, int id);

/* ModUp of c1 (rows 0..top of one polynomial, eval form, row r at c1 + r*N) into digits [dnum][rows][N]
 * (crates/pc-gpu/src/ks.rs:935-1040): only the target rows of each live digit are written */
void or_modup(const or_ctx* c, const uint32_t* c1, int top, uint32_t* digits);
/* key inner product of one key (crates/pc-host/src/ks.rs ks_dot / ks_dot_key, c0 mode 1): for every row t of
 * Q 0..top u P, s0 = sum_d D_d b_d + [t in Q] (P mod q_t) c0, s1 = sum_d D_d a_d, written at automorph_slot(autok, i)
 * of out[part][t] (ciphertext layout); a_d is the KSKA row of (seed, d, p_t) */
void or_ks_dot(const or_ctx* c, const uint32_t* ct, const uint32_t* digits, int top, const uint32_t seed[8],
               const uint32_t* b, uint32_t autok, uint32_t* ext);
/* ModDown of an extended ciphertext ext (Q rows 0..top and P, both parts) into out's Q rows 0..top
 * (crates/pc-gpu/src/ks.rs:1620-1649): out = (ext - NTT(bconv(INTT(ext_P) pre))) P^-1 */
void or_moddown(const or_ctx* c, const uint32_t* ext, int top, uint32_t* out);
/* one rotation by galois element g with key (seed, b): ModUp(c1), dot with autok = g^-1, ModDown
 * (crates/pc-gpu/src/rotate.rs:179-204); out gets Q rows 0..top of both parts */
void or_rotate(const or_ctx* c, const uint32_t* ct, int top, const uint32_t seed[8], const uint32_t* b, uint64_t g,
               uint32_t* out);
/* hoisted rotations (crates/pc-gpu/src/rotate.rs:456-507): one ModUp, then per key a dot and a ModDown */
void or_rotate_hoisted(const or_ctx* c, const uint32_t* ct, int top, int nkeys, const uint32_t* seeds,
                       const uint32_t* const* bs, const uint64_t* gs, uint32_t* const* outs);

/* summed rotations (crates/pc-gpu/src/rotate.rs:692-776 rotate_sum_core, InModDown form): one ModUp, the extended
 * rotations by keys (seeds, bs, gs) summed word by word, one ModDown; out (Q rows 0..top) = onto + that (onto may be
 * NULL, or alias ct / out). -1 for an identity key or no keys. */
int or_rotate_sum(const or_ctx* c, const uint32_t* ct, int top, int nkeys, const uint32_t* seeds,
                  const uint32_t* const* bs, const uint64_t* gs, const uint32_t* onto, uint32_t* out);
/* the giant-step sum over distinct inputs (crates/pc-gpu/src/bts/cts.rs:958-971): out (Q rows 0..top) = onto + ModDown
 * of the sum of the extended rotations of cts[j] by key j (a ModUp each); rescale: the ModDown fused with the
 * two-prime rescale (or_moddown_rescale, out at top - 2). -1 for an identity key or no keys. */
int or_rotate_many(const or_ctx* c, const uint32_t* const* cts, int top, int nkeys, const uint32_t* seeds,
                   const uint32_t* const* bs, const uint64_t* gs, const uint32_t* onto, int rescale, uint32_t* out);
/* the ModDown and two-prime rescale as one exact ModDown by B = P q_{top-1} q_top (crates/pc-gpu/src/bts/cts.rs:
 * 740-751): out's Q rows 0..top - 2 = round((ext + P onto) / B) (onto may be NULL); top >= 2 */
void or_moddown_rescale(const or_ctx* c, const uint32_t* ext, int top, const uint32_t* onto, uint32_t* out);
/* the rotate-and-sum ladder (crates/pc-gpu/src/rotate.rs:924-992) over the keys (seeds, bs, gs): out = the sum of x
 * over its rotations by every multiple of start below stop; radix_bits >= 2 rungs through or_rotate_sum. -1 when a
 * step's key is missing. */
int or_rotate_and_sum(const or_ctx* c, const uint32_t* x, int top, int64_t start, int64_t stop, int radix_bits,
                      int nkeys, const uint32_t* seeds, const uint32_t* const* bs, const uint64_t* gs, uint32_t* out);

/* fused CtS / StC stage (crates/pc-host/src/cts.rs:24-200 `run`, semantics crates/pc-kernels/kernels/cts.cuh:1-10):
 * K ciphertexts x (ct c at x + c*2*R*N) at limb top, with their ModUp digits (ct c at digits + c*dnum*R*N).
 * For every row t of Q 0..top u P and output slot o:
 *   baby 0:      (P c0[o], P c1[o]) on Q rows and 0 on special rows; with x0 non-null, x0's words as stored
 *                (ct c at x0 + c*2*R*N, every row);
 *   baby i >= 1: the key-switch dot of baby key i-1 at the source slot s = automorph_slot(kinv[i-1], o):
 *                (P c0[s] + sum_d D_d[s] b_d[s], sum_d D_d[s] a_d[s]), P c0 on Q rows only;
 *   res_j[o]:    sum_{i < B} rot_i[o] pt_{B j + i}[prow][ptidx(o, enc)], diagonals >= npts skipped.
 * Baby keys: seeds[8 (i-1)], b rows bs[i-1] (full layout [dnum][R][N]). a_d is regenerated from the seed for d < nregen,
 * else read from as[i-1] (same layout; may be null when nregen covers every digit). pmod: P mod q_t per Q prime id
 * (null: the context's). Diagonal k is pts[k] ([rows][ptw]); prow = t on Q rows, pt_prow + (t - nq) on special rows;
 * ptidx (crates/pc-kernels/kernels/arith.cuh:242-244) maps o to o >> (enc & 0xFF) when enc >> 24 == 0x7F, else o & enc.
 * Writes res ct (c, j) at res + (c*G + j)*2*R*N, rows of Q 0..top u P, both parts. */
void or_cts_fused(const or_ctx* c, int K, const uint32_t* x, const uint32_t* digits, int top, int B, int G, int npts,
                  const uint32_t* seeds, const uint32_t* const* bs, const uint32_t* const* as, int nregen,
                  const uint32_t* kinv, const uint32_t* const* pts, int ptw, int pt_prow, uint32_t enc,
                  const uint32_t* pmod, const uint32_t* x0, uint32_t* res);

/* switching-key generation (crates/pc-kernels/kernels/keygen.cuh ksk_gen; crates/pc-gpu/src/keygen.rs:172-262):
 * b[d][t] = e[d][t] - a_d[t] s_new[t] + [t in digit d] (P mod q_t) s_old[t], every digit and every row of Q u P
 * (eval form; a from the KSKA expander of seed) */
void or_ksk_gen(const or_ctx* c, const uint32_t* s_new, const uint32_t* s_old, const uint32_t seed[8],
                const uint32_t* e, uint32_t* b);
/* the reference flow of a rotation key for galois g from the caller's DRBG: seed = ksk_seed(), sub = ksk_seed(),
 * per-digit Gaussian errors from the stream (sub, d), s_new = sigma_{g^-1}(s). s_eval: the secret's eval rows
 * [rows][N]. Writes the seed, b [dnum][rows][N] */
void or_rotation_key(const or_ctx* c, or_prng* g, const uint32_t* s_eval, uint64_t galois, uint32_t seed[8],
                     uint32_t* b);
/* the secret's eval rows [rows][N] from ternary coefficients */
void or_secret_eval(const or_ctx* c, const int8_t* s, uint32_t* s_eval);
/* sigma_k as an eval-form gather out[o] = in[automorph_slot(k, o)] on nrows rows */
void or_automorph_rows(const or_ctx* c, const uint32_t* in, uint32_t k, int nrows, uint32_t* out);

/* ---- SPRU floating-point stages (crates/pc-host/src/spru.rs:83-140, encode.rs:85-101) ----
 * complex values as interleaved double pairs. fft_pass: one forward Stockham pass of half-size ns over batch size-n
 * transforms, tw of n/2 pairs; scatter: batch size-n FFT outputs y, zeta table zt of n pairs, to nl coefficient rows
 * per transform at out + e out_stride + l n (residues mod primes[l]). */
void or_spru_fft_pass(const double* in, double* out, const double* tw, uint32_t n, uint32_t ns, uint32_t batch);
void or_spru_scatter(const double* y, const double* zt, const uint64_t* primes, uint32_t nl, uint32_t n,
                     uint32_t batch, double scale, uint64_t out_stride, uint32_t* out);

#ifdef __cplusplus
}
#endif
