// Driver-internal launchers that fuse stages of the key-switching path beyond the kernel-table entries: the ModDown
// base conversion inside the forward NTT's column pass, and the forward row pass (with its epilogue) on its own.
// Not part of the C ABI; the driver (driver.cpp) is their only caller.
#pragma once
#include <stdint.h>

#include "pc_hip.h"

namespace pch {

// Conversion P -> Q rows 0..top of m extended ciphertexts, each target row then taken through the forward NTT's
// column pass. ext: [c][part][rows][N] whose P rows (ids nq .. nq + kp - 1) hold y_j = [x_j N^-1 pre_j]_{p_j} in
// coefficient order (the INTT's output); conv: same layout, receives the column pass of conv_t = sum_j y_j M[j][t]
// mod q_t in its Q rows (lazy words, as the plain column pass leaves them); mt: M[j][t] = [P / p_j]_{q_t}, row stride
// nq; ntg: target rows per workgroup.
struct MdcArgs {
    const uint32_t* ext;
    uint32_t* conv;
    const uint32_t* mt;
    const PrimeConst* pr;
    const uint32_t* fw;
    const uint32_t* fws;
    int nq, kp, rows, top, ntg, m, lazy;
};
constexpr int MDC_MAX_KP = 6;
constexpr int MDC_MAX_NTG = 8;
// 0, or -1 (bad arguments), -2 (kp outside 1..MDC_MAX_KP, ntg above MDC_MAX_NTG or logn outside 12..16), or a HIP
// error
int md_conv_cols(int logn, const MdcArgs* a, pc_stream_t s);
// Any conversion plan (a's jobs: prescaled sources, fast or exact; every job's targets within a->max_tgt) fused into the
// forward NTT's column pass: job k's target t gets the column pass of conv_t (prime tgt_prime) in dst row
// dst_off + tgt_row, lazy words as the plain column pass leaves them. ntg (1..3): the targets whose sums a thread
// carries at once; tpw: targets per workgroup (rounded up to a multiple of ntg); fw / fws: the forward twiddles by prime
// id; lazy: NttArgs.lazy; exact: nonzero when a's jobs include exact ones (0: every job taken as fast). 0, -1 (bad arguments), -2
// (logn outside 12..16) or a HIP error.
int conv_cols(int logn, const BconvArgs* a, const uint32_t* fw, const uint32_t* fws, int lazy, int exact, int ntg,
              int tpw, pc_stream_t s);
// The fused ModDown-rescale's preparation (moddown.hip mdr_prep_k): x rows top - 1, top += P onto; out rows
// 0..top - 2 = onto s2 (k: [s2 | Shoup | P mod q | Shoup] by prime id, rows words each); both parts of K consecutive
// ciphertexts (2 rows rows each)
int mdr_prep(int logn, void* x, const void* onto, void* out, const uint32_t* k, const PrimeConst* pr, int rows,
             int top, int K, pc_stream_t s);

// The forward transform's row pass alone (grid of every row of a), epilogue a->epi included: completes a forward NTT
// whose column pass was done by md_conv_cols.
int ntt_fwd_rows_only(int logn, const NttArgs* a, pc_stream_t s);

// The retry values of a key group's KSKA words (the rejected ChaCha words' accepted redraws, in slot order), built
// once when the keys are made: idx[((r ndig + d) rows + t) chunks + c] is the first value of key r, digit d, row t,
// 1024-slot chunk c in val (exclusive prefix over that order, one sentinel at the end). With them the fast dot
// regenerates a and never redraws: a rejected word's value is read from the table.
struct PatchTab {
    const uint32_t* idx;
    const uint32_t* val;
    int ndig, rows;
    int diag;  // nonzero: K = R, ciphertext c under key c alone (grid z = K); the table entries pass zero
};
// counts[((r ndig + d) rows + t) chunks + c] for the nkeys seeds (device array of seed pointers) and the context's primes
int kska_patch_count(int logn, const uint32_t* const* seeds, const PrimeConst* pr, int nkeys, int ndig, int rows,
                     uint32_t* counts, pc_stream_t s);
int kska_patch_fill(int logn, const uint32_t* const* seeds, const PrimeConst* pr, int nkeys, int ndig, int rows,
                    const uint32_t* idx, uint32_t* val, pc_stream_t s);
// the fast dot with the retry values read from P instead of redrawn; -2 where the fast dot does not apply. Beside the
// table entry's c0 modes it takes c0_mode 3 (no counterpart in the reference, which rejects it): both parts of the
// ciphertext at c0 (the second ct_stride / 2 words after the first) enter the Q rows as P c0 and P c0', so a
// relinearized product's (d0, d1) is added in the extended basis and its ModDown needs no add-onto step
int ks_dot_patched(int logn, const KsKeyArgs* g, const PatchTab* P, pc_stream_t s);

// The forward NTT of composite-rescale corrections (rescale_fwd): row i's input generated in the column pass from the
// two sources r (ndrop 2) names, top - rprime[i] and top - 1 - rprime[i] rows above row i; a's epilogue applies
int ntt_fwd_rescale(int logn, const NttArgs* a, const RescaleArgs* r, pc_stream_t s);

// The one-pass transforms of N = 2^16 (ntt1.hip): one 1024-thread workgroup per row of rows [r0, r0 + n) of a
// (checked by the caller), the forward with a's epilogue, the inverse with its es / N^-1 scale.
void ntt1_fwd(const NttArgs& a, int r0, int n, pc_stream_t st);
void ntt1_inv(const NttArgs& a, int r0, int n, pc_stream_t st);

// The forward NTT of dense rows: row i of a at base + i N with prime id i mod a->xnum (a->roff, a->rprime unused), no
// epilogue and no out-of-place source; the non-lazy butterflies (legal for every prime below 2^31)
int ntt_fwd_dense(int logn, const NttArgs* a, pc_stream_t s);
// the row count from which launches of N = 2^16 take the one-pass transform (0: never); returns the previous one
int ntt_one_pass_min(int rows);

// noalloc.hip: looks up the no-allocation ladder's scratch address on the current device (0 or the HIP error)
int noalloc_prepare();

// The tensor of K ciphertext pairs at their own addresses (driver-internal, no counterpart in the reference, whose
// tensor takes K consecutive ciphertexts): out ciphertext c = (a[c] b[c])'s (d0, d1), part 1 of d2 ciphertext c its
// d2, doubled when dbl; rows 0..n-1; a[c] / b[c] hold part 0, part 1 `part` words later; out and d2 are K consecutive
// ciphertexts (ct_stride apart)
constexpr int TLIST_MAX = 8;
// sum != 0: product c is the sum of pairs off[c] .. off[c + 1] - 1 (off[K] <= TLIST_MAX pairs in all); else pair c
struct TensorListArgs {
    const uint32_t* a[TLIST_MAX];
    const uint32_t* b[TLIST_MAX];
    uint32_t* out;
    uint32_t* d2;
    uint64_t part, ct_stride;
    const PrimeConst* pr;
    int n, K, dbl;
    int sum;
    int off[TLIST_MAX + 1];
    // product c's addend y[c] (a ciphertext: two parts part apart, rows by prime id; null: none), added to (d0, d1),
    // subtracted where bit c of ysub is set
    const uint32_t* y[TLIST_MAX];
    uint32_t ysub;
    // y[c]'s multiplier (null: 1): krows words k mod q by prime id, then their Shoup companions
    const uint32_t* yk[TLIST_MAX];
    int krows;
};
int tensor_list(int logn, const TensorListArgs* a, pc_stream_t s);
// The plaintext products of K ciphertexts (K consecutive, ct_stride apart; out likewise), ciphertext c by its own
// plaintext t[c] (evaluation-form rows by prime id): rows 0..n-1 of both parts (driver-internal: the reference's
// mul_table takes one plaintext for its K ciphertexts)
struct MulPtListArgs {
    const uint32_t* in;
    uint32_t* out;
    const uint32_t* t[TLIST_MAX];
    uint64_t part, ct_stride;
    const PrimeConst* pr;
    int n, K;
};
int mul_pt_list(int logn, const MulPtListArgs* a, pc_stream_t s);

// ks_dot_key's summed rotations (c0_mode | KS_SUM): out = sum_r sigma_r(dot_r), gathered in output order
int ks_dot_key_sum(int logn, const KsKeyArgs* g, pc_stream_t s);

}  // namespace pch
